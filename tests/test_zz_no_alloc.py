"""rh_matmul_batch_device_noalloc against rh_matmul_batch_device.

The allocation-free entry point keeps a batch's quantized activations in a
file-scope device array and runs K-split GEMMs unsplit; its outputs must
equal the allocating entry point's bit for bit. Each case makes two calls in
a row, the second on a smaller input, so the second reads an array that
still holds the first call's contents.
"""

import numpy as np
import pytest

import rusticide_amd as R
from rusticide_amd import hip as H
from rusticide_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = R.Context(0)
    yield c
    c.close()


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def run(ctx, fn, mats, x, tokens):
    """One batch of every matrix against `tokens` rows of x, on device buffers."""
    d_in = H.DeviceArray.from_numpy(x)
    outs = [H.DeviceArray(m.rows * tokens) for m in mats]
    for o in outs:
        o.fill_bytes(0xFF)
    fn(ctx, d_in, tokens, list(zip(mats, outs)))
    H.synchronize()
    res = [o.numpy() for o in outs]
    d_in.free()
    for o in outs:
        o.free()
    return res


# (tokens, width) pairs: the second of each is smaller than the first.
# 1 token: the quantize-fused decode kernels; 5: a quantize launch into the
# array, then the kernels reading it; 64: the MFMA GEMMs, which the
# allocating entry point splits along K for these 2048-row shapes.
CASES = [((1, 5632), (1, 2048)), ((5, 4096), (3, 2048)), ((64, 2048), (12, 1024))]


@pytest.mark.parametrize("first,second", CASES)
def test_noalloc_equals_the_allocating_entry_point(ctx, first, second):
    rng = np.random.default_rng(sum(first) + sum(second))
    for tokens, width in (first, second):
        mats = [R.Matrix.load(ctx, R.Q4_K, synth.matrix(R.Q4_K, 2048, width, seed=width), 2048, width),
                R.Matrix.load(ctx, R.Q6_K, synth.matrix(R.Q6_K, 300, width, seed=width + 1), 300, width),
                R.Matrix.load(ctx, R.I2_S, synth.i2s_matrix(1024, width, seed=width + 2), 1024, width)]
        x = rng.standard_normal(tokens * width).astype(np.float32)
        got = run(ctx, R.matmul_batch_device_noalloc, mats, x, tokens)
        want = run(ctx, R.matmul_batch_device, mats, x, tokens)
        for m, g, w in zip(mats, got, want):
            assert np.array_equal(bits(g), bits(w)), f"type {m.type_id}, {tokens} x {width}"
        for m in mats:
            m.free()


def test_noalloc_refuses_batches_beyond_its_array(ctx):
    # 4096 tokens of 2048 values need 23,068,672 bytes of quantized activations,
    # more than the 4 MiB array: refused before any launch
    m = R.Matrix.load(ctx, R.Q4_K, synth.matrix(R.Q4_K, 16, 2048, seed=1), 16, 2048)
    x = H.DeviceArray(4096 * 2048)
    out = H.DeviceArray(16 * 4096)
    with pytest.raises(R.RusticideError) as e:
        R.matmul_batch_device_noalloc(ctx, x, 4096, [(m, out)])
    assert e.value.kind == "INVALID_ARGUMENT" and "bytes" in str(e.value)
    x.free()
    out.free()
    m.free()
