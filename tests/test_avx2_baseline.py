"""The CPU baseline's avx2 restatement (oracle/rh_avx2.c) against the
portable restatement (oracle/rh_oracle.c), bit for bit.

bench.py times the avx2 restatement as the CPU baseline, so it has to compute
what the portable path computes: the reference's avx2 adapter
(crates/rusticide-kernels/src/adapter.rs:86-169) is required to agree with its
portable kernels exactly (crates/rusticide-kernels/src/matmul_group_tests.rs),
and this test holds the restatements to the same bar on TinyLlama-shaped
matrices, hostile scale bytes, one and many threads, and the refused case.
"""

import numpy as np
import pytest

import oracle as O
from rusticide_amd import synth

pytestmark = pytest.mark.skipif(not O.Avx2Matrix.available(), reason="host has no avx2+fma")


def portable(type_id, data, rows, cols, x):
    out = np.zeros(rows, np.float32)
    O.matvec_batch(x, [(O.Weights.blocks(type_id, data, synth.row_bytes(type_id, cols)), out)])
    return out


def assert_same_bits(got, want):
    # NaN rows must match as NaN; a NaN's sign and payload are not part of
    # the result (the GPU parity tests use the same rule)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def activation(cols, seed):
    return synth.normal_f32(cols, seed=seed)


@pytest.mark.parametrize("type_id", [12, 14])
@pytest.mark.parametrize("rows,cols", [(8, 256), (64, 2048), (40, 5632), (256, 2048), (96, 4096)])
@pytest.mark.parametrize("threads", [1, 4])
def test_avx2_matches_the_portable_restatement(type_id, rows, cols, threads):
    data = synth.matrix(type_id, rows, cols, seed=rows * 7 + cols + type_id)
    x = activation(cols, seed=rows + cols)
    m = O.Avx2Matrix(type_id, data, rows, synth.row_bytes(type_id, cols))
    out = np.full(rows, np.nan, np.float32)
    assert m.matvec(x, out, threads)
    want = portable(type_id, data, rows, cols, x)
    assert_same_bits(out, want)
    m.close()


@pytest.mark.parametrize("type_id", [12, 14])
def test_avx2_on_random_bytes(type_id):
    # every scale, dmin and quant byte pattern, including f16 NaN/inf scales
    rows, cols = 32, 1024
    rb = synth.row_bytes(type_id, cols)
    data = O.pseudo_random_bytes(rows * rb, seed=type_id + 99)
    x = activation(cols, seed=5)
    m = O.Avx2Matrix(type_id, data, rows, rb)
    out = np.zeros(rows, np.float32)
    assert m.matvec(x, out, 3)
    want = portable(type_id, data, rows, cols, x)
    assert_same_bits(out, want)


def test_avx2_on_the_reference_synthetic_blocks():
    # quant_kernel.rs's synthetic_blocks generator, TinyLlama's ffn_down width
    for type_id in (12, 14):
        rows, cols = 16, 5632
        data = O.synthetic_blocks(type_id, rows * cols // 256, 3)
        x = activation(cols, seed=11)
        m = O.Avx2Matrix(type_id, data, rows, synth.row_bytes(type_id, cols))
        out = np.zeros(rows, np.float32)
        assert m.matvec(x, out, 2)
        assert_same_bits(out, portable(type_id, data, rows, cols, x))


def test_super_block_quants_never_reach_minus_128():
    # The avx2 views refuse an input holding the quant -128 (group_views.rs:6,
    # :91), which their sign trick cannot negate; Q8_K rounds and clamps to
    # [-127, 127] (portable/q8.rs:86-95, :113-115), so for these kernels no
    # input is refused, hostile ones included.
    rows, cols = 8, 512
    data = synth.matrix(14, rows, cols, seed=1)
    m = O.Avx2Matrix(14, data, rows, synth.row_bytes(14, cols))
    for sign in (1.0, -1.0):
        x = activation(cols, seed=2)
        x[300] = sign * 1e6  # one block's quants pinned at the ends of the range
        q = O.quantize(x, 1)
        assert int(q.quants.min()) >= -127 and int(q.quants.max()) <= 127
        out = np.zeros(rows, np.float32)
        assert m.matvec(x, out, 1)
        assert_same_bits(out, portable(14, data, rows, cols, x))


def test_shapes_the_units_cannot_hold_are_refused():
    data = synth.matrix(12, 12, 256, seed=1)
    with pytest.raises(ValueError):
        O.Avx2Matrix(12, data, 12, synth.row_bytes(12, 256))  # rows not a multiple of 8
    with pytest.raises(ValueError):
        O.Avx2Matrix(36, data, 8, 64)  # I2_S has no avx2 units here
