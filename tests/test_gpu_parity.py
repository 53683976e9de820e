"""GPU parity: the HIP path against the CPU oracle, through the C ABI.

The bar: I2_S int32 accumulators bit-exact; k-quant f32 outputs
bit-identical to the CPU integer path (stricter than a 1e-4 relative
tolerance); every token of a batch identical to a single-token call. Shapes include the benchmark workloads at full size.
"""

import os

import numpy as np
import pytest

import oracle as O
import rusticide_amd as R
from rusticide_amd import hip as H
from rusticide_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = R.Context(0)
    yield c
    c.close()


VARIANTS = {
    # the default: the quantize-fused kernels for decode-sized batches
    "auto": {},
    # a quantize launch, then the kernels reading its result, at 1, 2 and 4
    # blocks per team
    "lds-1": {"RUSTICIDE_HIP_GEMV": "lds", "RUSTICIDE_HIP_GEMV_NI": "1"},
    "lds-2": {"RUSTICIDE_HIP_GEMV": "lds", "RUSTICIDE_HIP_GEMV_NI": "2"},
    "lds-4": {"RUSTICIDE_HIP_GEMV": "lds", "RUSTICIDE_HIP_GEMV_NI": "4"},
    # one-token k-quant launches on 256-lane workgroups only, and on 512-lane
    # ones (half the blocks per team) wherever a launch has two or more
    "nt-256": {"RUSTICIDE_HIP_KQ_NT": "256"},
    "nt-512": {"RUSTICIDE_HIP_KQ_NT": "512"},
    # the general block walk where the fixed-column one would run
    "walk": {"RUSTICIDE_HIP_KQ_FIX": "0"},
    # grids of one to two workgroups per CU kept as they are
    "no-balance": {"RUSTICIDE_HIP_KQ_BALANCE": "0"},
    # 17- to 32-block rows on 512 lanes (two rounds of quantization) instead
    # of 768 or 1024
    "no-onepass": {"RUSTICIDE_HIP_KQ_ONEPASS": "0"},
}
SWITCHES = ("RUSTICIDE_HIP_GEMV", "RUSTICIDE_HIP_GEMV_NI", "RUSTICIDE_HIP_KQ_NT", "RUSTICIDE_HIP_KQ_FIX",
            "RUSTICIDE_HIP_KQ_BALANCE", "RUSTICIDE_HIP_KQ_ONEPASS")


@pytest.fixture(params=list(VARIANTS))
def variant(request):
    """Every decode GEMV kernel variant must give the CPU path's bits."""
    saved = {k: os.environ.get(k) for k in SWITCHES}
    for k in SWITCHES:
        os.environ.pop(k, None)
    os.environ.update(VARIANTS[request.param])
    R.reload_tuning()
    yield request.param
    for k, v in saved.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v
    R.reload_tuning()


@pytest.fixture
def tuning(monkeypatch):
    """monkeypatch.setenv for the kernel switches, re-read by the library."""
    class Env:
        def set(self, name, value):
            monkeypatch.setenv(name, value)
            R.reload_tuning()
    yield Env()
    monkeypatch.undo()
    R.reload_tuning()


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def assert_same_bits(got, want, what=""):
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    assert got.shape == want.shape, what
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan), what
    bad = np.flatnonzero(bits(got)[~nan] != bits(want)[~nan])
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first {bad[:5]}: {got[~nan][bad[:5]]} vs {want[~nan][bad[:5]]}"


def oracle_matmul(type_id, data, rows, cols, x, tokens, scale=0.0, threads=8):
    rb = synth.row_bytes(type_id, cols) if type_id != 0 else cols
    if type_id == 36:
        w = O.Weights.ternary(data[: rows * rb], rb, scale)
    elif type_id == 0:
        w = O.Weights.dense(data, cols)
    else:
        w = O.Weights.blocks(type_id, data, rb)
    out = np.full(rows * tokens, np.nan, np.float32)
    O.matmul_batch(x, tokens, [(w, out)], threads=threads)
    return out


# ------------------------------------------------------------- quantizers


def quant_cases():
    rng = np.random.default_rng(7)
    cases = [rng.standard_normal(2048).astype(np.float32),
             (rng.standard_normal(5632) * 30).astype(np.float32),
             np.zeros(512, np.float32),
             O.pseudo_random_values(768, 3)]
    ties = np.zeros(256, np.float32)
    ties[:6] = [127.0, 2.5, 3.5, -2.5, -3.5, 0.5]
    cases.append(ties)
    nan = rng.standard_normal(512).astype(np.float32)
    nan[[3, 300]] = np.nan
    cases.append(nan)
    inf = rng.standard_normal(256).astype(np.float32)
    inf[17] = -np.inf
    cases.append(inf)
    tail_nan = rng.standard_normal(64).astype(np.float32)
    tail_nan[-1] = np.nan
    cases.append(tail_nan)
    sub = (rng.standard_normal(256) * 1e-40).astype(np.float32)
    cases.append(sub)
    cases.append(rng.standard_normal(300).astype(np.float32))  # partial blocks
    cases.append(rng.standard_normal(8192).astype(np.float32))  # widest row the one-wave I8_S kernel holds
    wide = rng.standard_normal(6912).astype(np.float32)  # BitNet down width, NaN and inf mid-row
    wide[5000] = np.nan
    wide[6000] = np.inf
    cases.append(wide)
    cases.append(rng.standard_normal(8224).astype(np.float32))  # past it: the workgroup kernel
    return cases


@pytest.mark.parametrize("kind", [R.SUPER_BLOCK, R.ROW])
def test_device_quantizers_match_the_oracle(ctx, kind):
    for i, x in enumerate(quant_cases()):
        q, s, m = ctx.quantize(x, kind)
        want = O.quantize(x, kind)
        assert np.array_equal(q, want.quants), (kind, i)
        assert_same_bits(s, want.scales, f"scales kind={kind} case={i}")
        assert np.array_equal(m, want.sums), (kind, i)


# ---------------------------------------------------------- k-quant GEMV


KQ_SHAPES = [
    (12, 5632, 2048, [1, 2]),   # Q4_K ffn_gate shape (benchmark workload)
    (12, 2048, 5632, [1, 2]),   # Q4_K ffn_down shape (22 blocks per row)
    (12, 37, 512, [1, 3, 8, 11]),
    (14, 32000, 2048, [1, 2]),  # Q6_K lm_head (benchmark workload)
    (12, 64, 4096, [1, 2]),     # 16 blocks: one full pass
    (14, 19, 8192, [1, 2]),     # 32 blocks: two passes (one token: 1024 lanes)
    (12, 1000, 8192, [1]),      # 32 blocks, 125 workgroups of 1024 lanes
    (14, 333, 4608, [1, 2]),    # 18 blocks, 34 workgroups of 768 lanes
    (14, 100, 6144, [1, 2]),    # 24 blocks: 8-row workgroups of 12 groups, the last of 4 rows
    (12, 77, 7680, [1]),        # 30 blocks: 1024 lanes, 8 rows = 15 groups
    (12, 11, 256, [1, 2]),      # one block per row: 16 rows per wave
    (14, 2048, 5632, [1, 3]),   # Q6_K ffn_down: 4620-byte rows, padded stride
    (14, 45, 768, [1, 2, 9]),
    (12, 40, 25600, [1, 2]),    # 100 blocks per row: two blocks per team
    (14, 24, 38400, [1, 2]),    # 150 blocks per row: four blocks per team
    (12, 16384, 2048, [1]),     # 512 workgroups of 32 rows: interleaved 8-row chunks
    (14, 12800, 2048, [1]),     # 400 workgroups of 32 rows: interleaved 8-row chunks
]


@pytest.mark.parametrize("type_id,rows,cols", [(12, 16384, 2048), (14, 32000, 2048)])
def test_interleaved_rows_give_the_contiguous_bits(ctx, tuning, type_id, rows, cols):
    # a workgroup's rows as interleaved chunks (grids of a workgroup per CU
    # or more) or as one contiguous run: the same outputs in the same rows
    data = synth.matrix(type_id, rows, cols, seed=7 * rows + cols)
    m = R.Matrix.load(ctx, type_id, data, rows, cols)
    x = synth.normal_f32(cols, seed=3)
    outs = []
    for il in ("1", "0"):
        tuning.set("RUSTICIDE_HIP_GEMV_IL", il)
        out = np.full(rows, np.nan, np.float32)
        R.matmul_batch(ctx, x, 1, [(m, out)])
        outs.append(out)
    assert_same_bits(outs[0], outs[1], f"type={type_id} {rows}x{cols}")
    assert_same_bits(outs[0], oracle_matmul(type_id, data, rows, cols, x, 1), "oracle")


@pytest.mark.parametrize("type_id,rows,cols,token_counts", KQ_SHAPES)
def test_kquant_gemv_is_bit_identical_to_the_cpu_path(ctx, variant, type_id, rows, cols, token_counts):
    data = synth.matrix(type_id, rows, cols, seed=rows + cols)
    m = R.Matrix.load(ctx, type_id, data, rows, cols)
    for tokens in token_counts:
        x = synth.normal_f32(tokens * cols, seed=tokens)
        want = oracle_matmul(type_id, data, rows, cols, x, tokens)
        out = np.full(rows * tokens, np.nan, np.float32)
        R.matmul_batch(ctx, x, tokens, [(m, out)])
        assert_same_bits(out, want, f"type={type_id} {rows}x{cols} tokens={tokens}")


@pytest.mark.parametrize("type_id", [12, 14])
def test_activations_at_any_dword_offset(ctx, variant, type_id):
    # device inputs 4, 8 or 12 bytes past a 16-byte boundary, and token rows
    # of 2049 or 2051 values (later tokens start off one too): the fused
    # kernels' 16-byte activation loads need only dword alignment
    class At:  # the device values from float `off` of `buf` on
        def __init__(self, buf, off, n):
            self.buf, self.off, self.n = buf, off, n

        def data_ptr(self):
            return self.buf.data_ptr() + 4 * self.off

        def numel(self):
            return self.n

    rows, cols = 64, 2048
    data = synth.matrix(type_id, rows, cols, seed=31)
    m = R.Matrix.load(ctx, type_id, data, rows, cols)
    for tokens, width in ((1, 2048), (2, 2049), (3, 2051)):
        x = synth.normal_f32(tokens * width, seed=width)
        want = oracle_matmul(type_id, data, rows, cols, x, tokens)
        for off in (1, 2, 3):
            buf = H.DeviceArray.from_numpy(np.concatenate([np.zeros(off, np.float32), x, np.zeros(4, np.float32)]))
            out = H.DeviceArray(rows * tokens)
            out.fill_bytes(0xFF)
            R.matmul_batch_device(ctx, At(buf, off, tokens * width), tokens, [(m, out)])
            H.synchronize()
            assert_same_bits(out.numpy(), want, f"tokens {tokens} width {width} offset {off}")
            buf.free()
            out.free()


@pytest.mark.parametrize("type_id", [12, 14])
def test_reference_synthetic_blocks(ctx, type_id):
    # the reference's own generator (format.rs:204-214) and activations
    rows, cols = 24, 1024
    data = O.synthetic_blocks(type_id, rows * cols // 256, 1)
    x = O.bench_activations(cols, 2)
    m = R.Matrix.load(ctx, type_id, data, rows, cols)
    out = np.zeros(rows, np.float32)
    m.matvec(x, out)
    assert_same_bits(out, oracle_matmul(type_id, data, rows, cols, x, 1))


@pytest.mark.parametrize("type_id", [12, 14])
def test_kquant_dot_within_1e4_of_dequantize_and_dot(ctx, type_id):
    # quant_kernel_tests.rs:60-79: against the dequantized operands
    rows, cols = 16, 2048
    data = synth.matrix(type_id, rows, cols, seed=3)
    x = synth.normal_f32(cols, seed=4)
    m = R.Matrix.load(ctx, type_id, data, rows, cols)
    out = np.zeros(rows, np.float32)
    m.matvec(x, out)
    xq = O.quantize(x, O.SUPER_BLOCK).dequantize()
    rb = synth.row_bytes(type_id, cols)
    for r in range(rows):
        row = data[r * rb:(r + 1) * rb]
        w = O.dequantize_row(type_id, row)
        ref = float(np.dot(w.astype(np.float64), xq.astype(np.float64)))
        assert abs(out[r] - ref) <= 1e-4 * max(1.0, float(np.abs(w).sum()))


# ------------------------------------------------------ prefill GEMM (MFMA)


GEMM_SHAPES = [
    (12, 5632, 2048, [128, 512, 2048]),  # prefill on the ffn_gate shape: 128/512/2048 tokens
    (12, 37, 512, [9, 77]),               # ragged rows and tokens
    (14, 45, 768, [9, 70]),
    (14, 2048, 5632, [64]),               # Q6_K ffn_down: 22 blocks, 4620-byte rows
    (14, 32000, 2048, [64]),              # Q6_K lm_head over a 64-token prefill chunk
    (12, 130, 25600, [16]),               # 100 blocks per row
    (12, 6400, 2304, [64]),               # K split into segments of 2 blocks, the last one short
]


@pytest.mark.parametrize("type_id,rows,cols,token_counts", GEMM_SHAPES)
def test_prefill_gemm_is_bit_identical_to_the_cpu_path(ctx, type_id, rows, cols, token_counts):
    # matmul_batch with many tokens (matmul.rs:229-248): the MFMA GEMM must give
    # the CPU integer path's bits, token by token
    assert R.lib().rh_gemm_min_tokens() <= min(token_counts)
    data = synth.matrix(type_id, rows, cols, seed=rows + 3 * cols)
    m = R.Matrix.load(ctx, type_id, data, rows, cols)
    for tokens in token_counts:
        x = synth.normal_f32(tokens * cols, seed=100 + tokens)
        want = oracle_matmul(type_id, data, rows, cols, x, tokens, threads=16)
        out = np.full(rows * tokens, np.nan, np.float32)
        R.matmul_batch(ctx, x, tokens, [(m, out)])
        assert_same_bits(out, want, f"type={type_id} {rows}x{cols} tokens={tokens}")


@pytest.mark.parametrize("type_id,rows,cols,tokens", [(12, 2048, 2048, 64), (14, 2048, 5632, 64),
                                                       (12, 2560, 2048, 64), (12, 6400, 2304, 64),
                                                       (14, 45, 768, 9), (12, 300, 25600, 33)])
def test_split_k_gives_the_unsplit_bits(ctx, tuning, type_id, rows, cols, tokens):
    # a launch with too few row and token tiles to fill the chip splits K
    # across workgroups and adds the later blocks' terms in block order
    # afterwards; RUSTICIDE_HIP_GEMM_SPLIT=0 keeps every block in one workgroup
    data = synth.matrix(type_id, rows, cols, seed=rows + cols)
    m = R.Matrix.load(ctx, type_id, data, rows, cols)
    x = synth.normal_f32(tokens * cols, seed=7 + tokens)
    split = np.full(rows * tokens, np.nan, np.float32)
    R.matmul_batch(ctx, x, tokens, [(m, split)])
    tuning.set("RUSTICIDE_HIP_GEMM_SPLIT", "0")
    whole = np.full(rows * tokens, np.nan, np.float32)
    R.matmul_batch(ctx, x, tokens, [(m, whole)])
    assert_same_bits(split, whole, f"type={type_id} {rows}x{cols} tokens={tokens}")
    assert_same_bits(split, oracle_matmul(type_id, data, rows, cols, x, tokens, threads=16))


@pytest.mark.parametrize("bn", ["", "64"])
@pytest.mark.parametrize("tokens", [64, 36, 12])
def test_split_k_tile_fixup_matches_the_combine_launch(ctx, tuning, tokens, bn):
    # a split launch of up to 9 planes whose token count is a multiple of 4
    # sums each tile's planes in the tile's last-arriving workgroup
    # (device-scope arrival counters, reset by that workgroup);
    # RUSTICIDE_HIP_GEMM_FIXUP=0 sums them in gemm_combine_kernel. Jobs whose
    # rows end mid-tile (two in one Q4_K launch), a 21-plane Q6_K launch
    # (always combined) between them, the calls repeated so that a counter
    # left non-zero shows; RUSTICIDE_HIP_GEMM_BN=64 takes the fixup's
    # 64-token tiles
    if bn:
        tuning.set("RUSTICIDE_HIP_GEMM_BN", bn)
    cols = 2048
    specs = [(12, 300, synth.matrix(12, 300, cols, seed=11)), (12, 45, synth.matrix(12, 45, cols, seed=12)),
             (14, 100, synth.matrix(14, 100, cols, seed=14))]
    mats = [R.Matrix.load(ctx, t, d, rows, cols) for t, rows, d in specs]
    big = synth.matrix(14, 2048, 5632, seed=13)
    mbig = R.Matrix.load(ctx, 14, big, 2048, 5632)
    x = synth.normal_f32(tokens * cols, seed=21 + tokens)
    xb = synth.normal_f32(tokens * 5632, seed=22 + tokens)

    def run():
        outs = [np.full(rows * tokens, np.nan, np.float32) for _, rows, _ in specs]
        R.matmul_batch(ctx, x, tokens, list(zip(mats, outs)))
        ob = np.full(2048 * tokens, np.nan, np.float32)
        R.matmul_batch(ctx, xb, tokens, [(mbig, ob)])
        return outs + [ob]

    first = [run() for _ in range(3)]
    tuning.set("RUSTICIDE_HIP_GEMM_FIXUP", "0")
    combined = run()
    for outs in first:
        for a, b in zip(outs, combined):
            assert_same_bits(a, b, f"tokens={tokens}")
    for (t, rows, d), out in zip(specs, combined[:-1]):
        assert_same_bits(out, oracle_matmul(t, d, rows, cols, x, tokens), f"type {t} rows {rows}")
    assert_same_bits(combined[-1], oracle_matmul(14, big, 2048, 5632, xb, tokens, threads=16))


def test_prefill_gemm_batch_of_projections_and_hostile_bytes(ctx):
    # Q/K/V in one batch (attention.rs:215-223) on the GEMM, plus random block
    # bytes (f16 inf/NaN scales) that must compute what the CPU path computes
    cols, tokens = 2048, 24
    specs = [(12, 2048, synth.matrix(12, 2048, cols, seed=1)),
             (12, 256, synth.matrix(12, 256, cols, seed=2)),
             (14, 100, O.pseudo_random_bytes(100 * synth.row_bytes(14, cols), 7)),
             (12, 64, O.pseudo_random_bytes(64 * synth.row_bytes(12, cols), 8))]
    mats = [R.Matrix.load(ctx, t, d, rows, cols) for t, rows, d in specs]
    x = synth.normal_f32(tokens * cols, seed=5)
    outs = [np.full(rows * tokens, np.nan, np.float32) for _, rows, _ in specs]
    R.matmul_batch(ctx, x, tokens, list(zip(mats, outs)))
    for (t, rows, d), out in zip(specs, outs):
        assert_same_bits(out, oracle_matmul(t, d, rows, cols, x, tokens), f"type {t} rows {rows}")


# ---------------------------------------------------- I2_S prefill GEMM (MFMA)


I2S_GEMM_SHAPES = [
    (6912, 2560, [64, 512]),   # BitNet 2B4T up/gate over a prefill chunk and a long prompt
    (2560, 6912, [128]),       # down: 54 blocks per row
    (33, 384, [9, 77, 300]),   # ragged rows and tokens, both token tiles
    (130, 128, [16]),          # one block per row
]


@pytest.mark.parametrize("rows,cols,token_counts", I2S_GEMM_SHAPES)
def test_i2s_prefill_gemm_is_bit_exact(ctx, rows, cols, token_counts):
    # ternary.rs:11-57 on int8 MFMA: the i32 dots equal the CPU path's, and
    # the scaled outputs its bits
    assert R.lib().rh_gemm_min_tokens() <= min(token_counts)
    data = synth.i2s_matrix(rows, cols, seed=rows + cols)
    m = R.Matrix.load(ctx, 36, data, rows, cols)
    rb = cols // 4
    for tokens in token_counts:
        x = synth.normal_f32(tokens * cols, seed=30 + tokens)
        raw = ctx.ternary_dot_i32(m, x, tokens)
        want = O.ternary_dot_matrix_i32(data[: rows * rb], rb, x, tokens)
        assert np.array_equal(raw, want), f"{rows}x{cols} tokens={tokens}"
        out = np.full(rows * tokens, np.nan, np.float32)
        R.matmul_batch(ctx, x, tokens, [(m, out)])
        assert_same_bits(out, oracle_matmul(36, data, rows, cols, x, tokens, scale=0.02, threads=16),
                         f"{rows}x{cols} tokens={tokens}")


@pytest.mark.parametrize("bn", ["32", "64"])
def test_i2s_gemm_token_tiles(ctx, tuning, bn):
    # the I2_S GEMM at both token tiles: ragged rows (a wave's rows past the
    # end) and tokens, one block, 54 blocks (the loads three blocks ahead run
    # past the last block), two jobs in one launch; its i32 dots against the
    # CPU path's
    tuning.set("RUSTICIDE_HIP_GEMM_BN", bn)
    for rows, cols, tokens in ((300, 384, 77), (33, 128, 9), (2560, 6912, 40), (257, 1024, 130), (64, 256, 33)):
        data = synth.i2s_matrix(rows, cols, seed=rows * 3 + cols)
        m = R.Matrix.load(ctx, 36, data, rows, cols)
        x = synth.normal_f32(tokens * cols, seed=tokens + cols)
        raw = ctx.ternary_dot_i32(m, x, tokens)
        want = O.ternary_dot_matrix_i32(data[: rows * cols // 4], cols // 4, x, tokens)
        assert np.array_equal(raw, want), f"{rows}x{cols} tokens={tokens} bn={bn}"
    specs = [(96, synth.i2s_matrix(96, 512, seed=1)), (200, synth.i2s_matrix(200, 512, seed=2))]
    mats = [R.Matrix.load(ctx, 36, d, r, 512) for r, d in specs]
    x = synth.normal_f32(50 * 512, seed=9)
    outs = [np.full(r * 50, np.nan, np.float32) for r, _ in specs]
    R.matmul_batch(ctx, x, 50, list(zip(mats, outs)))
    for (r, d), out in zip(specs, outs):
        assert_same_bits(out, oracle_matmul(36, d, r, 512, x, 50, scale=0.02), f"two jobs, rows {r}")


def test_i2s_prefill_gemm_every_code_and_hostile_activations(ctx):
    # random packed bytes use code 3 (+2, i2_s.rs:96-104); activations with
    # NaN, infinities and zeros exercise the I8_S rules (q8.rs:38-49,99-105);
    # two ternary matrices share the launch
    rows, cols, tokens = 96, 1024, 40
    specs = []
    for seed, scale in ((11, 0.75), (12, -3.0)):
        body = O.pseudo_random_bytes(rows * cols // 4, seed)
        data = np.concatenate([body, np.array([scale], np.float32).view(np.uint8), np.zeros(28, np.uint8)])
        specs.append((data, scale))
    mats = [R.Matrix.load(ctx, 36, d, rows, cols) for d, _ in specs]
    x = synth.normal_f32(tokens * cols, seed=41).reshape(tokens, cols)
    x[3, 17] = np.nan
    x[5, :] = 0.0
    x[7, 100] = np.inf
    x[9, 1000] = -np.inf
    x[11, -1] = np.nan
    x = x.reshape(-1)
    outs = [np.full(rows * tokens, np.nan, np.float32) for _ in mats]
    R.matmul_batch(ctx, x, tokens, list(zip(mats, outs)))
    for (d, scale), m, out in zip(specs, mats, outs):
        raw = ctx.ternary_dot_i32(m, x, tokens)
        assert np.array_equal(raw, O.ternary_dot_matrix_i32(d[: rows * cols // 4], cols // 4, x, tokens))
        assert_same_bits(out, oracle_matmul(36, d, rows, cols, x, tokens, scale=scale), f"scale {scale}")


# --------------------------------------------------------------- I2_S GEMV


I2S_SHAPES = [(6912, 2560, [1, 2]), (2560, 6912, [1, 2]), (33, 384, [1, 4, 9]), (17, 8192, [1, 2])]


@pytest.mark.parametrize("rows,cols,token_counts", I2S_SHAPES)
def test_i2s_i32_accumulators_are_bit_exact(ctx, variant, rows, cols, token_counts):
    data = synth.i2s_matrix(rows, cols, seed=rows)
    m = R.Matrix.load(ctx, 36, data, rows, cols)
    assert m.ternary_scale == np.float32(0.02)
    rb = cols // 4
    for tokens in token_counts:
        x = synth.normal_f32(tokens * cols, seed=10 + tokens)
        raw = ctx.ternary_dot_i32(m, x, tokens)
        want = O.ternary_dot_matrix_i32(data[: rows * rb], rb, x, tokens)
        assert np.array_equal(raw, want), f"{rows}x{cols} tokens={tokens}"
        out = np.full(rows * tokens, np.nan, np.float32)
        R.matmul_batch(ctx, x, tokens, [(m, out)])
        assert_same_bits(out, oracle_matmul(36, data, rows, cols, x, tokens, scale=0.02))


@pytest.mark.parametrize("groups", ["1", "2", "4"])
def test_i2s_row_groups_per_workgroup(ctx, tuning, groups):
    # RUSTICIDE_HIP_I2S_GROUPS: one activation quantization per workgroup
    # serves 1, 2 or 4 groups of rows; ragged row counts leave groups empty
    tuning.set("RUSTICIDE_HIP_I2S_GROUPS", groups)
    for rows, cols in ((6912, 2560), (2560, 6912), (37, 384), (300, 1024)):
        data = synth.i2s_matrix(rows, cols, seed=rows + 1)
        m = R.Matrix.load(ctx, 36, data, rows, cols)
        rb = cols // 4
        for tokens in (1, 2):
            x = synth.normal_f32(tokens * cols, seed=20 + tokens)
            raw = ctx.ternary_dot_i32(m, x, tokens)
            assert np.array_equal(raw, O.ternary_dot_matrix_i32(data[: rows * rb], rb, x, tokens)), (rows, cols)
            out = np.full(rows * tokens, np.nan, np.float32)
            R.matmul_batch(ctx, x, tokens, [(m, out)])
            assert_same_bits(out, oracle_matmul(36, data, rows, cols, x, tokens, scale=0.02), f"{rows}x{cols}")


def test_i2s_code_three_and_hostile_bytes(ctx):
    # i2_s.rs:96-104: code 3 decodes to +2; random bytes use every code
    rows, cols = 16, 512
    body = O.pseudo_random_bytes(rows * cols // 4, 9)
    data = np.concatenate([body, np.array([0.75], np.float32).view(np.uint8), np.zeros(28, np.uint8)])
    m = R.Matrix.load(ctx, 36, data, rows, cols)
    x = O.pseudo_random_values(cols, 5)
    raw = ctx.ternary_dot_i32(m, x, 1)
    assert np.array_equal(raw, O.ternary_dot_matrix_i32(body, cols // 4, x, 1))


@pytest.mark.parametrize("threads", ["256", "512", "1024"])
def test_i2s_one_token_kernel_at_every_workgroup_size(ctx, tuning, threads):
    # 256, 512 or 1024 threads a workgroup (lanes per row scaled with them):
    # ragged rows, 128 to 8192 values, hostile activations
    tuning.set("RUSTICIDE_HIP_I2S_NT", threads)
    for rows, cols in ((6912, 2560), (2560, 6912), (37, 384), (300, 1024), (17, 8192), (5, 128)):
        data = synth.i2s_matrix(rows, cols, seed=rows + 5)
        m = R.Matrix.load(ctx, 36, data, rows, cols)
        rb = cols // 4
        xs = [synth.normal_f32(cols, seed=cols + 1)] + (hostile_rows(cols) if rows == 300 else [])
        for i, x in enumerate(xs):
            raw = ctx.ternary_dot_i32(m, x, 1)
            assert np.array_equal(raw, O.ternary_dot_matrix_i32(data[: rows * rb], rb, x, 1)), (rows, cols, i)
            out = np.full(rows, 7.0, np.float32)
            R.matmul_batch(ctx, x, 1, [(m, out)])
            assert_same_bits(out, oracle_matmul(36, data, rows, cols, x, 1, scale=0.02), f"{rows}x{cols} x{i}")


def hostile_rows(cols):
    # q8.rs:38-49: a NaN restarts the running maximum, a trailing NaN leaves
    # it NaN, an infinity makes the divisor 0, all zeros floor it at 1e-5
    rows = []
    for case in range(5):
        x = synth.normal_f32(cols, seed=40 + case)
        if case == 0:
            x[cols // 3] = np.nan
            x[cols // 3 + 7] = 9.0
            x[cols // 5] = -50.0  # larger, but before the NaN
        elif case == 1:
            x[-1] = np.nan
        elif case == 2:
            x[cols // 2] = np.inf
        elif case == 3:
            x[:] = 0.0
        else:
            x[3] = -np.inf
            x[cols - 40] = np.nan
        rows.append(x)
    return rows


@pytest.mark.parametrize("family", ["fused", "lds"])
@pytest.mark.parametrize("lanes", ["8", "16", "32", "64", "two-token"])
def test_i2s_one_token_kernel_at_every_team_width(ctx, tuning, lanes, family):
    # the one-token kernel with 8..64 lanes per row (and the two-token kernel
    # it replaces), fused or on a separately quantized activation: ragged row
    # counts, 128 to 8192 values, hostile activations, and one launch over
    # matrices that cover different numbers of blocks of the activation
    # (ternary.rs:21-26); on the pre-quantized path also 3 to 8 tokens at once
    if family == "lds":
        tuning.set("RUSTICIDE_HIP_GEMV", "lds")
    if lanes == "two-token":
        tuning.set("RUSTICIDE_HIP_I2S_ONE", "0")
    else:
        tuning.set("RUSTICIDE_HIP_I2S_LPR", lanes)
    for rows, cols in ((6912, 2560), (2560, 6912), (37, 384), (300, 1024), (17, 8192), (5, 128)):
        data = synth.i2s_matrix(rows, cols, seed=rows + 3)
        m = R.Matrix.load(ctx, 36, data, rows, cols)
        rb = cols // 4
        xs = [synth.normal_f32(cols, seed=cols)] + (hostile_rows(cols) if rows == 300 else [])
        for i, x in enumerate(xs):
            raw = ctx.ternary_dot_i32(m, x, 1)
            assert np.array_equal(raw, O.ternary_dot_matrix_i32(data[: rows * rb], rb, x, 1)), (rows, cols, i)
            out = np.full(rows, 7.0, np.float32)
            R.matmul_batch(ctx, x, 1, [(m, out)])
            assert_same_bits(out, oracle_matmul(36, data, rows, cols, x, 1, scale=0.02), f"{rows}x{cols} x{i}")
    specs = [(70, 1024), (33, 512), (129, 384), (8, 1280)]
    datas = [synth.i2s_matrix(r, c, seed=r) for r, c in specs]
    mats = [R.Matrix.load(ctx, 36, d, r, c) for d, (r, c) in zip(datas, specs)]
    for width in (1024, 1000):
        x = synth.normal_f32(width, seed=width)
        outs = [np.full(r, 7.0, np.float32) for r, _ in specs]
        R.matmul_batch(ctx, x, 1, list(zip(mats, outs)))
        for (r, c), d, out in zip(specs, datas, outs):
            assert_same_bits(out, oracle_matmul(36, d, r, c, x, 1, scale=0.02), f"{r}x{c} width {width}")
    if family == "lds":
        rows, cols = 300, 2560
        data = synth.i2s_matrix(rows, cols, seed=5)
        m = R.Matrix.load(ctx, 36, data, rows, cols)
        for tokens in (3, 5, 8):
            x = np.concatenate([synth.normal_f32(cols * (tokens - 1), seed=tokens), hostile_rows(cols)[0]])
            raw = ctx.ternary_dot_i32(m, x, tokens)
            assert np.array_equal(raw, O.ternary_dot_matrix_i32(data[: rows * cols // 4], cols // 4, x, tokens))
            out = np.full(rows * tokens, 7.0, np.float32)
            R.matmul_batch(ctx, x, tokens, [(m, out)])
            assert_same_bits(out, oracle_matmul(36, data, rows, cols, x, tokens, scale=0.02), f"tokens {tokens}")


# ------------------------------------------------------------ batch rules


def test_one_round_jobs_of_several_widths(ctx, variant):
    # one launch of 17- to 32-block jobs: 22 and 24 blocks both have the
    # unit-layout copy and 8-row workgroups of whole groups; a 23-block job
    # (no copy) puts the whole launch on the native rows
    width = 6144
    specs = [(14, 2048, 5632), (14, 300, 6144), (14, 50, 5888)]
    mats, datas = [], []
    for i, (t, rows, cols) in enumerate(specs):
        d = synth.matrix(t, rows, cols, seed=300 + i)
        datas.append(d)
        mats.append(R.Matrix.load(ctx, t, d, rows, cols))
    x = synth.normal_f32(width, seed=78)
    for n in (2, 3):
        outs = [np.full(rows, np.nan, np.float32) for _, rows, _ in specs[:n]]
        R.matmul_batch(ctx, x, 1, list(zip(mats[:n], outs)))
        for (t, rows, cols), d, out in zip(specs, datas, outs):
            assert_same_bits(out, oracle_matmul(t, d, rows, cols, x[:cols], 1), f"{n} jobs: {rows}x{cols}")


def test_one_batch_mixes_formats_and_matches_per_token_calls(ctx, variant):
    # attention.rs:215-223 (Q/K/V in one batch) + matmul_tests.rs:237-271
    cols, tokens = 2048, 5
    specs = [(12, 2048), (12, 256), (14, 256), (36, 300), (14, 40)]
    mats, datas = [], []
    for i, (t, rows) in enumerate(specs):
        d = synth.matrix(t, rows, cols, seed=100 + i)
        datas.append(d)
        mats.append(R.Matrix.load(ctx, t, d, rows, cols))
    x = synth.normal_f32(tokens * cols, seed=77)
    outs = [np.full(rows * tokens, np.nan, np.float32) for _, rows in specs]
    R.matmul_batch(ctx, x, tokens, list(zip(mats, outs)))
    for (t, rows), d, m, out in zip(specs, datas, mats, outs):
        assert_same_bits(out, oracle_matmul(t, d, rows, cols, x, tokens, scale=0.02), f"type {t}")
        for tok in range(tokens):
            single = np.zeros(rows, np.float32)
            R.matvec_batch(ctx, x[tok * cols:(tok + 1) * cols], [(m, single)])
            assert_same_bits(out[tok::tokens], single, f"type {t} token {tok}")


def test_no_ops_and_output_bounds(ctx):
    # matmul_tests.rs:188-235; quant_kernel.rs:106-111
    rows, cols = 20, 512
    data = synth.matrix(12, rows, cols, seed=5)
    m = R.Matrix.load(ctx, 12, data, rows, cols)
    out = np.full(rows, 7.0, np.float32)
    R.matmul_batch(ctx, np.ones(cols, np.float32), 0, [(m, out)])
    R.matmul_batch(ctx, np.ones(cols, np.float32), cols + 1, [(m, out)])
    assert np.all(out == 7.0)
    x = synth.normal_f32(2 * cols, seed=6)
    full = np.zeros(rows * 2, np.float32)
    R.matmul_batch(ctx, x, 2, [(m, full)])
    short = np.full(13, 5.0, np.float32)  # 6.5 rows of 2 tokens
    R.matmul_batch(ctx, x, 2, [(m, short)])
    assert_same_bits(short, full[:13])
    long = np.full(rows * 2 + 3, 5.0, np.float32)
    R.matmul_batch(ctx, x, 2, [(m, long)])
    assert_same_bits(long[:-3], full)
    assert np.all(long[-3:] == 5.0)


def test_an_input_narrower_than_the_rows_bounds_the_dot(ctx, variant):
    # int_dot.rs:36-47 and ternary.rs:21-26: the shorter operand bounds the work
    rows, cols = 12, 1024
    for t in (12, 14, 36):
        data = synth.matrix(t, rows, cols, seed=8)
        m = R.Matrix.load(ctx, t, data, rows, cols)
        for width in (512, 300, 100, 0 if t != 36 else 40):
            if width == 0:
                continue
            x = synth.normal_f32(width, seed=9)
            out = np.full(rows, np.nan, np.float32)
            R.matvec_batch(ctx, x, [(m, out)])
            assert_same_bits(out, oracle_matmul(t, data, rows, cols, x, 1, scale=0.02), f"type {t} width {width}")


def test_dense_f32_rows_follow_the_eight_lane_dot(ctx):
    # rusticide-simd/src/float.rs:23-36
    rng = np.random.default_rng(1)
    for rows, cols in ((7, 37), (65, 2048), (3, 5)):
        w = rng.standard_normal(rows * cols).astype(np.float32)
        m = R.Matrix.load(ctx, R.F32, w, rows, cols)
        x = rng.standard_normal(cols * 2).astype(np.float32)
        out = np.zeros(rows * 2, np.float32)
        R.matmul_batch(ctx, x, 2, [(m, out)])
        assert_same_bits(out, oracle_matmul(0, w, rows, cols, x, 2))


def test_hostile_block_bytes_match_the_oracle(ctx, variant):
    # the fuzz idea (rusticide-fuzz dequantize target): any bytes, incl. f16
    # inf/NaN scales, must compute what the CPU path computes
    rows, cols = 40, 512
    for t in (12, 14):
        data = O.pseudo_random_bytes(rows * synth.row_bytes(t, cols), 21 + t)
        m = R.Matrix.load(ctx, t, data, rows, cols)
        x = synth.normal_f32(cols * 2, seed=3)
        out = np.zeros(rows * 2, np.float32)
        R.matmul_batch(ctx, x, 2, [(m, out)])
        assert_same_bits(out, oracle_matmul(t, data, rows, cols, x, 2), f"type {t}")


# ------------------------------------------------------------ load errors


def test_load_errors_mirror_model_error(ctx):
    # model/src/weights.rs:41-47,190-211
    with pytest.raises(R.RusticideError) as e:
        R.Matrix.load(ctx, 12, np.zeros(144, np.uint8), 1, 0)
    assert e.value.kind == "INVALID_CONFIG"
    for scale in (np.nan, np.inf, -np.inf):
        data = np.concatenate([np.zeros(32, np.uint8), np.array([scale], np.float32).view(np.uint8)])
        with pytest.raises(R.RusticideError) as e:
            R.Matrix.load(ctx, 36, data, 1, 128)
        assert e.value.kind == "INVALID_TENSOR" and "not finite" in str(e.value)
    with pytest.raises(R.RusticideError) as e:
        R.Matrix.load(ctx, 36, np.zeros(34, np.uint8), 1, 128)
    assert e.value.kind == "INVALID_TENSOR" and "too short" in str(e.value)
    with pytest.raises(R.RusticideError) as e:
        R.Matrix.load(ctx, 12, np.zeros(143, np.uint8), 1, 256)
    assert e.value.kind == "SHAPE_MISMATCH"
    with pytest.raises(R.RusticideError) as e:
        R.Matrix.load(ctx, 2, np.zeros(18, np.uint8), 1, 32)
    assert e.value.kind == "MISSING_KERNEL"
    # the kernels' 24-bit row / 32-bit offset addressing is checked at load
    with pytest.raises(R.RusticideError) as e:
        R.Matrix.load(ctx, 12, np.zeros(144, np.uint8), 1 << 24, 256)
    assert e.value.kind == "SHAPE_MISMATCH" and "4 GiB" in str(e.value)


# --------------------------------------------------------------- copy_row


@pytest.mark.parametrize("type_id", [12, 14, 36])
def test_copy_row_dequantizes_like_the_cpu_path(ctx, type_id):
    # model/src/weights.rs:120-150
    rows, cols = 9, 768 if type_id != 36 else 384
    data = synth.matrix(type_id, rows, cols, seed=4)
    m = R.Matrix.load(ctx, type_id, data, rows, cols)
    rb = synth.row_bytes(type_id, cols)
    for r in (0, rows - 1):
        out = np.full(cols, np.nan, np.float32)
        assert m.copy_row(r, out)
        want = O.dequantize_row(type_id, data[r * rb:(r + 1) * rb])
        if type_id == 36:
            want = (want * np.float32(0.02)).astype(np.float32)
        assert_same_bits(out, want)
    assert not m.copy_row(rows, np.zeros(cols, np.float32))


# ------------------------------------------- Q8Input::quantize + dot_matrix


@pytest.mark.parametrize("type_id,rows,cols", [(12, 300, 2048), (14, 257, 1536), (36, 333, 2560)])
@pytest.mark.parametrize("tokens", [1, 2, 9, 33])
def test_dot_matrix_device_matches_the_oracle(ctx, type_id, rows, cols, tokens):
    # QuantKernel::dot_matrix (quant_kernel.rs:112-119, tested at
    # quant_kernel_tests.rs:202-230): every row against each pre-quantized
    # input, out[row * tokens + token], here with the activation quantized on
    # the device (rh_q8_quantize_device) and 9+ tokens taking the MFMA GEMM
    from rusticide_amd import hip as H
    data = synth.i2s_matrix(rows, cols, seed=rows) if type_id == 36 else synth.matrix(type_id, rows, cols, seed=rows)
    m = R.Matrix.load(ctx, type_id, data, rows, cols)
    x = synth.normal_f32(tokens * cols, seed=tokens + cols)
    want = oracle_matmul(type_id, data, rows, cols, x, tokens, scale=0.02, threads=16)
    d_x = H.DeviceArray.from_numpy(x)
    q8 = R.Q8(ctx).quantize(d_x, tokens, R.ROW if type_id == 36 else R.SUPER_BLOCK)
    out = H.DeviceArray(rows * tokens)
    out.fill_bytes(0xFF)
    R.dot_matrix_device(m, q8, out)
    H.synchronize()
    assert_same_bits(out.numpy(), want, f"type={type_id} {rows}x{cols} tokens={tokens}")
    # out.len() bounds the rows computed: nothing past it is written
    short = H.DeviceArray(rows * tokens)
    short.fill_bytes(0xFF)
    n = 5 * tokens + 1
    lib_out = R.lib().rh_dot_matrix_device(ctx.handle, m.handle, q8.handle, short.data_ptr(), n, None)
    ctx.check(lib_out)
    H.synchronize()
    got = short.numpy()
    assert_same_bits(got[:n], want[:n], "short output")
    assert np.all(got[n:].view(np.uint32) == 0xFFFFFFFF), "wrote past out_len"
    for a in (d_x, out, short):
        a.free()
    q8.free()
    m.free()


def test_device_block_terms_round_like_the_reference(ctx):
    # the rounding pins of test_oracle_rounding.py, on the device path: a
    # Q4_K and a Q6_K matrix whose rows separate the reference's combine
    # (d8 * d.mul_add(isum, -(dmin*msum)); (d*d8)*isum; the fold from -0.0
    # in block order) from its plausible slips, with the expected bits from
    # exact rationals on the activation the quantizer produced
    from fractions import Fraction
    import test_oracle_rounding as T
    rng = np.random.default_rng(4)
    cols, rows = 2048, 24
    x = rng.standard_normal(cols).astype(np.float32)
    q = O.quantize(x, O.SUPER_BLOCK)
    steps = [Fraction(float(q.scales[8 * b])) for b in range(cols // 256)]  # one step per super-block
    quants = q.quants.astype(np.int64)
    for type_id in (12, 14):
        data, want = b"", []
        for r in range(rows):
            blocks, seq = [], Fraction(0)
            for b in range(cols // 256):
                qb = quants[256 * b:256 * (b + 1)]
                if type_id == 12:
                    d, dmin, sc, mn, nib, _ = T.q4k_parts(rng)
                    isum, msum = T.q4k_sums(sc, mn, nib, qb)
                    blocks.append(T.q4k_block(d, dmin, sc, mn, nib))
                    term = T.q4k_term(T.f16_value(d), T.f16_value(dmin), steps[b], isum, msum)
                else:
                    qq = [int(v) for v in rng.integers(0, 64, 256)]
                    scales = rng.integers(-32, 32, 16)
                    d = T.f16_bits(float(rng.uniform(-0.01, 0.01)))
                    blocks.append(T.q6k_block(qq, scales, d))
                    term = T.f32(T.f32(T.f16_value(d) * steps[b]) * T.q6k_isum(qq, scales, qb))
                seq = T.f32(seq + term)  # from -0.0: the first term unchanged
            data += b"".join(blocks)
            assert seq != 0  # a zero sum's sign is not a rational's to tell
            want.append(float(seq))
        m = R.Matrix.load(ctx, type_id, np.frombuffer(data, np.uint8), rows, cols)
        for tokens in (1, 9):  # the decode GEMV and the MFMA GEMM
            xt = np.tile(x, tokens)
            out = np.full(rows * tokens, np.nan, np.float32)
            R.matmul_batch(ctx, xt, tokens, [(m, out)])
            got = out.reshape(rows, tokens)
            for t in range(tokens):
                assert [T.bits32(v) for v in got[:, t]] == [T.bits32(v) for v in want], (type_id, tokens, t)
        m.free()
