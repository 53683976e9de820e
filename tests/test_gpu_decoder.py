"""The device decoder against the CPU restatement of rusticide's decoder.

Bar: end-to-end greedy tokens from random-init models identical to the CPU
path. The products are bit-identical by construction;
the f32 glue follows the reference's operation order, so logits are compared
bit for bit as well, with the largest difference reported if they ever part.
"""

import numpy as np
import pytest

import oracle as O
import rusticide_amd as R
from rusticide_amd import synth

pytestmark = pytest.mark.gpu

SMALL = dict(embedding_length=256, block_count=2, feed_forward_length=512, head_count=4, head_count_kv=2,
             head_dim=64, context_length=160, vocab_size=320, rope_freq_base=10000.0, rms_norm_eps=1e-5)


@pytest.fixture(scope="module")
def ctx():
    c = R.Context(0)
    yield c
    c.close()


@pytest.fixture(params=["fused", "separate"])
def norm_path(request, monkeypatch):
    # one-token forwards fold each RMSNorm into the GEMV after it unless
    # RUSTICIDE_HIP_NORM_FUSE=0, and batches quantize the normed rows in the
    # norm kernel unless RUSTICIDE_HIP_NORM_QUANT=0 (both read when a decoder
    # is created); every combination gives the CPU path's bits
    if request.param == "separate":
        monkeypatch.setenv("RUSTICIDE_HIP_NORM_FUSE", "0")
        monkeypatch.setenv("RUSTICIDE_HIP_NORM_QUANT", "0")
    else:
        monkeypatch.delenv("RUSTICIDE_HIP_NORM_FUSE", raising=False)
        monkeypatch.delenv("RUSTICIDE_HIP_NORM_QUANT", raising=False)
    return request.param


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def diff(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def test_small_decoder_logits_match_the_cpu_path(ctx, norm_path):
    model = synth.decoder_model(SMALL, seed=11)
    gpu, cpu = R.Decoder(ctx, model), O.Decoder(model, threads=8)
    rng = np.random.default_rng(3)
    tokens = rng.integers(0, SMALL["vocab_size"], 70).astype(np.uint32)
    # a 64-token prefill chunk, a ragged one, then single tokens
    for start, chunk in ((0, tokens[:64]), (64, tokens[64:69]), (69, tokens[69:70])):
        g = gpu.forward_batch(chunk, start)
        c = cpu.forward_batch(chunk, start)
        assert same_bits(g, c), f"start {start}: max |diff| {diff(g, c)}"
    assert gpu.position == 70
    gpu.close()
    cpu.close()


def test_small_decoder_batch_equals_token_by_token(ctx, norm_path):
    # decoder_batch_tests.rs:50-66: a batch's last logits equal those of the
    # same tokens fed one at a time
    model = synth.decoder_model(SMALL, seed=12)
    gpu = R.Decoder(ctx, model)
    tokens = [5, 17, 300, 2, 99, 41, 7]
    batch = gpu.forward_batch(tokens, 0)
    gpu.reset()
    for i, t in enumerate(tokens):
        single = gpu.forward(t, i)
    assert same_bits(batch, single), diff(batch, single)
    gpu.close()


def test_small_decoder_greedy_generation_matches(ctx, norm_path):
    model = synth.decoder_model(SMALL, seed=13)
    gpu, cpu = R.Decoder(ctx, model), O.Decoder(model, threads=8)
    prompt = np.random.default_rng(4).integers(0, SMALL["vocab_size"], 70).astype(np.uint32)
    want = cpu.generate_greedy(prompt, 40)
    got = gpu.generate_greedy(prompt, 40)
    assert np.array_equal(got, want), (got, want)
    # generation stops at the context end (generate.rs:102-104)
    near = np.arange(150, dtype=np.uint32) % SMALL["vocab_size"]
    got = gpu.generate_greedy(near, 40)
    want = cpu.generate_greedy(near, 40)
    assert len(got) == len(want) == 11 and np.array_equal(got, want)
    gpu.close()
    cpu.close()


def test_batched_forward_graph_replays_match_the_eager_run(ctx, monkeypatch):
    # with RUSTICIDE_HIP_GRAPHS=1 (read at creation) a decoder replays the
    # graph it captured for a (tokens, start) batch; every replay, with eager
    # work and synchronizations between replays, must give the bits of a
    # decoder that launches one kernel at a time and of the CPU path
    model = synth.decoder_model(SMALL, seed=15)
    monkeypatch.setenv("RUSTICIDE_HIP_GRAPHS", "0")
    eager = R.Decoder(ctx, model)
    monkeypatch.setenv("RUSTICIDE_HIP_GRAPHS", "1")
    graphed = R.Decoder(ctx, model)
    monkeypatch.delenv("RUSTICIDE_HIP_GRAPHS")
    cpu = O.Decoder(model, threads=8)
    rng = np.random.default_rng(8)
    for rep in range(5):
        prompt = rng.integers(0, SMALL["vocab_size"], 70).astype(np.uint32)
        graphed.reset()
        eager.reset()
        g = graphed.forward_batch(prompt[:64], 0)  # rep 0 captures, later reps replay
        e = eager.forward_batch(prompt[:64], 0)
        assert same_bits(g, e), f"replay {rep}: max |diff| {diff(g, e)}"
        if rep in (0, 4):
            cpu.reset()
            assert same_bits(g, cpu.forward_batch(prompt[:64], 0))
        # eager work between replays: a single token, then a ragged chunk
        assert same_bits(graphed.forward(int(prompt[64]), 64), eager.forward(int(prompt[64]), 64))
        assert same_bits(graphed.forward_batch(prompt[65:70], 65), eager.forward_batch(prompt[65:70], 65))
        # generation replays the (64, 0) and (6, 64) prefill graphs
        assert np.array_equal(graphed.generate_greedy(prompt, 6), eager.generate_greedy(prompt, 6))
    graphed.close()
    eager.close()
    cpu.close()


def test_one_token_attention_kernels_agree_at_every_length(ctx, monkeypatch):
    # a one-token step up to 224 cached rows runs the LDS-staged attention
    # kernel (RUSTICIDE_HIP_ATTN_LDS=0 keeps the tiled one); every length from
    # 1 to 241 rows, across all seven of its row-count variants and past its
    # limit, gives the tiled kernel's bits and the CPU path's
    model = synth.decoder_model(dict(SMALL, context_length=256), seed=16)
    lds, tiled = R.Decoder(ctx, model), R.Decoder(ctx, model)
    cpu = O.Decoder(model, threads=8)
    tokens = np.random.default_rng(9).integers(0, SMALL["vocab_size"], 241).astype(np.uint32)
    for pos, tok in enumerate(tokens):
        monkeypatch.setenv("RUSTICIDE_HIP_ATTN_LDS", "1")
        R.reload_tuning()
        a = lds.forward(int(tok), pos)
        monkeypatch.setenv("RUSTICIDE_HIP_ATTN_LDS", "0")
        R.reload_tuning()
        b = tiled.forward(int(tok), pos)
        assert same_bits(a, b), f"rows {pos + 1}: max |diff| {diff(a, b)}"
        c = cpu.forward(int(tok), pos)
        if pos in (0, 1, 31, 32, 100, 191, 223, 224, 240):
            assert same_bits(a, c), f"rows {pos + 1}: max |diff| {diff(a, c)}"
    monkeypatch.delenv("RUSTICIDE_HIP_ATTN_LDS")
    R.reload_tuning()
    lds.close()
    tiled.close()
    cpu.close()


def test_graph_cache_evicts_within_one_generate_call(ctx, monkeypatch):
    # the decoder keeps 8 graphs. A first call caches the 8 prefill chunks of
    # a 512-token prompt; a second call on a 583-token prompt replays those 8
    # (queued on the stream) and then captures two more chunks, evicting
    # graphs it replayed earlier in the same call. Every pick must equal the
    # eager decoder's.
    cfg = dict(SMALL, context_length=640)
    model = synth.decoder_model(cfg, seed=21)
    monkeypatch.setenv("RUSTICIDE_HIP_GRAPHS", "0")
    eager = R.Decoder(ctx, model)
    monkeypatch.setenv("RUSTICIDE_HIP_GRAPHS", "1")
    graphed = R.Decoder(ctx, model)
    monkeypatch.delenv("RUSTICIDE_HIP_GRAPHS")
    rng = np.random.default_rng(21)
    prompt = rng.integers(0, cfg["vocab_size"], 64 * 9 + 7).astype(np.uint32)
    for n in (512, 64 * 9 + 7, 512, 64 * 9 + 7):
        want = eager.generate_greedy(prompt[:n], 8)
        assert np.array_equal(graphed.generate_greedy(prompt[:n], 8), want), f"prompt of {n}"
    graphed.close()
    eager.close()


@pytest.mark.parametrize("head_dim,heads,kv_heads,width",
                         [(32, 8, 2, 256), (48, 16, 4, 768), (80, 16, 4, 1280), (128, 4, 2, 512)])
def test_head_dims_other_than_64_take_the_generic_attention(ctx, norm_path, head_dim, heads, kv_heads, width):
    # attention_kernel<0> (any even head_dim up to 128; above 64, 32-row value
    # tiles and a second wave of output lanes) in the batched and the
    # one-token forwards, against the CPU path
    cfg = dict(SMALL, embedding_length=width, head_count=heads, head_count_kv=kv_heads, head_dim=head_dim)
    model = synth.decoder_model(cfg, seed=head_dim)
    gpu, cpu = R.Decoder(ctx, model), O.Decoder(model, threads=8)
    tokens = np.random.default_rng(head_dim).integers(0, cfg["vocab_size"], 70).astype(np.uint32)
    for start, chunk in ((0, tokens[:64]), (64, tokens[64:69]), (69, tokens[69:70])):
        g, c = gpu.forward_batch(chunk, start), cpu.forward_batch(chunk, start)
        assert same_bits(g, c), f"start {start}: max |diff| {diff(g, c)}"
    assert np.array_equal(gpu.generate_greedy(tokens, 12), cpu.generate_greedy(tokens, 12))
    gpu.close()
    cpu.close()


@pytest.mark.parametrize("heads,kv_heads,width", [(8, 2, 512), (16, 2, 1024)])
def test_grouped_attention_matches_the_cpu_path(ctx, norm_path, heads, kv_heads, width):
    # attention_group_kernel (head_dim 64, four or eight query heads a kv
    # head) in batched forwards, its output stored or, with the norms'
    # quantization on, quantized for the O matrix; against the CPU path
    # chunks after the first reach past one 64-row value tile and start
    # mid-context (the cached rows before `start` and the chunk's own)
    cfg = dict(SMALL, embedding_length=width, head_count=heads, head_count_kv=kv_heads, head_dim=64,
               context_length=256)
    model = synth.decoder_model(cfg, seed=heads)
    gpu, cpu = R.Decoder(ctx, model), O.Decoder(model, threads=8)
    tokens = np.random.default_rng(heads).integers(0, cfg["vocab_size"], 200).astype(np.uint32)
    for start, end in ((0, 64), (64, 69), (69, 70), (70, 134), (134, 200)):
        g, c = gpu.forward_batch(tokens[start:end], start), cpu.forward_batch(tokens[start:end], start)
        assert same_bits(g, c), f"start {start}: max |diff| {diff(g, c)}"
    assert np.array_equal(gpu.generate_greedy(tokens[:70], 12), cpu.generate_greedy(tokens[:70], 12))
    gpu.close()
    cpu.close()


def test_token_major_split_gemms_over_partial_token_tiles(ctx):
    # batches of 36, 12 and 52 tokens (multiples of 4, not of 32): the split
    # QKV GEMM's tile fixup transposes the last, partial token tile of its
    # token-major outputs through LDS, the O planes and the down combine are
    # token-major; 66 tokens (not a multiple of 4) take the combine launch
    cfg = dict(SMALL, embedding_length=1024, head_count=16, head_count_kv=2, head_dim=64, context_length=256)
    model = synth.decoder_model(cfg, seed=37)
    gpu, cpu = R.Decoder(ctx, model), O.Decoder(model, threads=16)
    tokens = np.random.default_rng(37).integers(0, cfg["vocab_size"], 166).astype(np.uint32)
    for start, end in ((0, 36), (36, 48), (48, 100), (100, 166)):
        g, c = gpu.forward_batch(tokens[start:end], start), cpu.forward_batch(tokens[start:end], start)
        assert same_bits(g, c), f"start {start}: max |diff| {diff(g, c)}"
    gpu.close()
    cpu.close()


@pytest.mark.parametrize("tokens", [200, 320])
def test_long_batches_store_the_residual_token_major_without_a_split(ctx, tokens):
    # batches long enough that the O and down GEMMs run unsplit store the
    # residual delta token-major from the GEMM epilogue itself (shorter ones
    # through the split-K combine); a single forward_batch against the CPU path
    cfg = dict(SMALL, embedding_length=1024, head_count=16, head_count_kv=2, head_dim=64, context_length=512)
    model = synth.decoder_model(cfg, seed=71)
    gpu, cpu = R.Decoder(ctx, model), O.Decoder(model, threads=16)
    seq = np.random.default_rng(tokens).integers(0, cfg["vocab_size"], tokens + 1).astype(np.uint32)
    g, c = gpu.forward_batch(seq[:tokens], 0), cpu.forward_batch(seq[:tokens], 0)
    assert same_bits(g, c), f"max |diff| {diff(g, c)}"
    g, c = gpu.forward_batch(seq[tokens:], tokens), cpu.forward_batch(seq[tokens:], tokens)
    assert same_bits(g, c), f"next token: max |diff| {diff(g, c)}"
    gpu.close()
    cpu.close()


def test_grouped_attention_one_token_forwards_without_norm_fusion(ctx, monkeypatch):
    # RUSTICIDE_HIP_NORM_FUSE=0 with the quantizing kernels on: one-token
    # forwards take the batched path, where the grouped attention's Q8_K
    # output feeds the O matrix's one-token GEMV
    monkeypatch.setenv("RUSTICIDE_HIP_NORM_FUSE", "0")
    monkeypatch.delenv("RUSTICIDE_HIP_NORM_QUANT", raising=False)
    cfg = dict(SMALL, embedding_length=1024, head_count=16, head_count_kv=2, head_dim=64)
    model = synth.decoder_model(cfg, seed=61)
    gpu, cpu = R.Decoder(ctx, model), O.Decoder(model, threads=8)
    tokens = np.random.default_rng(61).integers(0, cfg["vocab_size"], 20).astype(np.uint32)
    for start, chunk in ((0, tokens[:16]), (16, tokens[16:17]), (17, tokens[17:20])):
        g, c = gpu.forward_batch(chunk, start), cpu.forward_batch(chunk, start)
        assert same_bits(g, c), f"start {start}: max |diff| {diff(g, c)}"
    assert np.array_equal(gpu.generate_greedy(tokens, 8), cpu.generate_greedy(tokens, 8))
    gpu.close()
    cpu.close()


def test_contexts_past_64_kib_of_attention_lds(ctx):
    # the attention kernels keep a context's weights in one workgroup's LDS:
    # at 9,000 rows that is more than 64 KiB (gfx950 gives a workgroup
    # 160 KiB). A batch's last logits equal those of the same tokens fed one
    # at a time (decoder_batch_tests.rs:50-66), here deep in the context
    model = synth.decoder_model(dict(SMALL, context_length=9100), seed=17)
    batched, single = R.Decoder(ctx, model), R.Decoder(ctx, model)
    tokens = np.random.default_rng(10).integers(0, SMALL["vocab_size"], 8969).astype(np.uint32)
    for d in (batched, single):
        for start in range(0, 8960, 64):
            d.forward_batch(tokens[start:start + 64], start)
    b = batched.forward_batch(tokens[8960:], 8960)
    for pos in range(8960, 8969):
        s_ = single.forward(int(tokens[pos]), pos)
    assert same_bits(b, s_), diff(b, s_)
    assert np.all(np.isfinite(b))
    batched.close()
    single.close()


def test_decoder_errors_mirror_model_error(ctx):
    # decoder.rs:111-136, cache.rs:35-65, generate.rs:45-48
    model = synth.decoder_model(SMALL, seed=14)
    gpu = R.Decoder(ctx, model)
    with pytest.raises(R.RusticideError) as e:
        gpu.forward_batch([1, 2], SMALL["context_length"] - 1)
    assert e.value.kind == "CONTEXT_FULL"
    with pytest.raises(R.RusticideError) as e:
        gpu.forward_batch([SMALL["vocab_size"]], 0)
    assert e.value.kind == "INVALID_CONFIG"
    gpu.forward_batch([1, 2, 3], 0)
    with pytest.raises(R.RusticideError) as e:
        gpu.forward_batch([4], 5)
    assert e.value.kind == "CACHE_POSITION"
    with pytest.raises(R.RusticideError) as e:
        gpu.generate_greedy(np.zeros(SMALL["context_length"], np.uint32), 4)
    assert e.value.kind == "CONTEXT_FULL"
    gpu.close()


def test_tinyllama_shaped_greedy_decode_matches_the_cpu_path(ctx, norm_path):
    # 22 layers, hidden 2048, 32/4 heads of 64, FFN 5632, vocab 32000,
    # Q4_K_M mix; 64-token random prompt, then 128 greedy tokens
    model = synth.decoder_model(synth.TINYLLAMA, seed=2026)
    prompt = np.random.default_rng(7).integers(0, 32000, 64).astype(np.uint32)
    gpu = R.Decoder(ctx, model)
    cpu = O.Decoder(model, threads=16)
    g = gpu.forward_batch(prompt, 0)
    c = cpu.forward_batch(prompt, 0)
    assert same_bits(g, c), f"prefill logits: max |diff| {diff(g, c)}"
    want = cpu.generate_greedy(prompt, 128)
    got = gpu.generate_greedy(prompt, 128)
    assert len(got) == 128
    assert np.array_equal(got, want), f"first mismatch at {np.flatnonzero(got != want)[:1]}"
    gpu.close()
    cpu.close()


def test_one_token_launches_at_both_workgroup_sizes(ctx, monkeypatch):
    # RUSTICIDE_HIP_KQ_NT / RUSTICIDE_HIP_NORM_NT: the one-token k-quant
    # launches (norm-fused Q/K/V, attention output, gate/up, output; the
    # down projection) on 256-lane workgroups, or on 512-lane ones with half
    # the blocks per team wherever a launch has two or more; with the
    # fixed-column block walk and (RUSTICIDE_HIP_KQ_FIX=0) without: the CPU
    # path's logits every way
    model = synth.decoder_model(synth.TINYLLAMA, seed=2027)
    prompt = np.random.default_rng(8).integers(0, 32000, 9).astype(np.uint32)
    follow = [311, 7, 29999, 0, 1234]
    cpu = O.Decoder(model, threads=16)
    want = [cpu.forward_batch(prompt, 0)]
    for i, t in enumerate(follow):
        want.append(cpu.forward(t, len(prompt) + i))
    cpu.close()
    try:
        for nt, fix, bal in (("256", "1", "1"), ("512", "1", "1"), ("256", "0", "1"), ("512", "0", "1"),
                             ("0", "1", "0")):
            for name, v in (("RUSTICIDE_HIP_KQ_NT", nt), ("RUSTICIDE_HIP_NORM_NT", nt)):
                if v == "0":
                    monkeypatch.delenv(name, raising=False)
                else:
                    monkeypatch.setenv(name, v)
            monkeypatch.setenv("RUSTICIDE_HIP_KQ_FIX", fix)
            monkeypatch.setenv("RUSTICIDE_HIP_KQ_BALANCE", bal)
            R.reload_tuning()
            gpu = R.Decoder(ctx, model)
            got = [gpu.forward_batch(prompt, 0)]
            for i, t in enumerate(follow):
                got.append(gpu.forward(t, len(prompt) + i))
            gpu.close()
            for k, (g, c) in enumerate(zip(got, want)):
                assert same_bits(g, c), f"{nt} lanes, fixed walk {fix}, balance {bal}, step {k}: {diff(g, c)}"
    finally:
        for name in ("RUSTICIDE_HIP_KQ_NT", "RUSTICIDE_HIP_NORM_NT", "RUSTICIDE_HIP_KQ_FIX", "RUSTICIDE_HIP_KQ_BALANCE"):
            monkeypatch.delenv(name, raising=False)
        R.reload_tuning()


def _device_math(ctx, op, a, b=None):
    import ctypes
    L = R.lib()
    L.rh_math_device.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p,
                                 ctypes.c_void_p, ctypes.c_size_t]
    a = np.ascontiguousarray(a, np.float32)
    b = None if b is None else np.ascontiguousarray(b, np.float32)
    y = np.empty_like(a)
    ctx.check(L.rh_math_device(ctx.handle, op, a.ctypes.data, None if b is None else b.ctypes.data,
                               y.ctypes.data, len(a)))
    return y


def _assert_same(y, want, x):
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(y), nan)
    bad = np.flatnonzero(y[~nan].view(np.uint32) != want[~nan].view(np.uint32))
    assert bad.size == 0, f"{bad.size} mismatches, e.g. x={x[~nan][bad[:3]]}"


def test_device_expf_matches_libm(ctx):
    # the expf of the softmax and SiLU kernels, on the device, against libm's
    # (every 4099th bit pattern plus the special cases)
    x = np.arange(0, 1 << 32, 4099, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = np.concatenate([x, np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 88.72283, 88.72284, -103.97207,
                                     -103.97208, -87.3366, 1e-45], np.float32)])
    _assert_same(_device_math(ctx, 0, x), O.expf(x), x)


def test_device_sqrt_is_rounded_to_nearest(ctx):
    # RMSNorm's square root on the device against IEEE sqrt (numpy's), every
    # 1021st positive float plus the special cases
    x = np.arange(0, 0x7F800000, 1021, dtype=np.uint32).view(np.float32)
    x = np.concatenate([x, np.array([0.0, -0.0, np.inf, -1.0, np.nan, 1e-5, 2 ** -64, 2 ** -126], np.float32)])
    with np.errstate(invalid="ignore"):
        want = np.sqrt(x)
    _assert_same(_device_math(ctx, 1, x), want, x)


def _device_ordered_sum(ctx, values, init):
    import ctypes
    L = R.lib()
    L.rh_ordered_sum_device.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_float,
                                        ctypes.c_void_p, ctypes.c_void_p]
    v = np.ascontiguousarray(values, np.float32)
    out = np.zeros(1, np.float32)
    rounds = np.zeros(1, np.uint32)
    ctx.check(L.rh_ordered_sum_device(ctx.handle, v.ctypes.data if v.size else None, v.size, float(init),
                                      out.ctypes.data, rounds.ctypes.data))
    return out[0], int(rounds[0])


def _fold(values, init):
    # ((init + v0) + v1) + ...: numpy's accumulate adds in order, one float32
    # rounding per step
    seq = np.concatenate([np.float32([init]), np.asarray(values, np.float32)])
    with np.errstate(all="ignore"):
        return np.add.accumulate(seq, dtype=np.float32)[-1]


def _ordered_sum_cases():
    rng = np.random.default_rng(11)
    cases = []
    for n in (0, 1, 2, 31, 32, 33, 63, 64, 65, 100, 2047, 2048, 2049, 2560, 4096, 5000, 8191, 8192):
        v = rng.standard_normal(n).astype(np.float32)
        cases.append(("squares", v * v, -0.0))
    for _ in range(24):
        n = int(rng.integers(1, 8193))
        v = (rng.standard_normal(n) * np.exp(rng.uniform(-30, 30, n))).astype(np.float32)
        cases.append(("wide squares", v * v, -0.0))
        cases.append(("signed", rng.standard_normal(n).astype(np.float32) * np.float32(1e3), 0.0))
        cases.append(("exp weights", rng.exponential(1.0, n).astype(np.float32), 0.0))
    n = 2048
    cases.append(("zeros from -0", np.zeros(n, np.float32), -0.0))
    cases.append(("negative zeros from -0", np.full(n, -0.0, np.float32), -0.0))
    cases.append(("zeros from +0", np.zeros(n, np.float32), 0.0))
    cases.append(("ties", np.float32(2.0 ** -24) * rng.integers(0, 4, n).astype(np.float32) + np.float32(1.0), 0.0))
    sub = rng.integers(1, 1 << 23, n, dtype=np.uint32).view(np.float32)
    cases.append(("subnormals", sub, -0.0))
    big = np.full(n, 3e37, np.float32)
    cases.append(("overflow to inf", big, 0.0))
    cases.append(("inf and -inf", np.float32([1.0, np.inf, 2.0, -np.inf, 3.0] * 10), 0.0))
    with_nan = rng.standard_normal(n).astype(np.float32) ** 2
    with_nan[1500] = np.nan
    cases.append(("a NaN", with_nan, -0.0))
    cancel = rng.standard_normal(n).astype(np.float32)
    cancel = np.concatenate([cancel, -cancel[::-1]])
    cases.append(("cancellation", cancel, 0.0))
    cases.append(("init 1e30", rng.standard_normal(3000).astype(np.float32), 1e30))
    return cases


def test_device_ordered_sum_is_the_sequential_fold(ctx):
    # the RMSNorm sum of squares (and any float sum the kernels must keep in
    # element order) against a sequential float32 fold, bit for bit, NaN
    # aside (any NaN)
    for name, values, init in _ordered_sum_cases():
        got, rounds = _device_ordered_sum(ctx, values, init)
        want = _fold(values, init)
        if np.isnan(want):
            assert np.isnan(got), name
            continue
        assert got.view(np.uint32) == want.view(np.uint32), (name, values.size, got, want, rounds)


def _device_ordered_sum4(ctx, values, init):
    import ctypes
    L = R.lib()
    L.rh_ordered_sum4_device.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_float,
                                         ctypes.c_void_p, ctypes.c_void_p]
    v = np.ascontiguousarray(values, np.float32)
    out = np.zeros(1, np.float32)
    rounds = np.zeros(1, np.uint32)
    ctx.check(L.rh_ordered_sum4_device(ctx.handle, v.ctypes.data if v.size else None, v.size, float(init),
                                       out.ctypes.data, rounds.ctypes.data))
    return out[0], int(rounds[0])


def test_device_short_ordered_sum_is_the_sequential_fold(ctx):
    # the four-values-a-lane form (softmax denominators of up to 256 rows):
    # every length to 256, and the hostile cases cut to 256 values
    rng = np.random.default_rng(17)
    cases = [("exps", rng.exponential(1.0, n).astype(np.float32), 0.0) for n in range(0, 257)]
    cases += [(name, v[:256], init) for name, v, init in _ordered_sum_cases()]
    for _ in range(64):
        n = int(rng.integers(1, 257))
        cases.append(("softmax", np.exp(rng.standard_normal(n) * 4).astype(np.float32), 0.0))
    for name, values, init in cases:
        got, rounds = _device_ordered_sum4(ctx, values, init)
        want = _fold(values, init)
        if np.isnan(want):
            assert np.isnan(got), name
            continue
        assert got.view(np.uint32) == want.view(np.uint32), (name, values.size, got, want, rounds)


def test_device_ordered_sum_settles_in_few_rounds(ctx):
    # the speculative rounds, not the closing sequential chain, finish the
    # RMSNorm-shaped sums (squares of hidden states, 2048 and 4096 wide)
    rounds = []
    rng = np.random.default_rng(12)
    for n in (2048, 4096) * 16:
        v = (rng.standard_normal(n) * rng.uniform(0.01, 10)).astype(np.float32)
        got, r = _device_ordered_sum(ctx, v * v, -0.0)
        assert got.view(np.uint32) == _fold(v * v, -0.0).view(np.uint32)
        rounds.append(r)
    assert max(rounds) <= 6 and np.mean(rounds) <= 3.5, rounds


def test_greedy_pick_matches_the_cpu_rule(ctx):
    # filters.rs:37-43 / sampler.rs:75-87 on the device: NaN as -inf,
    # total_cmp order (-0.0 below +0.0), the last maximum wins; vocabularies
    # past one pass of loads (32768) included
    import ctypes
    L = R.lib()
    L.rh_greedy_pick_device.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                        ctypes.c_void_p]
    rng = np.random.default_rng(21)

    def pick(x):
        x = np.ascontiguousarray(x, np.float32)
        tok, fin = ctypes.c_uint32(), ctypes.c_uint32()
        ctx.check(L.rh_greedy_pick_device(ctx.handle, x.ctypes.data, x.size, ctypes.byref(tok), ctypes.byref(fin)))
        return tok.value, fin.value

    cases = []
    for n in (1, 2, 63, 1000, 32000, 32768, 32769, 50000, 128256):
        cases.append(rng.standard_normal(n).astype(np.float32))
    ties = np.zeros(32000, np.float32)
    ties[[5, 700, 31999]] = 3.0
    cases.append(ties)
    ties2 = np.full(32000, -1.0, np.float32)
    ties2[[10, 20000]] = 2.0
    cases.append(ties2)
    zeros = np.zeros(5000, np.float32)
    zeros[[100, 4000]] = -0.0
    cases.append(zeros)
    signed_zeros = np.full(4096, -0.0, np.float32)
    signed_zeros[17] = 0.0
    cases.append(signed_zeros)
    nan = rng.standard_normal(32000).astype(np.float32)
    nan[[3, 77, 31000]] = np.nan
    cases.append(nan)
    inf = rng.standard_normal(32000).astype(np.float32)
    inf[[9, 30000]] = np.inf
    cases.append(inf)
    for x in cases:
        tok, fin = pick(x)
        assert fin == 1
        assert tok == O.greedy(x), (x.size, tok, O.greedy(x))
    # no finite logit: the CPU path reports NoValidTokens
    for x in (np.full(100, np.nan, np.float32), np.float32([np.inf, -np.inf, np.nan])):
        tok, fin = pick(x)
        assert fin == 0
        with pytest.raises(O.DecoderError):
            O.greedy(x)


def test_device_division_is_rounded_to_nearest(ctx):
    rng = np.random.default_rng(5)
    a = rng.integers(0, 0x7F800000, 1 << 22, dtype=np.uint32).view(np.float32)
    b = rng.integers(0, 0x7F800000, 1 << 22, dtype=np.uint32).view(np.float32)
    a[::2] = -a[::2]
    x = np.concatenate([a, np.float32([1.0, -127.0, 0.0, 1.0, np.inf])])
    y = np.concatenate([b, np.float32([3.0, 0.37, 0.0, 0.0, np.inf])])
    with np.errstate(all="ignore"):
        want = x / y
    _assert_same(_device_math(ctx, 2, x, y), want, x)


@pytest.mark.parametrize("width,ffn", [(2048, 101), (256, 520)])
def test_gate_up_pair_with_rows_that_end_mid_group(ctx, width, ffn):
    # Q4_K gate/up whose row count is not a whole number of the unit
    # layout's 16-block groups (2048 wide: 8 blocks a row, rows in pairs; 256
    # wide: one block a row, rows in sixteens), with an F32 ffn_down so the
    # decoder accepts any FFN width: the last workgroup's up rows start
    # mid-group, and the one-token pair launch must still read the right
    # blocks (feed_forward.rs:45-79 through the CPU path)
    heads = width // 64
    cfg = dict(SMALL, embedding_length=width, feed_forward_length=ffn, head_count=heads,
               head_count_kv=heads // 2, block_count=1, context_length=64)
    model = synth.decoder_model(cfg, seed=31)
    rng = np.random.default_rng(32)
    for b in model["blocks"]:
        down = (0.05 * rng.standard_normal((width, ffn))).astype(np.float32)
        b["ffn_down"] = (0, down.reshape(-1).view(np.uint8), width, ffn)
    gpu, cpu = R.Decoder(ctx, model), O.Decoder(model, threads=8)
    tokens = rng.integers(0, cfg["vocab_size"], 9).astype(np.uint32)
    for start, chunk in ((0, tokens[:5]), (5, tokens[5:6]), (6, tokens[6:7]), (7, tokens[7:9])):
        g = gpu.forward_batch(chunk, start)
        c = cpu.forward_batch(chunk, start)
        assert same_bits(g, c), f"start {start}: max |diff| {diff(g, c)}"
    prompt = tokens[:6]
    assert np.array_equal(gpu.generate_greedy(prompt, 12), cpu.generate_greedy(prompt, 12))
    gpu.close()
    cpu.close()
