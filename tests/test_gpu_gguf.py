"""Decoders uploaded from GGUF files (rh_gguf_model_load) against the CPU
restatement of rusticide's decoder, and the loader's errors
(DecoderWeights::from_source, crates/rusticide-transformer/src/loader.rs:19-92;
Matrix::load, crates/rusticide-model/src/weights.rs:48-98).

The files come from rusticide_amd.gguf.decoder_gguf over the seeded
synthetic models of rusticide_amd.synth, so the same weights reach the
oracle directly and the device through the GGUF path.
"""

import struct

import numpy as np
import pytest

import oracle as O
import rusticide_amd as R
from rusticide_amd import gguf as G
from rusticide_amd import synth

pytestmark = pytest.mark.gpu

SMALL = dict(embedding_length=256, block_count=2, feed_forward_length=512, head_count=4, head_count_kv=2,
             head_dim=64, context_length=160, vocab_size=320, rope_freq_base=10000.0, rms_norm_eps=1e-5)


@pytest.fixture(scope="module")
def ctx():
    c = R.Context(0)
    yield c
    c.close()


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def load(ctx, data: bytes):
    f = G.GgufFile(data)
    return f, G.GgufModel(ctx, f)


@pytest.mark.parametrize("alignment,tied", [(32, False), (256, True)])
def test_gguf_decoder_matches_the_cpu_path(ctx, alignment, tied):
    model = synth.decoder_model(SMALL, seed=21)
    if tied:
        model["output"] = None  # output.weight absent: the output shares token_embd
    f, m = load(ctx, G.decoder_gguf(model, alignment=alignment))
    assert m.config == {**SMALL, "rms_norm_eps": m.config["rms_norm_eps"]}
    dec = m.decoder()
    cpu = O.Decoder(model, threads=8)
    tokens = np.random.default_rng(5).integers(0, SMALL["vocab_size"], 70).astype(np.uint32)
    g, c = dec.forward_batch(tokens[:64], 0), cpu.forward_batch(tokens[:64], 0)
    assert same_bits(g, c)
    want = cpu.generate_greedy(tokens, 48)
    got = dec.generate_greedy(tokens, 48)
    assert len(got) == 48 and np.array_equal(got, want), (got, want)
    dec.free()
    m.free()
    f.close()
    cpu.close()


def test_gguf_decoder_equals_the_decoder_built_from_host_arrays(ctx):
    model = synth.decoder_model(SMALL, seed=22)
    f, m = load(ctx, G.decoder_gguf(model))
    a, b = m.decoder(), R.Decoder(ctx, model)
    prompt = np.arange(40, dtype=np.uint32) * 7 % SMALL["vocab_size"]
    assert same_bits(a.forward_batch(prompt, 0), b.forward_batch(prompt, 0))
    for pos in range(40, 48):
        t = (pos * 13) % SMALL["vocab_size"]
        assert same_bits(a.forward(t, pos), b.forward(t, pos))
    b.free()
    m.free()  # frees its decoder first
    f.close()


def writer_for(model, drop=(), replace=None, extra=()):
    """decoder_gguf's tensors with some dropped, replaced or added."""
    data = G.decoder_gguf(model)
    f = G.GgufFile(data)
    w = G.Writer()
    w.kv("general.architecture", G.STRING, "llama")
    for key in ("context_length", "embedding_length", "block_count", "feed_forward_length", "attention.head_count",
                "attention.head_count_kv"):
        w.kv(f"llama.{key}", G.UINT32, f.meta_uint(f"llama.{key}"))
    replace = replace or {}
    for name in f.tensor_names():
        if name in drop:
            continue
        if name in replace:
            shape, t, raw = replace[name]
        else:
            shape, t, _ = f.tensor_info(name)
            raw = f.tensor_bytes(name)
        w.tensor(name, shape, t, raw)
    for name, shape, t, raw in extra:
        w.tensor(name, shape, t, raw)
    f.close()
    return w.build()


def load_error(ctx, data: bytes) -> R.RusticideError:
    f = G.GgufFile(data)
    with pytest.raises(R.RusticideError) as e:
        G.GgufModel(ctx, f)
    f.close()
    return e.value


def test_loader_errors_mirror_model_error(ctx):
    model = synth.decoder_model(SMALL, seed=23)
    e = load_error(ctx, writer_for(model, drop=("blk.1.attn_k.weight",)))
    assert e.kind == "MISSING_TENSOR" and "blk.1.attn_k.weight" in str(e)
    e = load_error(ctx, writer_for(model, drop=("output_norm.weight",)))
    assert e.kind == "MISSING_TENSOR" and "output_norm.weight" in str(e)
    # a mis-shaped matrix (rows and cols swapped) and norm
    t, raw, rows, cols = model["blocks"][0]["ffn_gate"]
    e = load_error(ctx, writer_for(model, replace={"blk.0.ffn_gate.weight": ([cols, rows], t, raw.tobytes())}))
    assert e.kind == "SHAPE_MISMATCH" and "blk.0.ffn_gate.weight" in str(e)
    e = load_error(ctx, writer_for(model, replace={"blk.0.ffn_norm.weight": ([255], 0, bytes(4 * 255))}))
    assert e.kind == "SHAPE_MISMATCH"
    # a format no kernel here reads (Q8_0: 34 bytes per 32 weights)
    n = SMALL["embedding_length"] * SMALL["embedding_length"] // 32
    e = load_error(ctx, writer_for(model, replace={"blk.0.attn_output.weight": ([256, 256], 8, bytes(34 * n))}))
    assert e.kind == "MISSING_KERNEL"
    # an attention bias: this decoder adds none, so the file is refused
    e = load_error(ctx, writer_for(model, extra=(("blk.0.attn_q.bias", [256], 0, bytes(4 * 256)),)))
    assert e.kind == "MISSING_KERNEL" and "blk.0.attn_q.bias" in str(e)
    # an I2_S matrix whose scale is not finite (weights.rs:190-202)
    body = bytes(256 * 256 // 4)
    bad = body + struct.pack("<f", float("nan")) + bytes(28)
    e = load_error(ctx, writer_for(model, replace={"blk.0.attn_q.weight": ([256, 256], 36, bad)}))
    assert e.kind == "INVALID_TENSOR"


def test_dense_and_ternary_tensors_load(ctx):
    # F16 norms and an F32 / I2_S projection go through the same loader
    model = synth.decoder_model(SMALL, seed=24)
    norm = model["blocks"][0]["attn_norm"].astype(np.float16)
    wq = (np.random.default_rng(9).standard_normal((256, 256)) * 0.02).astype(np.float32)
    i2s = synth.i2s_matrix(256, 256, seed=25, scale=0.03)
    data = writer_for(model, replace={"blk.0.attn_norm.weight": ([256], 1, norm.tobytes()),
                                      "blk.0.attn_q.weight": ([256, 256], 0, wq.tobytes()),
                                      "blk.1.attn_output.weight": ([256, 256], 36, i2s.tobytes())})
    f, m = load(ctx, data)
    want = dict(model, blocks=[dict(b) for b in model["blocks"]])
    want["blocks"][0]["attn_norm"] = norm.astype(np.float32)
    want["blocks"][0]["attn_q"] = (0, wq.reshape(-1).view(np.uint8), 256, 256)
    want["blocks"][1]["attn_output"] = (36, i2s, 256, 256)
    cpu = O.Decoder(want, threads=8)
    dec = m.decoder()
    prompt = np.arange(20, dtype=np.uint32) * 11 % SMALL["vocab_size"]
    assert same_bits(dec.forward_batch(prompt, 0), cpu.forward_batch(prompt, 0))
    assert np.array_equal(dec.generate_greedy(prompt, 16), cpu.generate_greedy(prompt, 16))
    m.free()
    f.close()
    cpu.close()


def test_tinyllama_shaped_gguf_greedy_decode(ctx):
    # the 22-layer Q4_K_M TinyLlama-shaped model through a GGUF file: the
    # tokens equal those of the decoder built from the same host arrays
    # (itself pinned to the CPU path at this size)
    model = synth.decoder_model(synth.TINYLLAMA, seed=2026)
    data = G.decoder_gguf(model)
    f, m = load(ctx, data)
    del data
    prompt = np.random.default_rng(7).integers(0, 32000, 64).astype(np.uint32)
    got = m.decoder().generate_greedy(prompt, 32)
    m.free()
    f.close()
    ref = R.Decoder(ctx, model)
    want = ref.generate_greedy(prompt, 32)
    ref.free()
    assert len(got) == 32 and np.array_equal(got, want)


def test_q4_k_m_mix_with_q6_k_attn_v(ctx):
    # llama.cpp's Q4_K_M keeps attn_v (and some ffn_down) in Q6_K: the Q/K/V
    # launches then mix formats, in the fused one-token path and in the
    # batched one (its Q8_K norm and split GEMMs)
    model = synth.decoder_model(SMALL, seed=31)
    for i, b in enumerate(model["blocks"]):
        if i % 2 == 0:
            _, _, rows, cols = b["attn_v"]
            b["attn_v"] = (14, synth.q6k_centered(rows, cols, 900 + i), rows, cols)
    f, m = load(ctx, G.decoder_gguf(model))
    assert f.tensor_info("blk.0.attn_v.weight")[1] == 14 and f.tensor_info("blk.1.attn_v.weight")[1] == 12
    dec, cpu = m.decoder(), O.Decoder(model, threads=8)
    prompt = np.random.default_rng(9).integers(0, SMALL["vocab_size"], 70).astype(np.uint32)
    assert same_bits(dec.forward_batch(prompt[:64], 0), cpu.forward_batch(prompt[:64], 0))
    assert np.array_equal(dec.generate_greedy(prompt, 24), cpu.generate_greedy(prompt, 24))
    m.free()
    f.close()
    cpu.close()
