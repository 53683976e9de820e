"""Synthetic weights and activations for the benchmark workloads.

All generators draw from numpy's PCG64 with a fixed seed, so the bytes are
reproducible on any machine with the same numpy. f16 fields are produced by
IEEE round-to-nearest-even (numpy's float16 cast).

Block layouts follow the GGUF formats read by rusticide
(crates/rusticide-quantize/src/{q4_k,q6_k,i2_s}.rs):

* Q4_K, 144 B per 256 weights: d f16 @0, dmin f16 @2, scales[12] @4, qs[128] @16;
* Q6_K, 210 B per 256 weights: ql[128] @0, qh[64] @128, scales[16] i8 @192, d f16 @208;
* I2_S, 32 B per 128 weights: byte k holds weights k, k+32, k+64, k+96 at shifts
  6, 4, 2, 0 as code = weight + 1; the tensor ends with a 32-byte trailer whose
  first 4 bytes are the f32 scale.
"""

from __future__ import annotations

import numpy as np


def _rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def normal_f32(n: int, seed: int) -> np.ndarray:
    """x ~ N(0, 1) as f32."""
    return _rng(seed).standard_normal(n, dtype=np.float64).astype(np.float32)


def _f16_abs_normal(rng, n: int, scale: float) -> np.ndarray:
    return (np.abs(rng.standard_normal(n)) * scale).astype(np.float16)


def q4k_matrix(rows: int, cols: int, seed: int) -> np.ndarray:
    """Q4_K rows: d, dmin = f16(|N(0,1)| * 0.01); scale bytes and nibbles uniform."""
    assert cols % 256 == 0
    nblocks = rows * cols // 256
    rng = _rng(seed)
    blocks = rng.integers(0, 256, size=(nblocks, 144), dtype=np.uint8)
    d = _f16_abs_normal(rng, nblocks, 0.01).view(np.uint8).reshape(nblocks, 2)
    dmin = _f16_abs_normal(rng, nblocks, 0.01).view(np.uint8).reshape(nblocks, 2)
    blocks[:, 0:2] = d
    blocks[:, 2:4] = dmin
    return blocks.reshape(-1)


def q6k_matrix(rows: int, cols: int, seed: int) -> np.ndarray:
    """Q6_K rows: ql, qh uniform bits; scales int8 U{-32..31}; d = f16(|N| * 0.005)."""
    assert cols % 256 == 0
    nblocks = rows * cols // 256
    rng = _rng(seed)
    blocks = rng.integers(0, 256, size=(nblocks, 210), dtype=np.uint8)
    blocks[:, 192:208] = rng.integers(-32, 32, size=(nblocks, 16), dtype=np.int8).view(np.uint8)
    blocks[:, 208:210] = _f16_abs_normal(rng, nblocks, 0.005).view(np.uint8).reshape(nblocks, 2)
    return blocks.reshape(-1)


def i2s_codes(rows: int, cols: int, seed: int) -> np.ndarray:
    """Ternary weights iid from {-1, 0, +1} with p {0.3, 0.4, 0.3}, as codes w+1."""
    rng = _rng(seed)
    u = rng.random((rows, cols))
    return np.where(u < 0.3, 0, np.where(u < 0.7, 1, 2)).astype(np.uint8)


def pack_i2s(codes: np.ndarray, scale: float) -> np.ndarray:
    """Packs a [rows, cols] code matrix into I2_S blocks plus the 32-byte trailer."""
    rows, cols = codes.shape
    assert cols % 128 == 0
    c = codes.reshape(rows, cols // 128, 4, 32)  # [row, block, lane, k]
    packed = (c[:, :, 0] << 6) | (c[:, :, 1] << 4) | (c[:, :, 2] << 2) | c[:, :, 3]
    trailer = np.zeros(32, np.uint8)
    trailer[:4] = np.array([scale], np.float32).view(np.uint8)
    return np.concatenate([packed.astype(np.uint8).reshape(-1), trailer])


def i2s_matrix(rows: int, cols: int, seed: int, scale: float = 0.02) -> np.ndarray:
    return pack_i2s(i2s_codes(rows, cols, seed), scale)


def row_bytes(type_id: int, cols: int) -> int:
    return {12: cols // 256 * 144, 14: cols // 256 * 210, 36: cols // 128 * 32}[type_id]


def matrix(type_id: int, rows: int, cols: int, seed: int) -> np.ndarray:
    if type_id == 12:
        return q4k_matrix(rows, cols, seed)
    if type_id == 14:
        return q6k_matrix(rows, cols, seed)
    if type_id == 36:
        return i2s_matrix(rows, cols, seed)
    raise ValueError(type_id)


# ------------------------------------------------------- random-init decoders

def pack_q4k_scales(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """Packs 6-bit scales/mins [n, 8] into the 12 Q4_K scale bytes
    (the inverse of ggml get_scale_min_k4, quantize/src/q4_k.rs:17-25)."""
    sc = sc.astype(np.uint8)
    m = m.astype(np.uint8)
    out = np.zeros((sc.shape[0], 12), np.uint8)
    out[:, 0:4] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    out[:, 4:8] = (m[:, 0:4] & 63) | ((m[:, 4:8] >> 4) << 6)
    out[:, 8:12] = (sc[:, 4:8] & 0x0F) | ((m[:, 4:8] & 0x0F) << 4)
    return out


def q4k_centered(rows: int, cols: int, seed: int, sigma: float = 0.02) -> np.ndarray:
    """Q4_K rows whose weights are roughly N(0, sigma)-sized and centred:
    nibbles uniform 0..15, sub-block scales uniform 1..8, mins round(7.5*sc),
    d = dmin = f16(sigma / 20 * |N(1, 0.1)|)."""
    nblocks = rows * cols // 256
    rng = _rng(seed)
    blocks = rng.integers(0, 256, size=(nblocks, 144), dtype=np.uint8)
    sc = rng.integers(1, 9, size=(nblocks, 8), dtype=np.int32)
    m = np.rint(7.5 * sc).astype(np.int32)
    blocks[:, 4:16] = pack_q4k_scales(sc, m)
    d = (np.abs(rng.normal(1.0, 0.1, nblocks)) * (sigma / 20.0)).astype(np.float16)
    blocks[:, 0:2] = d.view(np.uint8).reshape(nblocks, 2)
    blocks[:, 2:4] = d.view(np.uint8).reshape(nblocks, 2)
    return blocks.reshape(-1)


def q6k_centered(rows: int, cols: int, seed: int, sigma: float = 0.02) -> np.ndarray:
    """Q6_K rows with N(0, sigma)-sized weights: 6-bit values uniform (centred
    by the -32 offset), int8 scales uniform +-(1..16), d = f16(sigma / 157)."""
    nblocks = rows * cols // 256
    rng = _rng(seed)
    blocks = rng.integers(0, 256, size=(nblocks, 210), dtype=np.uint8)
    mag = rng.integers(1, 17, size=(nblocks, 16), dtype=np.int32)
    sign = np.where(rng.random((nblocks, 16)) < 0.5, -1, 1)
    blocks[:, 192:208] = (mag * sign).astype(np.int8).view(np.uint8)
    d = (np.abs(rng.normal(1.0, 0.1, nblocks)) * (sigma / 157.0)).astype(np.float16)
    blocks[:, 208:210] = d.view(np.uint8).reshape(nblocks, 2)
    return blocks.reshape(-1)


TINYLLAMA = dict(embedding_length=2048, block_count=22, feed_forward_length=5632, head_count=32,
                 head_count_kv=4, head_dim=64, context_length=2048, vocab_size=32000,
                 rope_freq_base=10000.0, rms_norm_eps=1e-5)


def decoder_model(config: dict, seed: int) -> dict:
    """A random-init llama-family decoder in the Q4_K_M tensor mix: Q4_K for
    token_embd, attention and gate/up; Q6_K for the output and for ffn_down
    in even layers (Q4_K in odd ones); f32 norms 1 + 0.05*N(0, 1).

    Returns {"config": config, "token_embd", "output_norm", "output", "blocks"}
    where a matrix is (type_id, bytes, rows, cols)."""
    c = config
    width, kv = c["embedding_length"], c["head_count_kv"] * c["head_dim"]
    ffn, vocab = c["feed_forward_length"], c["vocab_size"]
    rng = _rng(seed)
    seeds = iter(rng.integers(0, 2 ** 31, size=16 + 16 * c["block_count"]).tolist())

    def mat(type_id, rows, cols):
        gen = q4k_centered if type_id == 12 else q6k_centered
        return (type_id, gen(rows, cols, next(seeds)), rows, cols)

    def norm():
        return (1.0 + 0.05 * _rng(next(seeds)).standard_normal(width)).astype(np.float32)

    blocks = []
    for layer in range(c["block_count"]):
        blocks.append({
            "attn_norm": norm(),
            "attn_q": mat(12, width, width), "attn_k": mat(12, kv, width), "attn_v": mat(12, kv, width),
            "attn_output": mat(12, width, width),
            "ffn_norm": norm(),
            "ffn_gate": mat(12, ffn, width), "ffn_up": mat(12, ffn, width),
            "ffn_down": mat(14 if layer % 2 == 0 else 12, width, ffn),
        })
    return {"config": dict(c), "token_embd": mat(12, vocab, width), "output_norm": norm(),
            "output": mat(14, vocab, width), "blocks": blocks}
