"""ctypes binding of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: a CPU restatement of rusticide's quantized
matrix-product arithmetic, used by ``tests/`` as the checker, by
``__graft_entry__.smoke()`` and by ``bench.py``'s ``cpu_baseline`` leg. The
product package (``rusticide_amd``) never imports it.

Each function cites the reference file it restates; see ``rh_oracle.c``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

SUPER_BLOCK = 1  # Q8Kind::SuperBlock (ggml Q8_K)
ROW = 2  # Q8Kind::Row (bitnet.cpp I8_S)

DENSE, BLOCKS, TERNARY = 0, 1, 2
Q4_K, Q6_K, I2_S = 12, 14, 36


def build() -> str:
    """Compile liboracle.so from rh_oracle.c with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


class _Job(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_uint32),
        ("type_id", ctypes.c_uint32),
        ("data", ctypes.c_void_p),
        ("data_len", ctypes.c_size_t),
        ("width", ctypes.c_size_t),
        ("scale", ctypes.c_float),
        ("out", ctypes.c_void_p),
        ("out_len", ctypes.c_size_t),
    ]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        S = ctypes.c_size_t
        L.orc_block_format.argtypes = [ctypes.c_uint32, P, P, P]
        L.orc_byte_len.argtypes = [ctypes.c_uint32, S]
        L.orc_byte_len.restype = S
        L.orc_row_bytes.argtypes = [ctypes.c_uint32, S]
        L.orc_row_bytes.restype = S
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_dequantize_row.argtypes = [ctypes.c_uint32, P, S, P, S]
        L.orc_i2s_scale.argtypes = [P, S, P]
        L.orc_pseudo_random_bytes.argtypes = [P, S, ctypes.c_uint32]
        L.orc_synthetic_blocks.argtypes = [ctypes.c_uint32, S, ctypes.c_uint32, P]
        L.orc_pseudo_random_values.argtypes = [P, S, ctypes.c_uint32]
        L.orc_bench_activations.argtypes = [P, S, ctypes.c_uint32]
        L.orc_quantize.argtypes = [ctypes.c_int, P, S, P, P, P]
        L.orc_quantize.restype = S
        L.orc_q8_dequantize.argtypes = [ctypes.c_int, P, P, S, P]
        for name in ("orc_q4k_dot", "orc_q6k_dot"):
            getattr(L, name).argtypes = [P, S, P, P, P, S]
            getattr(L, name).restype = ctypes.c_float
        L.orc_ternary_dot.argtypes = [P, S, P, P, S]
        L.orc_avx2_available.restype = ctypes.c_int
        L.orc_avx2_prepare.argtypes = [ctypes.c_uint32, P, S, S]
        L.orc_avx2_prepare.restype = P
        L.orc_avx2_free.argtypes = [P]
        L.orc_avx2_matvec.argtypes = [P, P, S, P, S, ctypes.c_int]
        L.orc_avx2_matvec.restype = ctypes.c_int
        L.orc_ternary_dot.restype = ctypes.c_int32
        L.orc_ternary_product.argtypes = [P, S, P, P, P, S, ctypes.c_float]
        L.orc_ternary_product.restype = ctypes.c_float
        L.orc_dot_f32.argtypes = [P, S, P, S]
        L.orc_dot_f32.restype = ctypes.c_float
        L.orc_dequant_dot.argtypes = [ctypes.c_uint32, P, S, P, S]
        L.orc_dequant_dot.restype = ctypes.c_float
        L.orc_matmul_batch.argtypes = [P, S, S, P, S, ctypes.c_int]
        L.orc_ternary_dot_matrix_i32.argtypes = [P, S, S, P, S, S, P, S]
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(np.frombuffer(bytes(a), np.uint8) if isinstance(a, (bytes, bytearray)) else a, dtype=np.uint8)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- formats

def block_format(type_id: int):
    bs, bb, tb = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
    ok = lib().orc_block_format(type_id, ctypes.byref(bs), ctypes.byref(bb), ctypes.byref(tb))
    return (bs.value, bb.value, tb.value) if ok else None


def byte_len(type_id: int, numel: int):
    v = lib().orc_byte_len(type_id, numel)
    return None if v == (1 << 64) - 1 else v


def row_bytes(type_id: int, cols: int):
    v = lib().orc_row_bytes(type_id, cols)
    return None if v == (1 << 64) - 1 else v


def f16_to_f32(bits: int) -> float:
    return lib().orc_f16_to_f32(bits)


def f32_to_f16(value: float) -> int:
    return lib().orc_f32_to_f16(value)


def dequantize_row(type_id: int, row) -> np.ndarray:
    row = _u8(row)
    bs, bb, _ = block_format(type_id)
    out = np.zeros(len(row) // bb * bs, np.float32)
    lib().orc_dequantize_row(type_id, _p(row), len(row), _p(out), len(out))
    return out


# ------------------------------------------------------------- generators

def pseudo_random_bytes(n: int, seed: int) -> np.ndarray:
    out = np.zeros(n, np.uint8)
    lib().orc_pseudo_random_bytes(_p(out), n, seed)
    return out


def synthetic_blocks(type_id: int, blocks: int, seed: int) -> np.ndarray:
    _, bb, _ = block_format(type_id)
    out = np.zeros(blocks * bb, np.uint8)
    lib().orc_synthetic_blocks(type_id, blocks, seed, _p(out))
    return out


def pseudo_random_values(n: int, seed: int) -> np.ndarray:
    out = np.zeros(n, np.float32)
    lib().orc_pseudo_random_values(_p(out), n, seed)
    return out


def bench_activations(n: int, seed: int) -> np.ndarray:
    out = np.zeros(n, np.float32)
    lib().orc_bench_activations(_p(out), n, seed)
    return out


# ------------------------------------------------------------- quantizers

class Q8Input:
    """Mirror of Q8Input (crates/rusticide-kernels/src/q8_input.rs:13-23)."""

    def __init__(self, kind, quants, scales, sums):
        self.kind, self.quants, self.scales, self.sums = kind, quants, scales, sums

    def __len__(self):
        return len(self.quants)

    def dequantize(self) -> np.ndarray:
        out = np.zeros(len(self.quants), np.float32)
        lib().orc_q8_dequantize(self.kind, _p(self.quants), _p(self.scales), len(self.scales), _p(out))
        return out


def quantize(x, kind: int) -> Q8Input:
    x = _f32(x)
    nb = len(x) // 32 + 1
    quants = np.zeros(nb * 32, np.int8)
    scales = np.zeros(nb, np.float32)
    sums = np.zeros(nb, np.int32)
    n = lib().orc_quantize(kind, _p(x), len(x), _p(quants), _p(scales), _p(sums))
    return Q8Input(kind, quants[: n * 32].copy(), scales[:n].copy(), sums[:n].copy())


# ------------------------------------------------------------------- dots

def dot_row(type_id: int, row, q: Q8Input) -> float:
    row = _u8(row)
    fn = {Q4_K: lib().orc_q4k_dot, Q6_K: lib().orc_q6k_dot}[type_id]
    return fn(_p(row), len(row), _p(q.quants), _p(q.scales), _p(q.sums), len(q.scales))


def ternary_dot(row, q: Q8Input) -> int:
    row = _u8(row)
    return lib().orc_ternary_dot(_p(row), len(row), _p(q.quants), _p(q.sums), len(q.scales))


def ternary_product(row, q: Q8Input, scale: float) -> float:
    row = _u8(row)
    return lib().orc_ternary_product(_p(row), len(row), _p(q.quants), _p(q.scales), _p(q.sums),
                                     len(q.scales), scale)


def dot_f32(lhs, rhs) -> float:
    lhs, rhs = _f32(lhs), _f32(rhs)
    return lib().orc_dot_f32(_p(lhs), len(lhs), _p(rhs), len(rhs))


def dequant_dot(type_id: int, row, x) -> float:
    row, x = _u8(row), _f32(x)
    return lib().orc_dequant_dot(type_id, _p(row), len(row), _p(x), len(x))


# ------------------------------------------------------------ matmul_batch

class Weights:
    """Mirror of Weights (crates/rusticide-kernels/src/matmul.rs:28-46)."""

    def __init__(self, kind, data, width, type_id=0, scale=0.0):
        self.kind, self.width, self.type_id, self.scale = kind, width, type_id, scale
        self.data = _f32(data) if kind == DENSE else _u8(data)

    @classmethod
    def dense(cls, data, cols):
        return cls(DENSE, data, cols)

    @classmethod
    def blocks(cls, type_id, data, row_bytes_):
        return cls(BLOCKS, data, row_bytes_, type_id=type_id)

    @classmethod
    def ternary(cls, data, row_bytes_, scale):
        return cls(TERNARY, data, row_bytes_, scale=scale)

    def rows(self) -> int:
        return len(self.data) // self.width if self.width else 0


def matmul_batch(inputs, tokens: int, jobs, threads: int = 1) -> None:
    """matmul.rs:229-248: ``jobs`` is a list of (Weights, out ndarray f32)."""
    inputs = _f32(inputs)
    arr = (_Job * max(1, len(jobs)))()
    for i, (w, out) in enumerate(jobs):
        assert out.dtype == np.float32 and out.flags.c_contiguous
        arr[i] = _Job(w.kind, w.type_id, _p(w.data), len(w.data), w.width, w.scale,
                      _p(out), len(out))
    lib().orc_matmul_batch(_p(inputs), len(inputs), tokens, arr, len(jobs), threads)


def matvec_batch(x, jobs, threads: int = 1) -> None:
    matmul_batch(x, 1, jobs, threads)


class Avx2Matrix:
    """A Q4_K / Q6_K matrix repacked into the reference's eight-row avx2 units
    (rh_avx2.c): the CPU baseline's timing of rusticide's x86 kernels."""

    def __init__(self, type_id: int, data, rows: int, row_bytes: int):
        self._data = np.ascontiguousarray(data, np.uint8)
        self.rows = rows
        self.h = lib().orc_avx2_prepare(type_id, self._data.ctypes.data, rows, row_bytes)
        if not self.h:
            raise ValueError("the avx2 units need avx2+fma, Q4_K/Q6_K and rows a multiple of 8")

    @staticmethod
    def available() -> bool:
        return bool(lib().orc_avx2_available())

    def matvec(self, x, out, threads: int = 1) -> bool:
        """out[r] = row r . x; False when x quantizes to the quant -128 (out untouched)."""
        x = np.ascontiguousarray(x, np.float32)
        return bool(lib().orc_avx2_matvec(self.h, x.ctypes.data, x.size, out.ctypes.data, out.size, threads))

    def close(self) -> None:
        if self.h:
            lib().orc_avx2_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def ternary_dot_matrix_i32(data, row_bytes_: int, inputs, tokens: int) -> np.ndarray:
    data, inputs = _u8(data), _f32(inputs)
    rows = len(data) // row_bytes_
    out = np.zeros(rows * tokens, np.int32)
    lib().orc_ternary_dot_matrix_i32(_p(data), len(data), row_bytes_, _p(inputs), len(inputs),
                                     tokens, _p(out), len(out))
    return out


# ------------------------------------------------------------------ decoder


class _Matrix(ctypes.Structure):
    _fields_ = [("type_id", ctypes.c_uint32), ("data", ctypes.c_void_p), ("rows", ctypes.c_size_t),
                ("cols", ctypes.c_size_t)]


class _Block(ctypes.Structure):
    _fields_ = [("attn_norm", ctypes.c_void_p), ("attn_q", _Matrix), ("attn_k", _Matrix), ("attn_v", _Matrix),
                ("attn_output", _Matrix), ("ffn_norm", ctypes.c_void_p), ("ffn_gate", _Matrix),
                ("ffn_up", _Matrix), ("ffn_down", _Matrix)]


class _DecoderWeights(ctypes.Structure):
    _fields_ = [("token_embd", _Matrix), ("output_norm", ctypes.c_void_p), ("output", ctypes.POINTER(_Matrix)),
                ("blocks", ctypes.POINTER(_Block))]


class _DecoderConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_size_t) for n in ("embedding_length", "block_count", "feed_forward_length",
                                               "head_count", "head_count_kv", "head_dim", "context_length",
                                               "vocab_size")] + [("rope_freq_base", ctypes.c_float),
                                                                 ("rms_norm_eps", ctypes.c_float)]


DECODER_ERRORS = {1: "NO_TOKENS", 2: "CONTEXT_FULL", 3: "TOKEN_RANGE", 4: "CACHE_POSITION",
                  5: "NO_VALID_TOKENS", 6: "NO_MEMORY"}


class DecoderError(RuntimeError):
    def __init__(self, code: int):
        self.kind = DECODER_ERRORS.get(code, str(code))
        super().__init__(self.kind)


def _dec_lib():
    L = lib()
    if not hasattr(L, "_dec_ready"):
        P, S = ctypes.c_void_p, ctypes.c_size_t
        L.orc_decoder_new.argtypes = [ctypes.POINTER(_DecoderConfig), ctypes.POINTER(_DecoderWeights), ctypes.c_int]
        L.orc_decoder_new.restype = P
        L.orc_decoder_free.argtypes = [P]
        L.orc_decoder_reset.argtypes = [P]
        L.orc_decoder_forward_batch.argtypes = [P, P, S, S, P]
        L.orc_greedy.argtypes = [P, S, P]
        L.orc_generate_greedy.argtypes = [P, P, S, S, P, P]
        L.orc_normalize.argtypes = [P, P, S, ctypes.c_float, P]
        L.orc_softmax.argtypes = [P, S]
        L.orc_rope_adjacent.argtypes = [P, S, S, ctypes.c_float, S]
        L.orc_rope_table.argtypes = [S, S, ctypes.c_float, P, P]
        L.orc_expf_array.argtypes = [P, P, S]
        L.orc_silu_array.argtypes = [P, P, S]
        L.orc_dot_rows.argtypes = [P, S, P, S, S, S, ctypes.c_float, P]
        L.orc_mix_rows.argtypes = [P, S, P, S, S, S, P, S]
        L._dec_ready = True
    return L


def _mat(m, keep):
    type_id, data, rows, cols = m
    arr = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
    keep.append(arr)
    return _Matrix(type_id, arr.ctypes.data, rows, cols)


class Decoder:
    """The reference decoder's forward pass on the CPU (rh_decoder.c) over a
    model dict from rusticide_amd.synth.decoder_model."""

    def __init__(self, model: dict, threads: int = 8):
        L = _dec_lib()
        c = model["config"]
        self.config = c
        self._keep = []
        cfg = _DecoderConfig(*[c[k] for k in ("embedding_length", "block_count", "feed_forward_length",
                                              "head_count", "head_count_kv", "head_dim", "context_length",
                                              "vocab_size")], c["rope_freq_base"], c["rms_norm_eps"])
        blocks = (_Block * len(model["blocks"]))()
        for i, b in enumerate(model["blocks"]):
            an = np.ascontiguousarray(b["attn_norm"], np.float32)
            fn = np.ascontiguousarray(b["ffn_norm"], np.float32)
            self._keep += [an, fn]
            blocks[i] = _Block(an.ctypes.data, _mat(b["attn_q"], self._keep), _mat(b["attn_k"], self._keep),
                               _mat(b["attn_v"], self._keep), _mat(b["attn_output"], self._keep), fn.ctypes.data,
                               _mat(b["ffn_gate"], self._keep), _mat(b["ffn_up"], self._keep),
                               _mat(b["ffn_down"], self._keep))
        on = np.ascontiguousarray(model["output_norm"], np.float32)
        self._keep.append(on)
        out = None
        if model.get("output") is not None:
            out = _Matrix()
            out = _mat(model["output"], self._keep)
            self._out = out
        w = _DecoderWeights(_mat(model["token_embd"], self._keep), on.ctypes.data,
                            ctypes.pointer(out) if out is not None else None, blocks)
        self._blocks, self._w, self._cfg = blocks, w, cfg
        self.handle = L.orc_decoder_new(ctypes.byref(cfg), ctypes.byref(w), threads)
        if not self.handle:
            raise MemoryError("orc_decoder_new")

    def forward_batch(self, tokens, start: int) -> np.ndarray:
        t = np.ascontiguousarray(tokens, np.uint32)
        logits = np.zeros(self.config["vocab_size"], np.float32)
        err = _dec_lib().orc_decoder_forward_batch(self.handle, t.ctypes.data, len(t), start, logits.ctypes.data)
        if err:
            raise DecoderError(err)
        return logits

    def forward(self, token: int, position: int) -> np.ndarray:
        return self.forward_batch([token], position)

    def reset(self) -> None:
        _dec_lib().orc_decoder_reset(self.handle)

    def generate_greedy(self, prompt, max_tokens: int) -> np.ndarray:
        p = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(max(1, max_tokens), np.uint32)
        n = ctypes.c_size_t()
        err = _dec_lib().orc_generate_greedy(self.handle, p.ctypes.data, len(p), max_tokens, out.ctypes.data,
                                             ctypes.byref(n))
        if err:
            raise DecoderError(err)
        return out[: n.value]

    def close(self) -> None:
        if self.handle:
            _dec_lib().orc_decoder_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def greedy(logits) -> int:
    x = _f32(logits)
    tok = ctypes.c_uint32()
    err = _dec_lib().orc_greedy(x.ctypes.data, len(x), ctypes.byref(tok))
    if err:
        raise DecoderError(err)
    return tok.value


def normalize(x, weight, eps: float) -> np.ndarray:
    x, w = _f32(x), _f32(weight)
    out = np.zeros_like(x)
    _dec_lib().orc_normalize(x.ctypes.data, w.ctypes.data, len(x), eps, out.ctypes.data)
    return out


def softmax(row) -> np.ndarray:
    r = _f32(row).copy()
    _dec_lib().orc_softmax(r.ctypes.data, len(r))
    return r


def rope_adjacent(row, position: int, theta: float, dim_pairs: int) -> np.ndarray:
    r = _f32(row).copy()
    _dec_lib().orc_rope_adjacent(r.ctypes.data, len(r), position, theta, dim_pairs)
    return r


def rope_table(positions: int, columns: int, theta: float):
    pairs = columns // 2
    c = np.zeros(positions * pairs, np.float32)
    s = np.zeros(positions * pairs, np.float32)
    _dec_lib().orc_rope_table(positions, columns, theta, c.ctypes.data, s.ctypes.data)
    return c, s


def silu(x) -> np.ndarray:
    """portable/elementwise.rs:6-9 over an array."""
    x = _f32(x)
    y = np.zeros_like(x)
    _dec_lib().orc_silu_array(x.ctypes.data, y.ctypes.data, len(x))
    return y


def dot_rows(query, rows, row_stride: int, offset: int, scale: float, n_out: int) -> np.ndarray:
    """float.rs:38-58 over the whole row_stride-wide rows of `rows`, at most n_out of them."""
    q, r = _f32(query), _f32(rows)
    nrows = min(n_out, len(r) // max(row_stride, 1))
    out = np.zeros(n_out, np.float32)
    _dec_lib().orc_dot_rows(q.ctypes.data, len(q), r.ctypes.data, nrows, row_stride, offset, scale, out.ctypes.data)
    return out


def mix_rows(weights, rows, row_stride: int, offset: int, out) -> np.ndarray:
    """float.rs:60-68 into a copy of `out`."""
    w, r = _f32(weights), _f32(rows)
    o = _f32(out).copy()
    nrows = len(r) // max(row_stride, 1)
    _dec_lib().orc_mix_rows(w.ctypes.data, len(w), r.ctypes.data, nrows, row_stride, offset, o.ctypes.data, len(o))
    return o


def expf(x) -> np.ndarray:
    """libm's expf over an array (the function rusticide's f32::exp calls)."""
    x = _f32(x)
    y = np.empty_like(x)
    _dec_lib().orc_expf_array(x.ctypes.data, y.ctypes.data, len(x))
    return y
