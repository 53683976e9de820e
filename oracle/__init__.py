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
    """Mirror of Q8Input (crates/rusticide-kernels/src/q8_input.rs:66-73)."""

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


def ternary_dot_matrix_i32(data, row_bytes_: int, inputs, tokens: int) -> np.ndarray:
    data, inputs = _u8(data), _f32(inputs)
    rows = len(data) // row_bytes_
    out = np.zeros(rows * tokens, np.int32)
    lib().orc_ternary_dot_matrix_i32(_p(data), len(data), row_bytes_, _p(inputs), len(inputs),
                                     tokens, _p(out), len(out))
    return out
