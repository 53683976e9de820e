"""rusticide_amd -- MI355X (gfx950) quantized matrix products for rusticide.

A thin Python mirror of rusticide's kernel facade over the C ABI of
``include/rusticide_hip.h`` (loaded with ctypes from the in-tree
``librusticide_hip.so``):

* ``Matrix.load``   -- ``Matrix::load_on`` (crates/rusticide-model/src/weights.rs:53-98):
  native GGUF blocks uploaded to HBM once;
* ``matmul_batch`` / ``matvec_batch`` -- crates/rusticide-kernels/src/matmul.rs:218-248;
* ``quantize``      -- ``Q8Input::quantize`` (q8_input.rs:52-58) on the device.

There is no CPU fallback: if the library is missing, or no gfx950 device is
present, calls raise ``RusticideError``.
"""

from __future__ import annotations

import ctypes
import os
import weakref

import numpy as np

__all__ = [
    "RusticideError", "Context", "Matrix", "Job", "matmul_batch", "matvec_batch",
    "Q4_K", "Q6_K", "I2_S", "F32", "F16", "SUPER_BLOCK", "ROW", "library_path",
]

F32, F16, Q4_K, Q6_K, I2_S = 0, 1, 12, 14, 36
SUPER_BLOCK, ROW = 1, 2

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "librusticide_hip.so")

STATUS = {
    0: "OK", 1: "INVALID_ARGUMENT", 2: "MISSING_KERNEL", 3: "INVALID_TENSOR",
    4: "SHAPE_MISMATCH", 5: "INVALID_CONFIG", 6: "DEVICE", 7: "OUT_OF_MEMORY", 8: "NO_DEVICE",
}


class RusticideError(RuntimeError):
    def __init__(self, status: int, message: str = ""):
        self.status = status
        self.kind = STATUS.get(status, str(status))
        super().__init__(f"{self.kind}: {message}" if message else self.kind)


def library_path() -> str:
    return _LIB


class _Job(ctypes.Structure):
    _fields_ = [("weights", ctypes.c_void_p), ("out", ctypes.c_void_p), ("out_len", ctypes.c_size_t)]


_lib = None


def lib() -> ctypes.CDLL:
    """The loaded C ABI; raises if the HIP library was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            raise RusticideError(6, f"{_LIB} is missing: run __graft_entry__.build()")
        L = ctypes.CDLL(_LIB)
        P, S, St = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        L.rh_init.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_void_p)]
        L.rh_init.restype = St
        L.rh_destroy.argtypes = [P]
        L.rh_last_error.argtypes = [P]
        L.rh_last_error.restype = ctypes.c_char_p
        L.rh_adapter_name.restype = ctypes.c_char_p
        L.rh_stream.argtypes = [P]
        L.rh_stream.restype = P
        L.rh_matrix_load.argtypes = [P, ctypes.c_uint32, P, S, S, S, ctypes.POINTER(ctypes.c_void_p)]
        L.rh_matrix_load.restype = St
        L.rh_matrix_free.argtypes = [P]
        for n in ("rh_matrix_rows", "rh_matrix_cols", "rh_matrix_device_bytes"):
            getattr(L, n).argtypes = [P]
            getattr(L, n).restype = S
        L.rh_matrix_type.argtypes = [P]
        L.rh_matrix_type.restype = ctypes.c_uint32
        L.rh_matrix_ternary_scale.argtypes = [P]
        L.rh_matrix_ternary_scale.restype = ctypes.c_float
        L.rh_matrix_copy_row.argtypes = [P, P, S, P, S, ctypes.POINTER(ctypes.c_int)]
        L.rh_matrix_copy_row.restype = St
        L.rh_matmul_batch.argtypes = [P, P, S, S, P, S]
        L.rh_matmul_batch.restype = St
        L.rh_matvec_batch.argtypes = [P, P, S, P, S]
        L.rh_matvec_batch.restype = St
        L.rh_matmul_batch_device.argtypes = [P, P, S, S, P, S, P]
        L.rh_matmul_batch_device.restype = St
        L.rh_quantize.argtypes = [P, ctypes.c_int, P, S, P, P, P, ctypes.POINTER(ctypes.c_size_t)]
        L.rh_quantize.restype = St
        L.rh_ternary_dot_i32.argtypes = [P, P, P, S, S, P, S]
        L.rh_ternary_dot_i32.restype = St
        L.rh_q8_new.argtypes = [P, ctypes.POINTER(ctypes.c_void_p)]
        L.rh_q8_new.restype = St
        L.rh_q8_free.argtypes = [P]
        L.rh_q8_quantize_device.argtypes = [P, P, ctypes.c_int, P, S, S, P]
        L.rh_q8_quantize_device.restype = St
        L.rh_dot_matrix_device.argtypes = [P, P, P, P, S, P]
        L.rh_dot_matrix_device.restype = St
        L.rh_gemm_min_tokens.restype = S
        L.rh_set_gemm_min_tokens.argtypes = [S]
        L.rh_matmul_batch_device_noalloc.argtypes = [P, P, S, S, P, S, P]
        L.rh_matmul_batch_device_noalloc.restype = St
        L.rh_matmul_batch_device_repeat.argtypes = [P, P, S, S, P, S, P, S, S, P]
        L.rh_matmul_batch_device_repeat.restype = St
        L.rh_reload_tuning.argtypes = []
        L.rh_reload_tuning.restype = None
        L.rh_hold_device.argtypes = [P, ctypes.c_uint32, P]
        L.rh_hold_device.restype = St
        _lib = L
    return _lib


def _ptr(a) -> int:
    if a is None:
        return 0
    if isinstance(a, np.ndarray):
        return a.ctypes.data
    return int(a.data_ptr())  # torch tensor on the device


class Context:
    """An open gfx950 device with its own stream (rh_init / rh_destroy)."""

    def __init__(self, device: int = 0):
        h = ctypes.c_void_p()
        st = lib().rh_init(device, ctypes.byref(h))
        if st != 0:
            raise RusticideError(st, f"rh_init({device})")
        self.handle = h
        self._children = weakref.WeakSet()  # matrices, activations, decoders

    def check(self, status: int) -> None:
        if status != 0:
            raise RusticideError(status, lib().rh_last_error(self.handle).decode())

    @property
    def stream(self) -> int:
        return lib().rh_stream(self.handle)

    def close(self) -> None:
        # everything made on this context goes first
        for child in list(self._children):
            child.free()
        if self.handle:
            lib().rh_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---------------------------------------------------------- test hooks
    def quantize(self, x, kind: int):
        """Device Q8Input::quantize of one row: (quants, scales, sums)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        nb = len(x) // 32 + 1
        q = np.zeros(nb * 32, np.int8)
        s = np.zeros(nb, np.float32)
        m = np.zeros(nb, np.int32)
        n = ctypes.c_size_t()
        self.check(lib().rh_quantize(self.handle, kind, _ptr(x), len(x), _ptr(q), _ptr(s), _ptr(m),
                                     ctypes.byref(n)))
        k = n.value
        return q[: k * 32], s[:k], m[:k]

    def ternary_dot_i32(self, m: "Matrix", inputs, tokens: int) -> np.ndarray:
        inputs = np.ascontiguousarray(inputs, dtype=np.float32)
        out = np.zeros(m.rows * tokens, np.int32)
        self.check(lib().rh_ternary_dot_i32(self.handle, m.handle, _ptr(inputs), len(inputs), tokens,
                                            _ptr(out), len(out)))
        return out


class Matrix:
    """A weight matrix resident in HBM (Matrix::load_on + upload)."""

    def __init__(self, ctx: Context, handle):
        self.ctx, self.handle = ctx, handle
        ctx._children.add(self)

    @classmethod
    def load(cls, ctx: Context, type_id: int, data, rows: int, cols: int) -> "Matrix":
        buf = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, (bytes, bytearray))
                                   else np.asarray(data).view(np.uint8).reshape(-1))
        h = ctypes.c_void_p()
        ctx.check(lib().rh_matrix_load(ctx.handle, type_id, _ptr(buf), buf.nbytes, rows, cols, ctypes.byref(h)))
        return cls(ctx, h)

    @property
    def rows(self) -> int:
        return lib().rh_matrix_rows(self.handle)

    @property
    def cols(self) -> int:
        return lib().rh_matrix_cols(self.handle)

    @property
    def type_id(self) -> int:
        return lib().rh_matrix_type(self.handle)

    @property
    def ternary_scale(self) -> float:
        return lib().rh_matrix_ternary_scale(self.handle)

    @property
    def device_bytes(self) -> int:
        return lib().rh_matrix_device_bytes(self.handle)

    def copy_row(self, index: int, out: np.ndarray) -> bool:
        found = ctypes.c_int()
        self.ctx.check(lib().rh_matrix_copy_row(self.ctx.handle, self.handle, index, _ptr(out), len(out),
                                                ctypes.byref(found)))
        return bool(found.value)

    def matvec(self, x, out: np.ndarray) -> None:
        matvec_batch(self.ctx, x, [(self, out)])

    def free(self) -> None:
        if self.handle:
            lib().rh_matrix_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Q8:
    """Device-quantized activations (Q8Input, q8_input.rs:13-23) of a batch."""

    def __init__(self, ctx: Context):
        h = ctypes.c_void_p()
        ctx.check(lib().rh_q8_new(ctx.handle, ctypes.byref(h)))
        self.ctx, self.handle = ctx, h
        ctx._children.add(self)

    def quantize(self, inputs, tokens: int, kind: int, stream: int = 0) -> "Q8":
        """Q8Input::quantize of every token of a device tensor `inputs`."""
        self.ctx.check(lib().rh_q8_quantize_device(self.ctx.handle, self.handle, kind, _ptr(inputs),
                                                   inputs.numel(), tokens, stream or None))
        return self

    def free(self) -> None:
        if self.handle:
            lib().rh_q8_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def dot_matrix_device(m: Matrix, q: Q8, out, stream: int = 0) -> None:
    """QuantKernel::dot_matrix (quant_kernel.rs:106-119) into a device tensor."""
    m.ctx.check(lib().rh_dot_matrix_device(m.ctx.handle, m.handle, q.handle, _ptr(out), out.numel(),
                                           stream or None))


Job = tuple  # (Matrix, out array)


def _jobs(jobs):
    arr = (_Job * max(1, len(jobs)))()
    for i, (m, out) in enumerate(jobs):
        n = out.numel() if hasattr(out, "numel") else len(out)
        arr[i] = _Job(m.handle.value if isinstance(m.handle, ctypes.c_void_p) else m.handle, _ptr(out), n)
    return arr


def matmul_batch(ctx: Context, inputs, tokens: int, jobs) -> None:
    """matmul.rs:229-248 on host arrays: out[row * tokens + token]."""
    inputs = np.ascontiguousarray(inputs, dtype=np.float32)
    for _, out in jobs:
        assert out.dtype == np.float32 and out.flags.c_contiguous
    ctx.check(lib().rh_matmul_batch(ctx.handle, _ptr(inputs), len(inputs), tokens, _jobs(jobs), len(jobs)))


def matvec_batch(ctx: Context, x, jobs) -> None:
    matmul_batch(ctx, x, 1, jobs)


def matmul_batch_device(ctx: Context, inputs, tokens: int, jobs, stream: int = 0) -> None:
    """Device-resident form: `inputs` and outputs are torch device tensors."""
    ctx.check(lib().rh_matmul_batch_device(ctx.handle, _ptr(inputs), inputs.numel(), tokens, _jobs(jobs),
                                           len(jobs), stream or None))


def matmul_batch_device_noalloc(ctx: Context, inputs, tokens: int, jobs, stream: int = 0) -> None:
    """rh_matmul_batch_device_noalloc: the device-resident form that allocates nothing."""
    ctx.check(lib().rh_matmul_batch_device_noalloc(ctx.handle, _ptr(inputs), inputs.numel(), tokens, _jobs(jobs),
                                                   len(jobs), stream or None))


def matmul_batch_device_repeat(ctx: Context, inputs, tokens: int, matrices, out, launches: int,
                               stream: int = 0) -> None:
    """`launches` rh_matmul_batch_device calls queued from C, call i on
    matrices[i % len(matrices)] (a bench hook)."""
    arr = (ctypes.c_void_p * len(matrices))(*[ctypes.cast(m.handle, ctypes.c_void_p).value for m in matrices])
    ctx.check(lib().rh_matmul_batch_device_repeat(ctx.handle, _ptr(inputs), inputs.numel(), tokens, arr,
                                                  len(matrices), _ptr(out), out.numel(), launches,
                                                  stream or None))


def matrix_handles(matrices, first: int = 0):
    """A ctypes array of the matrices' handles, rotated to start at `first`
    (built once, outside any timed region, for matmul_batch_device_repeat)."""
    n = len(matrices)
    order = [matrices[(first + i) % n] for i in range(n)]
    return (ctypes.c_void_p * n)(*[ctypes.cast(m.handle, ctypes.c_void_p).value for m in order])


def matmul_batch_device_repeat_handles(ctx: Context, inputs, tokens: int, handles, out, launches: int,
                                       stream: int = 0) -> None:
    """matmul_batch_device_repeat over a prebuilt handle array (matrix_handles)."""
    ctx.check(lib().rh_matmul_batch_device_repeat(ctx.handle, _ptr(inputs), inputs.numel(), tokens, handles,
                                                  len(handles), _ptr(out), out.numel(), launches,
                                                  stream or None))


def hold(ctx: Context, microseconds: int, stream: int = 0) -> None:
    """Occupies the stream for `microseconds` with one bounded wave (a bench
    hook): launches queued behind it start back to back."""
    ctx.check(lib().rh_hold_device(ctx.handle, int(microseconds), stream or None))


def reload_tuning() -> None:
    """Re-read the RUSTICIDE_HIP_* kernel switches (rh_init reads them once)."""
    lib().rh_reload_tuning()


# ------------------------------------------------------------------ decoder

STATUS.update({9: "CONTEXT_FULL", 10: "CACHE_POSITION", 11: "NO_VALID_TOKENS", 12: "GGUF", 13: "MISSING_METADATA",
               14: "MISSING_TENSOR", 15: "UNKNOWN_ARCHITECTURE"})


class _DecoderConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_size_t) for n in ("embedding_length", "block_count", "feed_forward_length",
                                               "head_count", "head_count_kv", "head_dim", "context_length",
                                               "vocab_size")] + [("rope_freq_base", ctypes.c_float),
                                                                 ("rms_norm_eps", ctypes.c_float)]


class _DecoderBlock(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output",
                                               "ffn_norm", "ffn_gate", "ffn_up", "ffn_down")]


class _DecoderWeights(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("token_embd", "output_norm", "output", "blocks")]


def _dec_lib() -> ctypes.CDLL:
    L = lib()
    if not hasattr(L, "_dec_ready"):
        P, S, St = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        L.rh_decoder_new.argtypes = [P, ctypes.POINTER(_DecoderConfig), ctypes.POINTER(_DecoderWeights),
                                     ctypes.POINTER(ctypes.c_void_p)]
        L.rh_decoder_new.restype = St
        L.rh_decoder_free.argtypes = [P]
        L.rh_decoder_reset.argtypes = [P]
        L.rh_decoder_position.argtypes = [P]
        L.rh_decoder_position.restype = S
        L.rh_decoder_forward_batch.argtypes = [P, P, S, S, P, S]
        L.rh_decoder_forward_batch.restype = St
        L.rh_decoder_generate_greedy.argtypes = [P, P, S, S, P, ctypes.POINTER(ctypes.c_size_t)]
        L.rh_decoder_generate_greedy.restype = St
        L._dec_ready = True
    return L


class Decoder:
    """The llama-family Decoder on the device (rh_decoder_*): a model dict of
    rusticide_amd.synth.decoder_model's shape, its matrices uploaded to HBM."""

    def __init__(self, ctx: Context, model: dict):
        L = _dec_lib()
        c = model["config"]
        self.ctx, self.config = ctx, c
        self._mats, self._keep = [], []

        def load(m):
            t, data, rows, cols = m
            mat = Matrix.load(ctx, t, data, rows, cols)
            self._mats.append(mat)
            return mat.handle.value if isinstance(mat.handle, ctypes.c_void_p) else mat.handle

        def vec(v):
            a = np.ascontiguousarray(v, np.float32)
            self._keep.append(a)
            return a.ctypes.data

        blocks = (_DecoderBlock * len(model["blocks"]))()
        for i, b in enumerate(model["blocks"]):
            blocks[i] = _DecoderBlock(vec(b["attn_norm"]), load(b["attn_q"]), load(b["attn_k"]), load(b["attn_v"]),
                                      load(b["attn_output"]), vec(b["ffn_norm"]), load(b["ffn_gate"]),
                                      load(b["ffn_up"]), load(b["ffn_down"]))
        out = load(model["output"]) if model.get("output") is not None else None
        w = _DecoderWeights(load(model["token_embd"]), vec(model["output_norm"]), out, ctypes.addressof(blocks))
        cfg = _DecoderConfig(*[c[k] for k in ("embedding_length", "block_count", "feed_forward_length",
                                              "head_count", "head_count_kv", "head_dim", "context_length",
                                              "vocab_size")], c["rope_freq_base"], c["rms_norm_eps"])
        h = ctypes.c_void_p()
        ctx.check(L.rh_decoder_new(ctx.handle, ctypes.byref(cfg), ctypes.byref(w), ctypes.byref(h)))
        self.handle = h
        self._blocks = blocks
        ctx._children.add(self)

    def forward_batch(self, tokens, start: int) -> np.ndarray:
        t = np.ascontiguousarray(tokens, np.uint32)
        logits = np.zeros(self.config["vocab_size"], np.float32)
        self.ctx.check(_dec_lib().rh_decoder_forward_batch(self.handle, t.ctypes.data, len(t), start,
                                                           logits.ctypes.data, len(logits)))
        return logits

    def forward(self, token: int, position: int) -> np.ndarray:
        return self.forward_batch([token], position)

    def reset(self) -> None:
        _dec_lib().rh_decoder_reset(self.handle)

    @property
    def position(self) -> int:
        return _dec_lib().rh_decoder_position(self.handle)

    def generate_greedy(self, prompt, max_tokens: int) -> np.ndarray:
        p = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(max(1, max_tokens), np.uint32)
        n = ctypes.c_size_t()
        self.ctx.check(_dec_lib().rh_decoder_generate_greedy(self.handle, p.ctypes.data, len(p), max_tokens,
                                                             out.ctypes.data, ctypes.byref(n)))
        return out[: n.value]

    def free(self) -> None:
        if self.handle:
            _dec_lib().rh_decoder_free(self.handle)
            self.handle = None
        for m in self._mats:
            m.free()
        self._mats = []

    close = free

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
