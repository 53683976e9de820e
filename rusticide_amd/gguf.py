"""GGUF v3 files: a writer for synthetic models, and the reader and HBM
upload of ``include/rusticide_hip.h`` (rh_gguf_*) over ctypes.

The writer lays files out as GGUF v3 does (crates/rusticide-io/src/gguf):
the 24-byte header (magic, version, tensor count, key count), the typed
key/value pairs, the tensor table (name, dimension count, dimensions
innermost first, type id, offset in the data section), then the data
section, every tensor starting on the alignment (``general.alignment``,
32 when absent).

``GgufFile`` parses bytes with ``rh_gguf_parse`` (GgufFile::from_bytes,
gguf/file.rs:39-62) and raises ``GgufError`` with the reference's error kind;
``GgufModel`` uploads a llama-family decoder's tensors to HBM
(DecoderWeights::from_source, crates/rusticide-transformer/src/loader.rs:19-92).
"""

from __future__ import annotations

import ctypes
import os
import struct

import numpy as np

from . import Context, Decoder, RusticideError, _DecoderConfig, _dec_lib, lib

__all__ = [
    "Writer", "GgufFile", "GgufModel", "GgufError", "decoder_gguf", "string_bytes", "header_bytes",
    "tensor_info_bytes", "value_bytes",
]

# metadata value type tags (gguf/value.rs:43-86)
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_SCALAR = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
           BOOL: "<B", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}

# GgufError kinds (crates/rusticide-io/src/error.rs), as rh_gguf_error.kind
KINDS = {
    1: "InvalidMagic", 2: "UnsupportedVersion", 3: "UnsupportedTensorType", 4: "CastOverflow",
    5: "InvalidAlignment", 6: "DuplicateKey", 7: "DuplicateTensor", 8: "TooManyDimensions",
    9: "ShapeOverflow", 10: "MisalignedTensor", 11: "OverlappingTensors", 12: "UnexpectedEof",
    13: "TensorNotFound", 14: "InvalidValueType", 15: "MetadataTooLarge", 16: "NestingTooDeep", 17: "NotAFile",
    18: "Io",
}

# ------------------------------------------------------------------ writer


def string_bytes(text) -> bytes:
    raw = text.encode() if isinstance(text, str) else bytes(text)
    return struct.pack("<Q", len(raw)) + raw


def header_bytes(version: int, tensor_count: int, kv_count: int, magic: bytes = b"GGUF") -> bytes:
    return magic + struct.pack("<IQQ", version, tensor_count, kv_count)


def tensor_info_bytes(name: str, dims, type_id: int, offset: int) -> bytes:
    """A tensor-table entry; `dims` in file order (innermost first)."""
    out = string_bytes(name) + struct.pack("<I", len(dims))
    out += b"".join(struct.pack("<Q", d) for d in dims)
    return out + struct.pack("<IQ", type_id, offset)


def value_bytes(tag: int, value) -> bytes:
    """The payload of a value of type `tag`; an array is (item_tag, items)."""
    if tag == STRING:
        return string_bytes(value)
    if tag == ARRAY:
        item, items = value
        return struct.pack("<IQ", item, len(items)) + b"".join(value_bytes(item, v) for v in items)
    return struct.pack(_SCALAR[tag], value)


def _align(n: int, a: int) -> int:
    return (n + a - 1) // a * a


class Writer:
    """Builds a GGUF v3 file in memory. Tensors are laid out in the order
    added, each at the next multiple of the alignment; `shape` is outermost
    first (rows, cols), as the reader reports it."""

    def __init__(self, magic: bytes = b"GGUF", version: int = 3):
        self.magic, self.version = magic, version
        self.kvs: list[bytes] = []
        self.tensors: list[tuple[str, list, int, bytes]] = []
        self.alignment_value = 32

    def kv(self, key: str, tag: int, value) -> "Writer":
        return self.raw_kv(key, tag, value_bytes(tag, value))

    def raw_kv(self, key: str, tag: int, payload: bytes) -> "Writer":
        self.kvs.append(string_bytes(key) + struct.pack("<I", tag) + payload)
        return self

    def alignment(self, alignment: int) -> "Writer":
        """Sets general.alignment (a UINT32) and pads the data to it."""
        self.alignment_value = alignment
        return self.kv("general.alignment", UINT32, alignment)

    def tensor(self, name: str, shape, type_id: int, data) -> "Writer":
        raw = data.tobytes() if isinstance(data, np.ndarray) else bytes(data)
        self.tensors.append((name, list(shape), type_id, raw))
        return self

    def build(self) -> bytes:
        a = self.alignment_value
        out = bytearray(header_bytes(self.version, len(self.tensors), len(self.kvs), self.magic))
        for kv in self.kvs:
            out += kv
        offset = 0
        for name, shape, type_id, raw in self.tensors:
            out += tensor_info_bytes(name, shape[::-1], type_id, offset)
            offset = _align(offset + len(raw), a)
        out += bytes(_align(len(out), a) - len(out))
        for _, _, _, raw in self.tensors:
            out += raw
            out += bytes(_align(len(out), a) - len(out))
        return bytes(out)


def decoder_gguf(model: dict, alignment: int = 32, tied_output: bool = False) -> bytes:
    """A llama-family GGUF of a decoder model dict (the layout of
    rusticide_amd.synth.decoder_model): the llama.* hyperparameters, norms
    as F32, matrices in their block formats under GGUF tensor names
    (crates/rusticide-transformer/src/loader.rs:49-92). `tied_output` leaves
    output.weight out, so the output shares token_embd."""
    c = model["config"]
    w = Writer()
    if alignment != 32:
        w.alignment(alignment)
    w.kv("general.architecture", STRING, "llama")
    for key, tag in (("context_length", UINT32), ("embedding_length", UINT32), ("block_count", UINT32),
                     ("feed_forward_length", UINT32), ("attention.head_count", UINT32),
                     ("attention.head_count_kv", UINT32)):
        w.kv(f"llama.{key}", tag, c[key.split(".")[-1]])
    w.kv("llama.rope.dimension_count", UINT32, c["head_dim"])
    w.kv("llama.rope.freq_base", FLOAT32, c["rope_freq_base"])
    w.kv("llama.attention.layer_norm_rms_epsilon", FLOAT32, c["rms_norm_eps"])

    def mat(name, m):
        type_id, data, rows, cols = m
        w.tensor(name, [rows, cols], type_id, data)

    def vec(name, v):
        v = np.ascontiguousarray(v, np.float32)
        w.tensor(name, [v.size], 0, v)

    mat("token_embd.weight", model["token_embd"])
    for i, b in enumerate(model["blocks"]):
        vec(f"blk.{i}.attn_norm.weight", b["attn_norm"])
        for part in ("attn_q", "attn_k", "attn_v", "attn_output"):
            mat(f"blk.{i}.{part}.weight", b[part])
        vec(f"blk.{i}.ffn_norm.weight", b["ffn_norm"])
        for part in ("ffn_gate", "ffn_up", "ffn_down"):
            mat(f"blk.{i}.{part}.weight", b[part])
    vec("output_norm.weight", model["output_norm"])
    if model.get("output") is not None and not tied_output:
        mat("output.weight", model["output"])
    return w.build()


# ------------------------------------------------------------------ reader

class _Error(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_uint32), ("value", ctypes.c_uint64), ("name", ctypes.c_char * 128),
                ("other", ctypes.c_char * 128)]


class GgufError(RusticideError):
    """A GgufError of the reference: `kind` is its variant name, `value`,
    `name` and `other` its payload (version, type id, offset or limit; the
    tensor or key; the second tensor of an overlap)."""

    def __init__(self, kind: str, value: int = 0, name: str = "", other: str = ""):
        self.gguf_kind, self.value, self.name, self.other = kind, value, name, other
        detail = ", ".join(x for x in (name, other) if x)
        RusticideError.__init__(self, 12, f"{kind}" + (f" ({detail})" if detail else ""))

    @classmethod
    def _from(cls, e: _Error) -> "GgufError":
        dec = lambda b: b.decode("utf-8", "replace")  # noqa: E731
        return cls(KINDS.get(e.kind, str(e.kind)), e.value, dec(e.name), dec(e.other))


def _gguf_lib() -> ctypes.CDLL:
    L = _dec_lib()
    if not hasattr(L, "_gguf_ready"):
        P, S, St, U32, U64 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_uint32, ctypes.c_uint64
        PE = ctypes.POINTER(_Error)
        L.rh_gguf_parse.argtypes = [P, S, ctypes.POINTER(P), PE]
        L.rh_gguf_parse.restype = St
        L.rh_gguf_free.argtypes = [P]
        L.rh_gguf_open.argtypes = [ctypes.c_char_p, ctypes.POINTER(P), PE]
        L.rh_gguf_open.restype = St
        for n in ("rh_gguf_metadata_count", "rh_gguf_tensor_count"):
            getattr(L, n).argtypes = [P]
            getattr(L, n).restype = S
        L.rh_gguf_tensor_at.argtypes = [P, S, ctypes.POINTER(P), ctypes.POINTER(S), ctypes.POINTER(U32),
                                        ctypes.POINTER(S), ctypes.POINTER(U64), ctypes.POINTER(U64)]
        L.rh_gguf_tensor_at.restype = St
        L.rh_gguf_tensor_find.argtypes = [P, ctypes.c_char_p, ctypes.POINTER(S)]
        L.rh_gguf_tensor_find.restype = St
        L.rh_gguf_tensor_data.argtypes = [P, ctypes.c_char_p, ctypes.POINTER(P), ctypes.POINTER(S), PE]
        L.rh_gguf_tensor_data.restype = St
        L.rh_gguf_meta_type.argtypes = [P, ctypes.c_char_p, ctypes.POINTER(U32)]
        L.rh_gguf_meta_uint.argtypes = [P, ctypes.c_char_p, ctypes.POINTER(U64)]
        L.rh_gguf_meta_float.argtypes = [P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float)]
        L.rh_gguf_meta_string.argtypes = [P, ctypes.c_char_p, ctypes.POINTER(P), ctypes.POINTER(S)]
        for n in ("rh_gguf_meta_type", "rh_gguf_meta_uint", "rh_gguf_meta_float", "rh_gguf_meta_string"):
            getattr(L, n).restype = St
        L.rh_gguf_decoder_config.argtypes = [P, P, ctypes.POINTER(_DecoderConfig)]
        L.rh_gguf_decoder_config.restype = St
        L.rh_gguf_model_load.argtypes = [P, P, ctypes.POINTER(P)]
        L.rh_gguf_model_load.restype = St
        L.rh_gguf_model_config.argtypes = [P]
        L.rh_gguf_model_config.restype = ctypes.POINTER(_DecoderConfig)
        L.rh_gguf_model_decoder.argtypes = [P, ctypes.POINTER(P)]
        L.rh_gguf_model_decoder.restype = St
        L.rh_gguf_model_free.argtypes = [P]
        L._gguf_ready = True
    return L


def _config_dict(c: _DecoderConfig) -> dict:
    return {name: getattr(c, name) for name, _ in _DecoderConfig._fields_}


class GgufFile:
    """A parsed GGUF v3 file (GgufFile): metadata, the tensor table in
    sorted-name order, and the bytes of each tensor."""

    def __init__(self, data: bytes):
        L = _gguf_lib()
        buf = bytes(data)
        h, err = ctypes.c_void_p(), _Error()
        st = L.rh_gguf_parse(buf, len(buf), ctypes.byref(h), ctypes.byref(err))
        if st == 12:
            raise GgufError._from(err)
        if st != 0:
            raise RusticideError(st, "rh_gguf_parse")
        self.handle = h

    @classmethod
    def load(cls, path) -> "GgufFile":
        """GgufFile::load (gguf/file.rs:62-77) by rh_gguf_open: the file is
        mapped, not copied. A directory, device or pipe is NotAFile; a file
        that cannot be opened is Io, with its errno as `value`."""
        L = _gguf_lib()
        self = cls.__new__(cls)
        self.handle = None
        h, err = ctypes.c_void_p(), _Error()
        st = L.rh_gguf_open(os.fsencode(path), ctypes.byref(h), ctypes.byref(err))
        if st == 12:
            raise GgufError._from(err)
        if st != 0:
            raise RusticideError(st, "rh_gguf_open")
        self.handle = h
        return self

    def _h(self):
        if not self.handle:
            raise RusticideError(1, "the file is closed")
        return self.handle

    def close(self) -> None:
        if getattr(self, "handle", None):
            _gguf_lib().rh_gguf_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def metadata_count(self) -> int:
        return _gguf_lib().rh_gguf_metadata_count(self._h())

    @property
    def tensor_count(self) -> int:
        return _gguf_lib().rh_gguf_tensor_count(self._h())

    def _at(self, index: int):
        name, nlen, t, n, off = ctypes.c_void_p(), ctypes.c_size_t(), ctypes.c_uint32(), ctypes.c_size_t(), ctypes.c_uint64()
        shape = (ctypes.c_uint64 * 4)()
        st = _gguf_lib().rh_gguf_tensor_at(self._h(), index, ctypes.byref(name), ctypes.byref(nlen), ctypes.byref(t),
                                           ctypes.byref(n), shape, ctypes.byref(off))
        if st != 0:
            raise IndexError(index)
        return ctypes.string_at(name, nlen.value).decode(), list(shape[: n.value]), t.value, off.value

    def tensor_info_at(self, index: int):
        """(name, shape outermost first, type id, offset) of tensor_names()[index]."""
        return self._at(index)

    def tensor_names(self) -> list:
        return [self._at(i)[0] for i in range(self.tensor_count)]

    def tensor_info(self, name: str):
        """(shape outermost first, type id, offset), or None."""
        i = ctypes.c_size_t()
        if _gguf_lib().rh_gguf_tensor_find(self._h(), name.encode(), ctypes.byref(i)) != 0:
            return None
        return self._at(i.value)[1:]

    def tensor_bytes(self, name: str) -> bytes:
        """The tensor's bytes (blocks and any trailer; F32/F16 values)."""
        p, n, err = ctypes.c_void_p(), ctypes.c_size_t(), _Error()
        st = _gguf_lib().rh_gguf_tensor_data(self._h(), name.encode(), ctypes.byref(p), ctypes.byref(n),
                                             ctypes.byref(err))
        if st == 12:
            raise GgufError._from(err)
        if st != 0:
            raise RusticideError(st, "rh_gguf_tensor_data")
        return ctypes.string_at(p, n.value) if n.value else b""

    def meta_type(self, key: str):
        t = ctypes.c_uint32()
        return t.value if _gguf_lib().rh_gguf_meta_type(self._h(), key.encode(), ctypes.byref(t)) == 0 else None

    def meta_uint(self, key: str):
        v = ctypes.c_uint64()
        return v.value if _gguf_lib().rh_gguf_meta_uint(self._h(), key.encode(), ctypes.byref(v)) == 0 else None

    def meta_float(self, key: str):
        v = ctypes.c_float()
        return v.value if _gguf_lib().rh_gguf_meta_float(self._h(), key.encode(), ctypes.byref(v)) == 0 else None

    def meta_string(self, key: str):
        v, n = ctypes.c_void_p(), ctypes.c_size_t()
        if _gguf_lib().rh_gguf_meta_string(self._h(), key.encode(), ctypes.byref(v), ctypes.byref(n)) != 0:
            return None
        return ctypes.string_at(v, n.value).decode()

    def decoder_config(self) -> dict:
        """DecoderConfig::from_source for the llama family; needs no device.
        Raises RusticideError (MISSING_METADATA, UNKNOWN_ARCHITECTURE,
        MISSING_TENSOR, INVALID_CONFIG)."""
        c = _DecoderConfig()
        st = _gguf_lib().rh_gguf_decoder_config(None, self._h(), ctypes.byref(c))
        if st != 0:
            raise RusticideError(st, lib().rh_last_error(None).decode())
        return _config_dict(c)


class GgufModel:
    """A llama-family decoder's weights uploaded from a GgufFile to HBM
    (rh_gguf_model_load); `decoder()` makes a Decoder over them."""

    def __init__(self, ctx: Context, file: GgufFile):
        L = _gguf_lib()
        h = ctypes.c_void_p()
        ctx.check(L.rh_gguf_model_load(ctx.handle, file._h(), ctypes.byref(h)))
        self.ctx, self.handle = ctx, h
        self.config = _config_dict(L.rh_gguf_model_config(h).contents)
        self._decoders = []
        ctx._children.add(self)

    def decoder(self) -> Decoder:
        h = ctypes.c_void_p()
        self.ctx.check(_gguf_lib().rh_gguf_model_decoder(self.handle, ctypes.byref(h)))
        d = Decoder.__new__(Decoder)
        d.ctx, d.config, d._mats, d._keep, d._blocks = self.ctx, dict(self.config), [], [self], None
        d.handle = h
        self.ctx._children.add(d)
        self._decoders.append(d)
        return d

    def free(self) -> None:
        # decoders borrow the matrices: they go first
        for d in getattr(self, "_decoders", []):
            d.free()
        self._decoders = []
        if getattr(self, "handle", None):
            _gguf_lib().rh_gguf_model_free(self.handle)
            self.handle = None

    close = free

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
