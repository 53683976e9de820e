"""The GGUF reader (rh_gguf_parse and friends) against the cases rusticide's
own GGUF tests hold (crates/rusticide-io/src/gguf/*_tests.rs) and the llama
config tests (crates/rusticide-llama/src/config_tests.rs,
crates/rusticide-model/src/registry_tests.rs). None of this needs a device.

String decoding is pinned independently: Python's bytes.decode("utf-8",
"replace") follows the same maximal-subpart replacement rule as Rust's
String::from_utf8_lossy, so random byte strings must decode alike.
"""

import errno
import os
import struct

import numpy as np
import pytest

import rusticide_amd as R
from rusticide_amd import gguf as G
from rusticide_amd.gguf import (ARRAY, BOOL, FLOAT32, FLOAT64, INT8, INT16, INT32, INT64, STRING, UINT8, UINT16,
                                UINT32, UINT64, GgufError, GgufFile, Writer, header_bytes, string_bytes,
                                tensor_info_bytes)

F32, F16 = 0, 1


def parse(data: bytes) -> GgufFile:
    return GgufFile(data)


def error(data: bytes) -> GgufError:
    with pytest.raises(GgufError) as e:
        GgufFile(data)
    return e.value


def one_kv(tag: int, payload: bytes) -> bytes:
    return Writer().raw_kv("k", tag, payload).build()


# ------------------------------------------------------------ header.rs

def test_header_errors():
    # header_tests.rs, file_tests.rs:43-53
    assert error(Writer(magic=b"NOPE").build()).gguf_kind == "InvalidMagic"
    for version in (2, 4):
        e = error(Writer(version=version).build())
        assert (e.gguf_kind, e.value) == ("UnsupportedVersion", version)
    assert error(header_bytes(3, 0, 0)[:23]).gguf_kind == "UnexpectedEof"
    assert error(b"XXXX").gguf_kind == "UnexpectedEof"  # a short file is EOF before its magic
    assert error(b"").gguf_kind == "UnexpectedEof"


def test_counts_beyond_the_file_are_eof():
    # file_tests.rs:122-132
    assert error(header_bytes(3, 2 ** 64 - 1, 0)).gguf_kind == "UnexpectedEof"
    assert error(header_bytes(3, 0, 2 ** 64 - 1)).gguf_kind == "UnexpectedEof"


# ------------------------------------------------------------ file.rs

def test_an_empty_file_parses():
    f = parse(Writer().build())
    assert (f.metadata_count, f.tensor_count, f.tensor_names()) == (0, 0, [])
    assert f.tensor_info("x") is None


def test_metadata_is_parsed():
    f = parse(Writer().kv("k", UINT32, 2).kv("other", UINT32, 3).build())
    assert f.metadata_count == 2
    assert (f.meta_type("k"), f.meta_uint("k")) == (UINT32, 2)
    assert f.meta_type("missing") is None


def test_an_invalid_value_type_is_rejected():
    e = error(Writer().raw_kv("k", 99, bytes(4)).build())
    assert (e.gguf_kind, e.value) == ("InvalidValueType", 99)
    assert error(Writer().raw_kv("k", 13, bytes(4)).build()).value == 13


def test_duplicate_keys_and_tensors_are_rejected():
    e = error(Writer().kv("k", UINT32, 1).kv("k", UINT32, 2).build())
    assert (e.gguf_kind, e.name) == ("DuplicateKey", "k")
    e = error(Writer().tensor("w", [1], F32, bytes(4)).tensor("w", [1], F32, bytes(4)).build())
    assert (e.gguf_kind, e.name) == ("DuplicateTensor", "w")


def test_tensor_names_are_sorted():
    w = Writer()
    for name in "hdagcfbe":
        w.tensor(name, [1], F32, bytes(4))
    f = parse(w.build())
    assert f.tensor_names() == list("abcdefgh")
    assert f.tensor_count == len(f.tensor_names())


def test_multiple_tensor_infos():
    # file_tests.rs:68-79: GGUF dims [2, 3] are shape [3, 2]
    f = parse(Writer().tensor("a", [3, 2], F32, bytes(24)).tensor("b", [4], F16, bytes(8)).build())
    assert f.tensor_info("a") == ([3, 2], F32, 0)
    assert f.tensor_info("b") == ([4], F16, 32)


def test_five_dimensions_are_rejected():
    data = header_bytes(3, 1, 0) + tensor_info_bytes("t", [1] * 5, F32, 0)
    e = error(data)
    assert (e.gguf_kind, e.value) == ("TooManyDimensions", 5)


def test_data_start_follows_the_alignment():
    for align in (32, 64, 256):
        w = Writer()
        if align != 32:
            w.alignment(align)
        data = w.tensor("a", [1], F32, bytes([7] * 4)).build()
        f = parse(data)
        assert f.tensor_bytes("a") == bytes([7] * 4)
        assert (len(data) - 32 if align == 32 else len(data) - align) % align == 0
        start = data.index(bytes([7] * 4))
        assert start % align == 0


def test_invalid_alignment_rejects_the_file():
    # file_tests.rs:163-176, metadata_tests.rs:115-139
    for tag, value in ((UINT32, 0), (UINT32, 48), (STRING, "32"), (UINT64, 32)):
        e = error(Writer().kv("general.alignment", tag, value).build())
        assert e.gguf_kind == "InvalidAlignment", (tag, value)


def test_a_misaligned_offset_is_rejected():
    data = header_bytes(3, 1, 0) + tensor_info_bytes("w", [1], F32, 4)
    data += bytes(-len(data) % 32 + 32)
    e = error(data)
    assert (e.gguf_kind, e.name, e.value) == ("MisalignedTensor", "w", 4)


def test_an_offset_on_a_custom_alignment_is_accepted():
    f = parse(Writer().alignment(64).tensor("a", [1], F32, bytes(4)).tensor("b", [1], F32, bytes(4)).build())
    assert f.tensor_info("b")[2] == 64


def test_the_data_section_may_start_at_eof_but_not_past_it():
    data = Writer().build()
    parse(data)
    assert error(data[:-8]).gguf_kind == "UnexpectedEof"


# ------------------------------------------------------------ value.rs

def test_each_scalar_type_parses_little_endian():
    cases = [
        (UINT8, bytes([200])), (INT8, bytes([0xFF])), (UINT16, bytes([1, 2])), (INT16, bytes([0xFE, 0xFF])),
        (UINT32, struct.pack("<I", 0x04030201)), (INT32, struct.pack("<i", -3)), (FLOAT32, struct.pack("<f", 1.5)),
        (BOOL, bytes([7])), (UINT64, struct.pack("<Q", 2 ** 64 - 1)), (INT64, struct.pack("<q", 6)),
        (FLOAT64, struct.pack("<d", 0.25)),
    ]
    for tag, payload in cases:
        f = parse(one_kv(tag, payload))
        assert f.meta_type("k") == tag
    # Metadata::arch_unsigned accepts u32, u64 and non-negative i32/i64 only
    assert parse(one_kv(UINT32, struct.pack("<I", 0x04030201))).meta_uint("k") == 0x04030201
    assert parse(one_kv(UINT64, struct.pack("<Q", 2 ** 64 - 1))).meta_uint("k") == 2 ** 64 - 1
    assert parse(one_kv(INT32, struct.pack("<i", 5))).meta_uint("k") == 5
    assert parse(one_kv(INT64, struct.pack("<q", 6))).meta_uint("k") == 6
    assert parse(one_kv(INT32, struct.pack("<i", -1))).meta_uint("k") is None
    assert parse(one_kv(INT64, struct.pack("<q", -1))).meta_uint("k") is None
    assert parse(one_kv(UINT16, bytes([1, 2]))).meta_uint("k") is None
    # arch_float: f32, or f64 narrowed
    assert parse(one_kv(FLOAT32, struct.pack("<f", 7.5))).meta_float("k") == 7.5
    assert parse(one_kv(FLOAT64, struct.pack("<d", 0.1))).meta_float("k") == float(np.float32(0.1))
    assert parse(one_kv(UINT32, struct.pack("<I", 1))).meta_float("k") is None


def test_truncated_scalars_are_eof():
    # value_tests.rs:155-165: the file ends one byte into the value
    for tag, width in ((UINT8, 1), (UINT16, 2), (UINT32, 4), (FLOAT32, 4), (BOOL, 1), (UINT64, 8), (FLOAT64, 8)):
        data = header_bytes(3, 0, 1) + string_bytes("k") + struct.pack("<I", tag) + bytes(width - 1)
        assert error(data).gguf_kind == "UnexpectedEof", tag
        parse(data + bytes(1 + (-(len(data) + 1)) % 32))


def test_strings_parse_and_replace_invalid_utf8():
    f = parse(Writer().kv("s", STRING, "héllo").raw_kv("bad", STRING, string_bytes(b"\xffa")).build())
    assert f.meta_string("s") == "héllo"
    assert f.meta_string("bad") == "�a"  # cursor_tests.rs:64-68
    raw = header_bytes(3, 0, 1) + string_bytes("s") + struct.pack("<I", STRING) + struct.pack("<Q", 10) + b"abc"
    assert error(raw).gguf_kind == "UnexpectedEof"


def test_lossy_utf8_matches_maximal_subpart_replacement():
    rng = np.random.default_rng(5)
    pieces = [b"\xe2\x82\xac", b"\xf0\x9f\x98\x80", b"\xc3\xa9", b"a", b"\xed\xa0\x80", b"\xf4\x90\x80\x80",
              b"\xe0\x80\xaf", b"\xc0\xaf", b"\xf8\x88\x80\x80\x80", b"\xe2\x82", b"\xf0\x9f\x98", b"\x80", b"\xbf",
              b"\xfe", b"\xff", b"\xc2", b"\xe1\x80", b"\xf1\x80\x80"]
    w = Writer()
    want = {}
    for i in range(300):
        if i % 2:
            s = b"".join(pieces[j] for j in rng.integers(0, len(pieces), rng.integers(0, 8)))
        else:
            s = rng.integers(0, 256, rng.integers(0, 12)).astype(np.uint8).tobytes()
        w.raw_kv(f"s{i}", STRING, string_bytes(s))
        want[f"s{i}"] = s.decode("utf-8", "replace")
    f = parse(w.build())
    for k, v in want.items():
        assert f.meta_string(k) == v, k


def array_header(item: int, n: int) -> bytes:
    return struct.pack("<IQ", item, n)


def test_arrays_parse():
    f = parse(Writer().kv("a", ARRAY, (STRING, ["x", "yz"])).kv("e", ARRAY, (UINT8, [])).build())
    assert f.meta_type("a") == ARRAY and f.meta_type("e") == ARRAY
    e = error(Writer().raw_kv("a", ARRAY, array_header(99, 0)).build())
    assert (e.gguf_kind, e.value) == ("InvalidValueType", 99)
    raw = header_bytes(3, 0, 1) + string_bytes("a") + struct.pack("<I", ARRAY) + array_header(UINT32, 3) + bytes(8)
    assert error(raw).gguf_kind == "UnexpectedEof"  # more items claimed than bytes


def nested(depth: int) -> bytes:
    return array_header(ARRAY, 1) * (depth - 1) + array_header(UINT8, 0)


def test_arrays_nest_eight_deep_and_no_deeper():
    # value_tests.rs:167-202
    parse(Writer().raw_kv("a", ARRAY, nested(8)).build())
    e = error(Writer().raw_kv("a", ARRAY, nested(9)).build())
    assert (e.gguf_kind, e.value) == ("NestingTooDeep", 8)
    e = error(Writer().raw_kv("a", ARRAY, array_header(ARRAY, 1) * 100_000).build())
    assert (e.gguf_kind, e.value) == ("NestingTooDeep", 8)


def test_the_metadata_element_budget_is_file_wide():
    # value.rs:14: 2^22 array elements across the file, spent per element
    limit = 1 << 22
    half = limit // 2
    ok = Writer().raw_kv("a", ARRAY, array_header(UINT8, half) + bytes(half))
    ok.raw_kv("b", ARRAY, array_header(UINT8, half) + bytes(half))
    parse(ok.build())
    over = Writer().raw_kv("a", ARRAY, array_header(UINT8, half) + bytes(half))
    over.raw_kv("b", ARRAY, array_header(UINT8, half + 1) + bytes(half + 1))
    e = error(over.build())
    assert (e.gguf_kind, e.value) == ("MetadataTooLarge", limit)
    # nested arrays spend one element for the inner array and one per item
    # (value_tests.rs:250-262): 2^21 of them spend exactly the limit
    inner = array_header(UINT8, 1) + bytes(1)
    parse(Writer().raw_kv("n", ARRAY, array_header(ARRAY, half) + inner * half).build())
    e = error(Writer().raw_kv("n", ARRAY, array_header(ARRAY, half + 1) + inner * (half + 1)).build())
    assert (e.gguf_kind, e.value) == ("MetadataTooLarge", limit)


# ------------------------------------------------------------ tensor_info.rs

def table(*entries, data: int = 128) -> bytes:
    out = header_bytes(3, len(entries), 0) + b"".join(tensor_info_bytes(*e) for e in entries)
    return out + bytes(-len(out) % 32 + data)


def test_tensor_info_shapes():
    f = parse(table(("w", [4, 3, 2], F32, 0)))
    assert f.tensor_info("w") == ([2, 3, 4], F32, 0)
    assert parse(table(("s", [], F32, 0))).tensor_info("s") == ([1], F32, 0)
    assert parse(table(("u", [4], 99, 0))).tensor_info("u") == ([4], 99, 0)  # recorded, fails on load
    assert parse(table(("q", [1, 1, 1, 1], F32, 0))).tensor_info("q")[0] == [1, 1, 1, 1]


def test_tensor_info_errors():
    e = error(header_bytes(3, 1, 0) + string_bytes("w") + struct.pack("<I", 2 ** 32 - 1))
    assert (e.gguf_kind, e.value) == ("TooManyDimensions", 2 ** 32 - 1)
    e = error(header_bytes(3, 1, 0) + string_bytes("w") + struct.pack("<IQ", 2, 4))
    assert e.gguf_kind == "UnexpectedEof"
    e = error(table(("big", [2 ** 32, 2 ** 32], F32, 0)))
    assert (e.gguf_kind, e.name) == ("ShapeOverflow", "big")
    # an extent past the address range still fits when another is zero
    f = parse(table(("z", [2 ** 64 - 1, 0], F32, 0)))
    assert f.tensor_info("z")[0] == [0, 2 ** 64 - 1]
    full = tensor_info_bytes("w", [1], F32, 0)
    assert error(header_bytes(3, 1, 0) + full[:-10]).gguf_kind == "UnexpectedEof"  # the type tag
    assert error(header_bytes(3, 1, 0) + full[:-4]).gguf_kind == "UnexpectedEof"  # the offset


# ------------------------------------------------------------ extent.rs

def overlap(first, second):
    try:
        parse(table(("a",) + first, ("b",) + second))
    except GgufError as e:
        assert e.gguf_kind == "OverlappingTensors", e
        return e.name, e.other
    return None


def test_overlapping_extents():
    # extent_tests.rs:31-113
    assert overlap(([4], F32, 0), ([4], F32, 0)) == ("a", "b")
    assert overlap(([16], F32, 0), ([4], F32, 32)) == ("a", "b")
    assert overlap(([4], F32, 32), ([16], F32, 0)) == ("b", "a")  # data order, not table order
    assert overlap(([8], F32, 0), ([8], F32, 32)) is None
    assert overlap(([0], F32, 0), ([4], F32, 0)) is None
    assert overlap(([4], F32, 0), ([4], 999, 0)) is None  # left to fail on load
    assert overlap(([4], F32, 0), ([4], F32, 2 ** 64 - 32)) is None  # end overflows: left to fail on load
    assert overlap(([16], F32, 0), ([0], F32, 32)) is None
    assert overlap(([128], 36, 0), ([4], F32, 32)) == ("a", "b")  # the I2_S trailer is the tensor's
    assert overlap(([128], 36, 0), ([4], F32, 64)) is None


def test_builder_files_never_overlap():
    parse(Writer().tensor("x", [3], F32, bytes(12)).tensor("y", [5], F32, bytes(20)).tensor("z", [1], F32, bytes(4))
          .build())


# ------------------------------------------------------------ load.rs

def test_tensor_bytes():
    values = np.arange(12, dtype=np.float32)
    halves = np.array([1.0, -2.0], np.float16)
    f = parse(Writer().tensor("m", [3, 4], F32, values).tensor("h", [2], F16, halves).build())
    assert np.array_equal(np.frombuffer(f.tensor_bytes("m"), np.float32), values)
    assert np.array_equal(np.frombuffer(f.tensor_bytes("h"), np.float16), halves)
    e = pytest.raises(GgufError, f.tensor_bytes, "nope").value
    assert (e.gguf_kind, e.name) == ("TensorNotFound", "nope")


def test_an_unknown_type_fails_only_when_read():
    # load_type_tests.rs:24-47
    f = parse(Writer().kv("general.architecture", STRING, "llama").tensor("good", [1], F32, bytes(4))
              .tensor("odd", [1], 99, bytes(4)).build())
    assert f.tensor_bytes("good") == bytes(4)
    e = pytest.raises(GgufError, f.tensor_bytes, "odd").value
    assert (e.gguf_kind, e.name, e.value) == ("UnsupportedTensorType", "odd", 99)


def test_block_tensors_borrow_their_blocks_and_trailer():
    block = bytes(range(34))
    f = parse(Writer().tensor("q8", [32], 8, block).build())
    assert f.tensor_bytes("q8") == block
    i2s = bytes([0xAA] * 32) + struct.pack("<f", 0.5) + bytes(28)
    f = parse(Writer().tensor("t", [128], 36, i2s).build())
    assert f.tensor_bytes("t") == i2s
    # without its trailer the tensor runs past the file
    short = header_bytes(3, 1, 0) + tensor_info_bytes("t", [128], 36, 0)
    short += bytes(-len(short) % 32) + bytes(32)
    assert pytest.raises(GgufError, parse(short).tensor_bytes, "t").value.gguf_kind == "UnexpectedEof"


def test_extents_past_the_file_are_eof():
    # load_tests.rs:192-216
    short = header_bytes(3, 1, 0) + tensor_info_bytes("q", [64], 2, 0)  # two Q4_0 blocks, one present
    short += bytes(-len(short) % 32) + bytes(18)
    assert pytest.raises(GgufError, parse(short).tensor_bytes, "q").value.gguf_kind == "UnexpectedEof"
    for offset in (2 ** 64 - 32, 2 ** 63):
        f = parse(table(("w", [1], F32, offset)))
        assert pytest.raises(GgufError, f.tensor_bytes, "w").value.gguf_kind == "UnexpectedEof"


def test_offsets_are_relative_to_the_data_section():
    f = parse(Writer().tensor("first", [1], F32, struct.pack("<f", 1.0)).tensor("second", [2], F32,
                                                                            struct.pack("<2f", 2.0, 3.0)).build())
    assert f.tensor_info("second")[2] == 32
    assert np.array_equal(np.frombuffer(f.tensor_bytes("second"), np.float32), [2.0, 3.0])


def test_load_maps_regular_files_only(tmp_path):
    # file_tests.rs:194-230
    p = tmp_path / "m.gguf"
    p.write_bytes(Writer().tensor("a", [1], F32, bytes([9] * 4)).build())
    f = GgufFile.load(p)
    assert f.tensor_names() == ["a"] and f.tensor_bytes("a") == bytes([9] * 4)
    f.close()
    e = pytest.raises(GgufError, GgufFile.load, tmp_path / "missing.gguf").value
    assert (e.gguf_kind, e.value) == ("Io", errno.ENOENT)
    fifo = tmp_path / "pipe"
    os.mkfifo(fifo)
    for special in (tmp_path, "/dev/zero", fifo):
        if os.path.exists(special):
            assert pytest.raises(GgufError, GgufFile.load, special).value.gguf_kind == "NotAFile"
    # an empty file and a truncated one fail as their bytes would
    (tmp_path / "empty.gguf").write_bytes(b"")
    assert pytest.raises(GgufError, GgufFile.load, tmp_path / "empty.gguf").value.gguf_kind == "UnexpectedEof"
    (tmp_path / "short.gguf").write_bytes(Writer().build()[:-8])
    assert pytest.raises(GgufError, GgufFile.load, tmp_path / "short.gguf").value.gguf_kind == "UnexpectedEof"


def test_a_mapped_file_reads_like_parsed_bytes(tmp_path):
    from rusticide_amd import synth
    model = synth.decoder_model(dict(embedding_length=256, block_count=1, feed_forward_length=512, head_count=4,
                                     head_count_kv=2, head_dim=64, context_length=64, vocab_size=64,
                                     rope_freq_base=10000.0, rms_norm_eps=1e-5), seed=3)
    data = G.decoder_gguf(model)
    (tmp_path / "m.gguf").write_bytes(data)
    a, b = GgufFile(data), GgufFile.load(tmp_path / "m.gguf")
    assert a.tensor_names() == b.tensor_names() and a.decoder_config() == b.decoder_config()
    for name in a.tensor_names():
        assert a.tensor_info(name) == b.tensor_info(name) and a.tensor_bytes(name) == b.tensor_bytes(name)


# ------------------------------------------------------------ decoder config

TINY_VOCAB = 6


def tiny(meta: dict = None, drop=(), tensors: dict = None) -> GgufFile:
    """The reference's tiny llama source (crates/rusticide-llama/src/testing.rs):
    embedding 4, one block, FFN 8, 2/1 heads, context 16, token_embd [vocab, 4]."""
    base = {"general.architecture": (STRING, "llama"), "llama.embedding_length": (UINT32, 4),
            "llama.block_count": (UINT32, 1), "llama.feed_forward_length": (UINT32, 8),
            "llama.attention.head_count": (UINT32, 2), "llama.attention.head_count_kv": (UINT32, 1),
            "llama.context_length": (UINT32, 16)}
    base.update(meta or {})
    w = Writer()
    for k, (tag, v) in base.items():
        if k not in drop:
            w.kv(k, tag, v)
    ts = {"token_embd.weight": [TINY_VOCAB, 4]}
    ts.update(tensors or {})
    for name, shape in ts.items():
        w.tensor(name, shape, F32, bytes(4 * int(np.prod(shape))))
    return parse(w.build())


def config_error(f: GgufFile) -> R.RusticideError:
    with pytest.raises(R.RusticideError) as e:
        f.decoder_config()
    return e.value


def invalid(f: GgufFile, reason: str):
    e = config_error(f)
    assert e.kind == "INVALID_CONFIG" and str(e).endswith(reason), str(e)


def test_config_reads_the_tiny_source():
    c = tiny().decoder_config()
    assert (c["vocab_size"], c["embedding_length"], c["block_count"], c["feed_forward_length"]) == (6, 4, 1, 8)
    assert (c["head_count"], c["head_count_kv"], c["head_dim"], c["context_length"]) == (2, 1, 2, 16)
    assert c["rope_freq_base"] == 10000.0 and c["rms_norm_eps"] == float(np.float32(1e-5))


def test_config_reads_explicit_rope_base_eps_and_kv_heads():
    f = tiny({"llama.rope.freq_base": (FLOAT32, 500.0), "llama.attention.layer_norm_rms_epsilon": (FLOAT32, 1e-6)},
             drop=("llama.attention.head_count_kv",))
    c = f.decoder_config()
    assert c["rope_freq_base"] == 500.0 and c["rms_norm_eps"] == float(np.float32(1e-6))
    assert c["head_count_kv"] == 2
    # f64 values are narrowed, unsigned keys accept i32/i64/u64
    c = tiny({"llama.rope.freq_base": (FLOAT64, 0.1), "llama.block_count": (INT64, 1),
              "llama.context_length": (UINT64, 16)}).decoder_config()
    assert c["rope_freq_base"] == float(np.float32(0.1)) and c["block_count"] == 1


def test_config_names_a_missing_key():
    for key in ("llama.context_length", "llama.embedding_length", "llama.block_count",
                "llama.feed_forward_length", "llama.attention.head_count"):
        e = config_error(tiny(drop=(key,)))
        assert e.kind == "MISSING_METADATA" and key in str(e)
    e = config_error(tiny({"llama.block_count": (INT32, -1)}))
    assert e.kind == "MISSING_METADATA"  # a negative count is no unsigned value


def test_config_needs_the_llama_architecture():
    # registry.rs:39-55, registry_tests.rs:66-90
    e = config_error(tiny(drop=("general.architecture",)))
    assert e.kind == "MISSING_METADATA" and "general.architecture" in str(e)
    e = config_error(tiny({"general.architecture": (UINT32, 1)}))
    assert e.kind == "MISSING_METADATA"  # architecture() needs a string
    e = config_error(tiny({"general.architecture": (STRING, "gpt9")}))
    assert e.kind == "UNKNOWN_ARCHITECTURE" and "gpt9" in str(e)


def test_config_rejects_inconsistent_sizes():
    # config_tests.rs:73-185
    invalid(tiny({"llama.attention.head_count": (UINT32, 0)}), "head count must be non-zero")
    invalid(tiny({"llama.embedding_length": (UINT32, 5)}),
            "embedding length must be divisible by the head count: it must equal the head count times the "
            "head dimension")
    for kv in (3, 0):
        invalid(tiny({"llama.attention.head_count_kv": (UINT32, kv)}),
                "kv head count must be non-zero and divide the head count")
    for e in (6, 0):
        invalid(tiny({"llama.embedding_length": (UINT32, e)}), "head dimension must be even and non-zero")
    for key in ("llama.block_count", "llama.feed_forward_length", "llama.context_length"):
        invalid(tiny({key: (UINT32, 0)}), "block count, feed-forward length and context length must be non-zero")


def test_config_checks_the_rope_dimension():
    reason = "rope dimension count must equal the head dimension"
    invalid(tiny({"llama.rope.dimension_count": (UINT32, 4)}), reason)
    invalid(tiny({"llama.rope.dimension_count": (UINT64, 4)}), reason)
    tiny({"llama.rope.dimension_count": (UINT32, 2)}).decoder_config()
    tiny({"llama.rope.dimension_count": (UINT64, 2)}).decoder_config()
    invalid(tiny({"llama.rope.dimension_count": (BOOL, 1)}), "rope dimension count must be an unsigned integer")
    invalid(tiny({"llama.rope.dimension_count": (INT32, 2)}), "rope dimension count must be an unsigned integer")


def test_config_rejects_sizes_that_overflow():
    too_large = "model dimensions are too large"
    invalid(tiny({"llama.embedding_length": (UINT64, 1 << 63)}), too_large)
    invalid(tiny({"llama.embedding_length": (UINT64, 1 << 62)}), too_large)
    invalid(tiny({"llama.embedding_length": (UINT64, 1 << 32), "llama.attention.head_count": (UINT64, 1 << 16),
                  "llama.attention.head_count_kv": (UINT64, 1)}), too_large)
    invalid(tiny({"llama.feed_forward_length": (UINT64, 1 << 63)}), too_large)


def test_config_reads_the_vocabulary_from_token_embd():
    reason = "token_embd.weight must have shape [vocab, embedding length]"
    invalid(tiny(tensors={"token_embd.weight": [4]}), reason)
    invalid(tiny(tensors={"token_embd.weight": [2, 3]}), reason)
    invalid(tiny(tensors={"token_embd.weight": [0, 4]}), reason)
    w = Writer()
    for k, (tag, v) in {"general.architecture": (STRING, "llama"), "llama.embedding_length": (UINT32, 4),
                        "llama.block_count": (UINT32, 1), "llama.feed_forward_length": (UINT32, 8),
                        "llama.attention.head_count": (UINT32, 2), "llama.context_length": (UINT32, 16)}.items():
        w.kv(k, tag, v)
    e = config_error(parse(w.build()))
    assert e.kind == "MISSING_TENSOR" and "token_embd.weight" in str(e)


def test_decoder_gguf_round_trips_a_synthetic_model():
    from rusticide_amd import synth
    cfg = dict(embedding_length=256, block_count=2, feed_forward_length=512, head_count=4, head_count_kv=2,
               head_dim=64, context_length=160, vocab_size=320, rope_freq_base=10000.0, rms_norm_eps=1e-5)
    model = synth.decoder_model(cfg, seed=11)
    for align in (32, 256):
        f = parse(G.decoder_gguf(model, alignment=align))
        c = f.decoder_config()
        assert {k: c[k] for k in cfg if k not in ("rope_freq_base", "rms_norm_eps")} == \
            {k: cfg[k] for k in cfg if k not in ("rope_freq_base", "rms_norm_eps")}
        assert c["rms_norm_eps"] == float(np.float32(1e-5))
        assert f.tensor_count == 1 + 2 * 9 + 2
        t, data, rows, cols = model["blocks"][1]["ffn_down"]
        assert f.tensor_info("blk.1.ffn_down.weight")[:2] == ([rows, cols], t)
        assert f.tensor_bytes("blk.1.ffn_down.weight") == data.tobytes()
        assert np.array_equal(np.frombuffer(f.tensor_bytes("output_norm.weight"), np.float32), model["output_norm"])


def test_tokenizer_sized_metadata_parses():
    # a llama file's tokenizer arrays: 32000 strings, f32 scores, i32 types
    # (crates/rusticide-tokenizer reads them; here they are parsed and skipped)
    rng = np.random.default_rng(2)
    tokens = [bytes(rng.integers(32, 127, rng.integers(1, 12)).astype(np.uint8)).decode() for _ in range(32000)]
    w = Writer().kv("general.architecture", STRING, "llama")
    w.kv("tokenizer.ggml.model", STRING, "llama")
    w.kv("tokenizer.ggml.tokens", ARRAY, (STRING, tokens))
    w.raw_kv("tokenizer.ggml.scores", ARRAY, struct.pack("<IQ", FLOAT32, 32000) + rng.random(32000, np.float32).tobytes())
    w.raw_kv("tokenizer.ggml.token_type", ARRAY, struct.pack("<IQ", INT32, 32000) + np.ones(32000, np.int32).tobytes())
    w.kv("tokenizer.ggml.bos_token_id", UINT32, 1)
    f = parse(w.tensor("token_embd.weight", [32000, 4], F32, bytes(32000 * 16)).build())
    assert f.metadata_count == 6
    assert f.meta_type("tokenizer.ggml.tokens") == ARRAY and f.meta_uint("tokenizer.ggml.bos_token_id") == 1
    assert f.meta_string("tokenizer.ggml.model") == "llama"
