"""Hostile GGUF bytes (the idea of rusticide's GGUF-load fuzz target,
crates/rusticide-fuzz): seeded mutations of valid files must each parse or
fail with a GgufError, never crash, and whatever parses must answer its
queries within the file. Runs on the CPU; no device is involved."""

import struct

import numpy as np
import pytest

from rusticide_amd import gguf as G
from rusticide_amd.gguf import ARRAY, FLOAT32, STRING, UINT32, UINT64, GgufError, GgufFile, Writer


def seeds():
    a = (Writer().kv("general.architecture", STRING, "llama").kv("llama.block_count", UINT32, 1)
         .kv("tok", ARRAY, (STRING, ["a", "bc", "é"])).kv("n", ARRAY, (ARRAY, [(UINT64, [1, 2]), (UINT64, [])]))
         .tensor("w", [4, 256], 12, bytes(4 * 144)).tensor("n", [4], 0, struct.pack("<4f", 1, 2, 3, 4))
         .tensor("t", [128], 36, bytes(32) + struct.pack("<f", 0.5) + bytes(28)).build())
    b = Writer().alignment(64).kv("x", FLOAT32, 1.5).tensor("q", [2, 256], 14, bytes(2 * 210)).build()
    c = Writer().build()
    return [a, b, c]


def mutate(rng, data: bytes) -> bytes:
    d = bytearray(data)
    kind = rng.integers(0, 5)
    if kind == 0 and d:  # flip bits
        for _ in range(int(rng.integers(1, 8))):
            i = int(rng.integers(0, len(d)))
            d[i] ^= 1 << int(rng.integers(0, 8))
    elif kind == 1 and d:  # overwrite a little-endian word with an extreme value
        i = int(rng.integers(0, max(1, len(d) - 8)))
        extremes = [0, 1, 4, 9, 13, 0xFF, 0xFFFF, 2 ** 31, 2 ** 32 - 1, 2 ** 63, 2 ** 64 - 1]
        v = extremes[int(rng.integers(0, len(extremes)))]
        d[i:i + 8] = struct.pack("<Q", v)[: len(d[i:i + 8])]
    elif kind == 2:  # truncate
        d = d[: int(rng.integers(0, len(d) + 1))]
    elif kind == 3 and d:  # duplicate a span
        i, j = sorted(int(x) for x in rng.integers(0, len(d), 2))
        d[j:j] = d[i:j]
    else:  # random bytes inside
        i = int(rng.integers(0, len(d) + 1))
        d[i:i] = rng.integers(0, 256, int(rng.integers(1, 32))).astype(np.uint8).tobytes()
    return bytes(d)


@pytest.mark.parametrize("seed", range(4))
def test_mutated_files_parse_or_fail_cleanly(seed):
    rng = np.random.default_rng(seed)
    parsed = failed = 0
    for base in seeds():
        for _ in range(600):
            data = mutate(rng, base)
            try:
                f = GgufFile(data)
            except GgufError:
                failed += 1
                continue
            parsed += 1
            # every query stays inside the file
            for i in range(f.tensor_count):
                name, shape, type_id, offset = f.tensor_info_at(i)
                assert len(shape) <= 4
                if "\0" in name:  # reachable by index only
                    continue
                assert f.tensor_info(name) == (shape, type_id, offset)
                try:
                    raw = f.tensor_bytes(name)
                    assert len(raw) <= len(data)
                except GgufError as e:
                    assert e.gguf_kind in ("UnsupportedTensorType", "UnexpectedEof", "CastOverflow")
            for key in ("general.architecture", "llama.block_count", "x", "tok"):
                f.meta_type(key)
                f.meta_uint(key)
                f.meta_float(key)
                f.meta_string(key)
            try:
                f.decoder_config()
            except Exception as e:  # RusticideError: MISSING_*, INVALID_CONFIG, ...
                assert type(e).__name__ == "RusticideError"
            f.close()
    assert parsed and failed


def test_deep_or_huge_declarations_fail_fast():
    # lengths and counts far beyond the file fail as UnexpectedEof without
    # allocating for them
    for payload in (struct.pack("<IQ", STRING, 2 ** 62), struct.pack("<IQ", UINT32, 2 ** 63)):
        with pytest.raises(GgufError):
            GgufFile(G.header_bytes(3, 0, 1) + G.string_bytes("k") + struct.pack("<I", ARRAY) + payload)
    with pytest.raises(GgufError):
        GgufFile(G.header_bytes(3, 0, 1) + G.string_bytes("k") + struct.pack("<IQ", STRING, 2 ** 64 - 1))
