"""Pins the CPU oracle before it is trusted as the checker.

Three kinds of evidence, none of which retypes the oracle's own formula:

* the reference's known-answer tests, transcribed with their literal expected
  values (file:line cited on each test);
* exact-arithmetic identities: inputs chosen so every float operation is exact,
  where the integer-dot kernels must equal the dequantized operands' dot
  product computed with Python fractions;
* brute force on tiny inputs and independent decoders written from the format
  description (the ggml block layouts), checked against the KATs first.
"""

from fractions import Fraction

import numpy as np
import pytest

import oracle as O


def f16_bytes(v: float) -> bytes:
    return int(np.array(v, np.float16).view(np.uint16)).to_bytes(2, "little")


def bits(a) -> list:
    return [int(x) for x in np.asarray(a, np.float32).view(np.uint32)]


# ------------------------------------------------------------------ formats


def test_format_table():
    # quantize/src/format.rs:52-91; quant_kernel_tests.rs:33-53
    assert O.block_format(12) == (256, 144, 0)
    assert O.block_format(14) == (256, 210, 0)
    assert O.block_format(36) == (128, 32, 32)
    assert O.block_format(99) is None


def test_i2s_sizes():
    # quantize/src/i2_s.rs:106-116
    assert O.byte_len(36, 6_553_600) == 1_638_432
    assert O.byte_len(36, 0) == 32
    assert O.row_bytes(36, 2560) == 640
    # survey table: Q4_K row(2048)=1152, Q6_K row(2048)=1680, row(5632)=4620
    assert O.row_bytes(12, 2048) == 1152
    assert O.row_bytes(14, 2048) == 1680
    assert O.row_bytes(14, 5632) == 4620
    assert O.row_bytes(12, 100) is None


def test_f16_widening_is_exact_for_all_65536_values():
    # rusticide-simd/src/scalar.rs:75-86 checks f16_to_f32 against `half`;
    # numpy's float16 widening is the same IEEE operation.
    allbits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = allbits.view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32(int(b)) for b in allbits], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_rounds_to_nearest_even():
    rng = np.random.default_rng(5)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504.0, 65520.0, 1e-8, 2.0 ** -25, 2.0 ** -24, 0.01, 0.07], np.float32),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    got = np.array([O.f32_to_f16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, want)


# ---------------------------------------------------------- Q4_K decode KATs


def test_q4k_zero_scale_yields_negative_min():
    # quantize/src/q4_k.rs:84-95
    block = bytearray(144)
    block[2:4] = f16_bytes(1.0)
    block[4 + 4] = 1
    out = O.dequantize_row(12, block)
    assert np.all(np.abs(out[:32] - -1.0) < 1e-4)


def test_q4k_full_block_uses_every_sub_block_pair():
    # quantize/src/q4_k.rs:97-122
    block = bytearray(144)
    block[0:2] = f16_bytes(1.0)
    block[2:4] = f16_bytes(1.0)
    block[4:8] = bytes([1, 2, 3, 4])
    block[8:12] = bytes([8, 7, 6, 5])
    block[12:16] = bytes([0x45, 0x36, 0x27, 0x18])
    block[16:] = bytes([0x32] * 128)
    out = O.dequantize_row(12, block)
    for sb in range(8):
        scale = sb + 1.0
        quant = 2.0 if sb % 2 == 0 else 3.0
        want = scale * quant - (8.0 - sb)
        for l in (0, 31):
            assert abs(out[sb * 32 + l] - want) < 1e-4


def test_q4k_scale_min_upper_sub_blocks():
    # quantize/src/q4_k.rs:124-132: q4_k_scale_min(4) == (53, 26), (0) == (0, 0)
    block = bytearray(144)
    block[0:2] = f16_bytes(1.0)
    block[2:4] = f16_bytes(1.0)
    block[4 + 0] = 0xC0
    block[4 + 4] = 0x40
    block[4 + 8] = 0xA5
    block[16:] = bytes([0x11] * 128)  # q = 1 everywhere
    out = O.dequantize_row(12, block)
    assert out[4 * 32] == 53.0 * 1 - 26.0
    assert out[0] == 0.0


# ---------------------------------------------------------- Q6_K decode KATs


def test_q6k_all_zero_quants_dequantize_to_minus_32():
    # quantize/src/q6_k.rs:57-68
    block = bytearray(210)
    block[192:208] = bytes([1] * 16)
    block[208:210] = f16_bytes(1.0)
    assert np.all(O.dequantize_row(14, block) == -32.0)


def test_q6k_high_bits_scales_and_second_half():
    # quantize/src/q6_k.rs:83-104
    block = bytearray(210)
    block[0] = 0x05
    block[128] = 0b10
    block[128] |= 0b01 << 2
    block[64] = 0x03
    block[128 + 32] = 0b10
    block[192 + 8] = 2
    block[192] = 3
    block[192 + 2] = 4
    block[208:210] = f16_bytes(1.0)
    out = O.dequantize_row(14, block)
    assert (out[0], out[32], out[128]) == (15.0, -64.0, 6.0)


def test_q6k_every_quadrant_scale_and_scale_group():
    # quantize/src/q6_k.rs:133-163
    block = bytearray(210)
    scales = [(-6 if i == 5 else i + 1) for i in range(16)]
    for i, s in enumerate(scales):
        block[192 + i] = s & 0xFF
    block[208:210] = f16_bytes(1.0)
    for h in range(2):
        for l in (0, 16):
            block[h * 64 + l] = 0x21
            block[h * 64 + l + 32] = 0x43
            block[128 + h * 32 + l] = 0b1110_0100
    out = O.dequantize_row(14, block)
    for h in range(2):
        for l in (0, 16):
            group = h * 8 + l // 16
            at = lambda quad: out[h * 128 + l + 32 * quad]
            assert at(0) == scales[group + 0] * -31.0
            assert at(1) == scales[group + 2] * -13.0
            assert at(2) == scales[group + 4] * 2.0
            assert at(3) == scales[group + 6] * 20.0


# ---------------------------------------------------------- I2_S decode KATs


def packed_i2s(code):
    return bytes(code(k) << 6 | code(k + 32) << 4 | code(k + 64) << 2 | code(k + 96) for k in range(32))


def test_i2s_byte_k_holds_weights_k_to_k_plus_96():
    # quantize/src/i2_s.rs:88-94
    code = lambda i: i % 3
    out = O.dequantize_row(36, packed_i2s(code))
    assert list(out) == [code(i) - 1.0 for i in range(128)]


def test_i2s_code_three_decodes_to_plus_two():
    # quantize/src/i2_s.rs:96-104
    block = bytearray(32)
    block[0] = 0b00_01_10_11
    out = O.dequantize_row(36, block)
    assert [out[0], out[32], out[64], out[96]] == [-1.0, 0.0, 1.0, 2.0]
    assert out[1] == -1.0


# --------------------------------------------------------------- generators


def test_lcg_generators_match_their_closed_form():
    # format.rs:109-117, test_support.rs:72-80, bench/src/kernels.rs:27-35
    state, want_b, want_v, want_a = 7, [], [], []
    for _ in range(50):
        state = (state * 1_664_525 + 1_013_904_223) & 0xFFFFFFFF
        want_b.append(state >> 24)
        want_v.append(np.float32(state >> 24) / np.float32(128.0) - np.float32(1.0))
        want_a.append(np.float32(state >> 16) / np.float32(32768.0) - np.float32(1.0))
    assert list(O.pseudo_random_bytes(50, 7)) == want_b
    assert bits(O.pseudo_random_values(50, 7)) == bits(want_v)
    assert bits(O.bench_activations(50, 7)) == bits(want_a)


def test_synthetic_blocks_set_every_scale_field():
    # format.rs:204-214: scales 0.01..0.07 in turn at offsets [0,2] / [208]
    q4 = O.synthetic_blocks(12, 9, 1).reshape(9, 144)
    q6 = O.synthetic_blocks(14, 9, 1).reshape(9, 210)
    raw4 = O.pseudo_random_bytes(9 * 144, 1).reshape(9, 144)
    for i in range(9):
        want = f16_bytes([0.01, 0.02, 0.03, 0.04, 0.05, 0.06, 0.07][i % 7])
        assert bytes(q4[i, 0:2]) == want and bytes(q4[i, 2:4]) == want
        assert bytes(q6[i, 208:210]) == want
        assert bytes(q4[i, 4:]) == bytes(raw4[i, 4:])


# ------------------------------------------------------------ quantizer KATs


def test_super_block_shares_one_signed_scale():
    # kernels/src/q8_input_tests.rs:60-76
    x = np.zeros(256, np.float32)
    x[0], x[40], x[255] = 1.0, -2.0, 0.5
    q = O.quantize(x, O.SUPER_BLOCK)
    scale = np.float32(1.0) / (np.float32(-127.0) / np.float32(-2.0))
    assert bits(q.scales) == bits([scale] * 8)
    assert (q.quants[0], q.quants[40], q.quants[255]) == (64, -127, 32)
    assert (q.sums[0], q.sums[1]) == (64, -127)


def test_all_zero_super_block_has_zero_scale():
    # kernels/src/q8_input_tests.rs:78-83
    q = O.quantize(np.zeros(256, np.float32), O.SUPER_BLOCK)
    assert list(q.scales) == [0.0] * 8


def test_super_block_drops_partial_super_blocks():
    # portable/q8.rs:67-70 and q8_input_tests.rs:34-41
    assert len(O.quantize(np.ones(300, np.float32), O.SUPER_BLOCK)) == 256
    assert len(O.quantize(np.zeros(0, np.float32), O.SUPER_BLOCK)) == 0


def test_super_block_first_max_wins_on_a_tie():
    # portable/q8.rs:19-33: the first element with |v| == amax sets the sign
    # and always maps to -127; the scale carries its sign.
    x = np.zeros(256, np.float32)
    x[3], x[7] = -2.0, 2.0
    q = O.quantize(x, O.SUPER_BLOCK)
    assert (q.quants[3], q.quants[7]) == (-127, 127) and q.scales[0] > 0
    x[3], x[7] = 2.0, -2.0
    q = O.quantize(x, O.SUPER_BLOCK)
    assert (q.quants[3], q.quants[7]) == (-127, 127) and q.scales[0] < 0


def row(head):
    v = np.zeros(32, np.float32)
    v[: len(head)] = head
    return v


def nearest_int(value: np.float32) -> int:
    # kernels/src/q8_input_tests.rs:98-102: ggml's 12582912 trick
    b = int(np.array(np.float32(value) + np.float32(12_582_912.0), np.float32).view(np.int32))
    return (b & 0x007F_FFFF) - 0x0040_0000


def reference_row(values):
    # kernels/src/q8_input_tests.rs:104-118 (bitnet.cpp quantize_row_i8_s)
    mx = 1e-5
    for v in values:
        mag = float(abs(np.float32(v)))
        mx = mx if mx > mag else mag
    scale = np.float32(127.0 / mx)
    quants = [max(-128, min(127, nearest_int(np.float32(v) * scale))) for v in values]
    return scale, quants


def test_row_scale_follows_the_legacy_formula():
    # kernels/src/q8_input_tests.rs:120-130
    q = O.quantize(np.concatenate([row([0.5, -2.0, 1.0]), row([])]), O.ROW)
    assert bits(q.scales) == bits([np.float32(127.0 / 2.0)] * 2)
    assert list(q.quants[:3]) == [32, -127, 64]
    assert list(q.sums) == [-31, 0]


def test_all_zero_row_quantizes_to_zeros():
    # kernels/src/q8_input_tests.rs:132-140
    q = O.quantize(row([]), O.ROW)
    assert bits(q.scales) == bits([np.float32(127.0 / 1e-5)])
    assert not q.quants.any() and list(q.sums) == [0]


def test_row_halfway_rounds_to_even():
    # kernels/src/q8_input_tests.rs:142-149
    values = row([127.0, 2.5, 3.5, -2.5, -3.5])
    q = O.quantize(values, O.ROW)
    assert list(q.scales) == [1.0]
    assert list(q.quants[:5]) == [127, 2, 4, -2, -4]
    assert reference_row(values)[1] == list(q.quants)


def test_row_clamps_to_i8_and_nan_to_zero():
    # kernels/src/q8_input_tests.rs:151-158
    values = row([-4.0, float("nan"), 1.0])
    q = O.quantize(values, O.ROW)
    assert list(q.scales) == [127.0]
    assert list(q.quants[:3]) == [-128, 0, 127]
    s, quants = reference_row(values)
    assert s == 127.0 and quants == list(q.quants)


def test_row_sums_are_the_block_quant_sums():
    # kernels/src/q8_input_tests.rs:160-175
    values = (O.pseudo_random_values(256, 3) * np.float32(3.7)).astype(np.float32)
    q = O.quantize(values, O.ROW)
    assert list(q.sums) == [int(q.quants[i:i + 32].astype(np.int32).sum()) for i in range(0, 256, 32)]
    s, quants = reference_row(values)
    assert bits(q.scales) == bits([s] * 8) and list(q.quants) == quants


def test_row_dequantize_divides_by_the_scale():
    # kernels/src/q8_input_tests.rs:177-183
    q = O.quantize(row([0.5, -2.0, 1.0]), O.ROW)
    want = q.quants.astype(np.float32) / q.scales[0]
    assert bits(q.dequantize()) == bits(want)


# ------------------------------------------------------------ integer dots


@pytest.mark.parametrize("type_id,seed", [(12, 3), (14, 4)])
def test_dot_row_matches_the_dequantized_operands(type_id, seed):
    # kernels/src/quant_kernel_tests.rs:60-79 (seeds follow the format order)
    rowdata = O.synthetic_blocks(type_id, 2, seed)
    q = O.quantize(O.pseudo_random_values(512, seed + 100), O.SUPER_BLOCK)
    values = O.dequantize_row(type_id, rowdata)
    expected = np.float32(0.0)
    for a, b in zip(values, q.dequantize()):
        expected = np.float32(expected + np.float32(a * b))
    got = O.dot_row(type_id, rowdata, q)
    tol = 1e-4 * max(1.0, float(np.abs(values).sum()))
    assert abs(got - expected) <= tol


def _exact_activation(rng, n):
    """Values k/64 with the first max +127/64: Q8_K maps them to q = -k with
    step -1/64 exactly, so the dequantized activation equals the input."""
    k = rng.integers(-126, 127, n)
    k[::256] = 127  # the first element of every super-block is its max
    return (k.astype(np.float32) / np.float32(64.0)).astype(np.float32), k


@pytest.mark.parametrize("type_id", [12, 14])
def test_integer_dot_equals_exact_dequantized_dot(type_id):
    """Exact identity: with power-of-two d, dmin and d8 every float step of the
    integer kernel is exact, so it must equal sum(w_i * x_i) in rationals."""
    rng = np.random.default_rng(type_id)
    nblocks = 4
    bb = 144 if type_id == 12 else 210
    data = bytearray(rng.integers(0, 256, nblocks * bb, dtype=np.uint8).tobytes())
    for b in range(nblocks):
        if type_id == 12:
            data[b * bb:b * bb + 2] = f16_bytes(2.0 ** -4)
            data[b * bb + 2:b * bb + 4] = f16_bytes(2.0 ** -5)
        else:
            data[b * bb + 208:b * bb + 210] = f16_bytes(2.0 ** -3)
    x, k = _exact_activation(rng, nblocks * 256)
    q = O.quantize(x, O.SUPER_BLOCK)
    assert list(q.quants) == list(-k) and q.scales[0] == np.float32(-1.0 / 64.0)
    w = O.dequantize_row(type_id, bytes(data))
    exact = sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(w, x))
    assert Fraction(O.dot_row(type_id, bytes(data), q)) == exact


def test_q4k_integer_dot_on_the_reference_1x256_matrix():
    # kernels/src/matmul_tests.rs:39-46,135-149: q4_k_data() against f(v%13)-6
    data = f16_bytes(1.0) + f16_bytes(0.5) + bytes([3] * 12) + bytes((v * 37) & 0xFF for v in range(128))
    x = np.array([(v % 13) - 6.0 for v in range(256)], np.float32)
    q = O.quantize(x, O.SUPER_BLOCK)
    got = O.dot_row(12, data, q)
    w = O.dequantize_row(12, data)
    exact = float(sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(w, q.dequantize())))
    assert abs(got - exact) <= 1e-4 * float(np.abs(w).sum())


def test_dot_f32_known_vectors():
    # rusticide-simd/src/float.rs:74-88,154-158
    assert O.dot_f32([1, 2, 3], [4, 5, 6]) == 32.0
    assert O.dot_f32(np.arange(1, 20, dtype=np.float32), np.ones(19, np.float32)) == 190.0
    assert O.dot_f32([1, 2, 3], [1, 1]) == 3.0
    assert O.dot_f32(np.ones(12), np.ones(24)) == 12.0


def test_dot_f32_is_eight_fused_lanes_then_the_tail():
    # float.rs:23-36, brute force in f64 on a case where fusing matters
    rng = np.random.default_rng(1)
    a = rng.standard_normal(37).astype(np.float32)
    b = rng.standard_normal(37).astype(np.float32)
    lanes = [np.float32(0.0)] * 8
    for c in range(4):
        for i in range(8):
            lanes[i] = np.float32(float(a[8 * c + i]) * float(b[8 * c + i]) + float(lanes[i]))
    tail = np.float32(-0.0)
    for i in range(32, 37):
        tail = np.float32(tail + np.float32(a[i] * b[i]))
    s = np.float32(-0.0)
    for v in lanes:
        s = np.float32(s + v)
    assert bits([O.dot_f32(a, b)]) == bits([np.float32(s + tail)])


# --------------------------------------------------------------- ternary


def ternary_rows(blocks, seed):
    # kernels/src/test_support.rs:84-92
    return O.pseudo_random_bytes(blocks * 32, seed)


def naive_ternary_dot(rowdata, q):
    # kernels/src/test_support.rs:100-110: from the format's own decoder
    values = O.dequantize_row(36, rowdata)
    n = min(len(values), len(q.quants))
    return int(sum(int(values[i]) * int(q.quants[i]) for i in range(n)))


def test_ternary_dot_equals_a_naive_integer_dot():
    # portable/ternary_tests.rs:15-24
    for seed in range(1, 6):
        r = ternary_rows(5, seed)
        assert {int(b) >> 6 for b in r} >= {0, 1, 2, 3}
        q = O.quantize(O.pseudo_random_values(640, seed + 50), O.ROW)
        assert O.ternary_dot(r, q) == naive_ternary_dot(r, q)


def test_code_three_counts_as_plus_two():
    # portable/ternary_tests.rs:26-33
    q = O.quantize(O.pseudo_random_values(128, 7), O.ROW)
    total = int(q.quants.astype(np.int32).sum())
    assert total != 0
    assert O.ternary_dot(bytes([0xFF] * 32), q) == 2 * total
    assert O.ternary_dot(bytes([0x55] * 32), q) == 0


def test_the_shorter_operand_bounds_the_ternary_dot():
    # portable/ternary_tests.rs:35-47
    r = ternary_rows(3, 9)
    q = O.quantize(O.pseudo_random_values(256, 10), O.ROW)
    assert O.ternary_dot(r, q) == naive_ternary_dot(r[:64], q)
    assert O.ternary_dot(r[:40], q) == naive_ternary_dot(r[:32], q)


def test_a_hostile_width_wraps_rather_than_panics():
    # portable/ternary_tests.rs:49-62
    blocks = (1 << 31) // (254 * 128) + 1
    q = O.Q8Input(O.ROW, np.full(blocks * 128, 127, np.int8), np.ones(blocks * 4, np.float32),
                  np.full(blocks * 4, 127 * 32, np.int32))
    exact = 254 * 128 * blocks
    assert exact > 2 ** 31 - 1
    assert O.ternary_dot(bytes([0xFF] * (blocks * 32)), q) == exact - (1 << 32)


def test_ternary_matrix_scales_each_row_and_token_in_the_legacy_order():
    # portable/ternary_tests.rs:73-88
    data = ternary_rows(6, 3)
    qs = [O.quantize(O.pseudo_random_values(256, s), O.ROW) for s in (4, 5)]
    for r in range(3):
        for q in qs:
            want = np.float32(np.float32(naive_ternary_dot(data[64 * r:64 * r + 64], q)) / q.scales[0]) * np.float32(1.25)
            assert bits([O.ternary_product(data[64 * r:64 * r + 64], q, 1.25)]) == bits([want])


def test_a_zero_ternary_row_is_exactly_zero():
    # portable/ternary_tests.rs:90-95
    q = O.quantize(O.pseudo_random_values(128, 8), O.ROW)
    assert bits([O.ternary_product(bytes([0x55] * 32), q, 3.0)]) == [0]
    empty = O.quantize(np.zeros(0, np.float32), O.ROW)
    assert bits([O.ternary_product(bytes([0xFF] * 32), empty, 1.0)]) == [0]


def test_i2s_matvec_is_the_integer_dot_over_s_times_the_scale():
    # model/src/weights_ternary_tests.rs:69-90: divisor exactly 2
    data = bytes([0b1010_1010] * 32 + [0b0001_1011] * 32)
    quants = [127 - 2 * i for i in range(128)]
    x = np.array([k / 2.0 for k in quants], np.float32)
    lanes = lambda v: [c for c in v for _ in range(32)]
    weights = [lanes([1.0] * 4), lanes([-1.0, 0.0, 1.0, 2.0])]
    want = [np.float32(np.float32(sum(w * q for w, q in zip(wr, quants))) / np.float32(2.0)) * np.float32(0.75)
            for wr in weights]
    out = np.full(2, np.nan, np.float32)
    O.matvec_batch(x, [(O.Weights.ternary(data, 32, 0.75), out)])
    assert bits(out) == bits(want) and want[1] != 0


# -------------------------------------------------------------- scheduler


def test_matmul_batch_layout_and_token_identity():
    # kernels/src/matmul_tests.rs:151-186 and :237-271 (batch == per token)
    rng = np.random.default_rng(2)
    for type_id in (12, 14):
        rows, cols, tokens = 37, 512, 3
        rb = O.row_bytes(type_id, cols)
        data = O.synthetic_blocks(type_id, rows * cols // 256, 11)
        x = rng.standard_normal(tokens * cols).astype(np.float32)
        out = np.full(rows * tokens, np.nan, np.float32)
        O.matmul_batch(x, tokens, [(O.Weights.blocks(type_id, data, rb), out)], threads=4)
        for t in range(tokens):
            single = np.full(rows, np.nan, np.float32)
            O.matvec_batch(x[t * cols:(t + 1) * cols], [(O.Weights.blocks(type_id, data, rb), single)])
            assert bits(out[t::tokens]) == bits(single)
            q = O.quantize(x[t * cols:(t + 1) * cols], O.SUPER_BLOCK)
            assert bits(single[:2]) == bits([O.dot_row(type_id, data[r * rb:(r + 1) * rb], q) for r in range(2)])


def test_matmul_batch_no_ops():
    # kernels/src/matmul_tests.rs:188-235
    data = O.synthetic_blocks(12, 2, 1)
    out = np.full(2, 7.0, np.float32)
    w = O.Weights.blocks(12, data, 144)
    O.matmul_batch(np.ones(256, np.float32), 0, [(w, out)])
    O.matmul_batch(np.ones(256, np.float32), 257, [(w, out)])
    O.matmul_batch(np.zeros(0, np.float32), 1, [(w, out)])
    assert list(out) == [7.0, 7.0]
    empty = np.full(2, 7.0, np.float32)
    O.matvec_batch(np.ones(256, np.float32), [(O.Weights.blocks(12, b"", 0), empty)])
    assert list(empty) == [7.0, 7.0]


def test_short_output_bounds_the_rows():
    # matmul.rs:239-244 + quant_kernel.rs:106-111: out.len() bounds the rows
    data = O.synthetic_blocks(12, 4, 2)
    x = O.pseudo_random_values(256, 3)
    full = np.zeros(4, np.float32)
    O.matvec_batch(x, [(O.Weights.blocks(12, data, 144), full)])
    short = np.full(3, np.nan, np.float32)
    O.matvec_batch(x, [(O.Weights.blocks(12, data, 144), short)])
    assert bits(short) == bits(full[:3])
