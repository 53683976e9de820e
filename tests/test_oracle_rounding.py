"""Pins on the oracle's float rounding, from exact rationals.

The k-quant dots are exact integer sums followed by a few float operations
whose order the reference fixes:

  Q4_K term  d8 * d.mul_add(isum, -(dmin * msum))   (int_dot.rs:169)
  Q6_K term  (d * d8) * isum                         (int_dot.rs:203)
  row        ((-0.0 + t0) + t1) + ...                (int_dot/rows.rs:9-12,59)

Each test builds blocks and a Q8 activation by hand, computes the expected
bits from exact rationals rounded to binary32 only where the reference
rounds, checks that the expected bits differ from those of a plausible slip
(an unfused combine, a regrouped product, a fold from +0.0, another order),
and then requires the oracle to give the expected bits. The values are
drawn from a seeded search for inputs on which the slips differ.
"""

from fractions import Fraction
import math

import numpy as np

import oracle as O

Q4_K, Q6_K = 12, 14


def f32(v: Fraction) -> Fraction:
    """Round an exact rational to the nearest binary32, ties to even
    (normal range only, which every value here stays in)."""
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = math.floor(math.log2(a.numerator) - math.log2(a.denominator))
    # settle e so that 2^e <= a < 2^(e+1)
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    assert -126 <= e <= 127
    scaled = a / Fraction(2) ** (e - 23)  # in [2^23, 2^24)
    m = scaled.numerator // scaled.denominator
    rem = scaled - m
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and m % 2 == 1):
        m += 1
    return sign * Fraction(m) * Fraction(2) ** (e - 23)


def bits32(x) -> int:
    return int(np.array(float(x), np.float32).view(np.uint32))


def f16_bits(v: float) -> int:
    return int(np.array(v, np.float16).view(np.uint16))


def f16_value(b: int) -> Fraction:
    return Fraction(float(np.array(b, np.uint16).view(np.float16)))


def q8_input(quants: np.ndarray, step: np.float32) -> O.Q8Input:
    """A Q8_K activation by hand: every 32-block scale is the super-block's step."""
    q = np.asarray(quants, np.int8)
    sums = q.reshape(-1, 32).astype(np.int32).sum(axis=1).astype(np.int32)
    scales = np.full(len(q) // 32, step, np.float32)
    return O.Q8Input(O.SUPER_BLOCK, q.copy(), scales, sums)


# ------------------------------------------------------------------ Q4_K

def q4k_block(d: int, dmin: int, sc, mn, nib) -> bytes:
    """144 bytes: f16 d, f16 dmin, the 12 scale bytes packing 6-bit scales and
    mins (q4_k.rs:17-25, get_scale_min_k4), then 128 bytes of nibbles, pair p
    holding sub-block 2p in its low and 2p+1 in its high nibbles."""
    s = bytearray(12)
    for j in range(4):
        s[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    qs = bytearray(128)
    for p in range(4):
        for l in range(32):
            qs[32 * p + l] = nib[2 * p][l] | (nib[2 * p + 1][l] << 4)
    return d.to_bytes(2, "little") + dmin.to_bytes(2, "little") + bytes(s) + bytes(qs)


def q4k_parts(rng):
    d = f16_bits(float(rng.uniform(0.002, 0.02)))
    dmin = f16_bits(float(rng.uniform(0.002, 0.02)))
    sc = [int(v) for v in rng.integers(0, 64, 8)]
    mn = [int(v) for v in rng.integers(0, 64, 8)]
    nib = [[int(v) for v in rng.integers(0, 16, 32)] for _ in range(8)]
    quants = rng.integers(-127, 128, 256)
    return d, dmin, sc, mn, nib, quants


def q4k_sums(sc, mn, nib, quants):
    isum = sum(sc[j] * sum(nib[j][l] * int(quants[32 * j + l]) for l in range(32)) for j in range(8))
    msum = sum(mn[j] * sum(int(quants[32 * j + l]) for l in range(32)) for j in range(8))
    return isum, msum


def q4k_term(d, dmin, d8, isum, msum, fused=True):
    """The block term with the reference's roundings (or an unfused slip)."""
    neg = -f32(dmin * msum)
    inner = f32(d * isum + neg) if fused else f32(f32(d * isum) + neg)
    return f32(d8 * inner)


def test_q4k_block_term_is_one_fused_multiply_add():
    rng = np.random.default_rng(169)
    for _ in range(200):
        d, dmin, sc, mn, nib, quants = q4k_parts(rng)
        step = np.float32(rng.uniform(0.01, 0.05))
        isum, msum = q4k_sums(sc, mn, nib, quants)
        D, M, S = f16_value(d), f16_value(dmin), Fraction(float(step))
        want = q4k_term(D, M, S, isum, msum)
        slips = {q4k_term(D, M, S, isum, msum, fused=False),  # d*isum rounded first
                 f32(f32(S * f32(D * isum)) - f32(S * f32(M * msum))),  # d8 distributed
                 f32(f32(S * D) * isum + -f32(S * f32(M * msum)))}  # d8 folded into d
        if want in slips:
            continue  # these inputs cannot tell the slips apart
        got = O.dot_row(Q4_K, q4k_block(d, dmin, sc, mn, nib), q8_input(quants, step))
        assert bits32(got) == bits32(want), (float(got), float(want))
        return
    raise AssertionError("no input separated the fused combine from its slips")


# ------------------------------------------------------------------ Q6_K

def q6k_block(q, scales, d: int) -> bytes:
    """210 bytes: ql[128], qh[64], scales[16] i8, f16 d (q6_k.rs:13-43). Element
    e = 128h + 32r + l takes its low nibble from ql[64h + 32(r&1) + l] (high
    half of the byte for r >= 2) and bits 2r..2r+1 of qh[32h + l]."""
    ql, qh = bytearray(128), bytearray(64)
    for h in range(2):
        for r in range(4):
            for l in range(32):
                v = q[128 * h + 32 * r + l]
                i = 64 * h + 32 * (r & 1) + l
                ql[i] |= (v & 15) << (4 if r >= 2 else 0)
                qh[32 * h + l] |= (v >> 4) << (2 * r)
    return bytes(ql) + bytes(qh) + bytes(np.asarray(scales, np.int8).tobytes()) + d.to_bytes(2, "little")


def q6k_isum(q, scales, quants):
    return sum(int(scales[e // 16]) * (q[e] - 32) * int(quants[e]) for e in range(256))


def test_q6k_block_term_rounds_d_times_d8_first():
    rng = np.random.default_rng(203)
    for _ in range(200):
        q = [int(v) for v in rng.integers(0, 64, 256)]
        scales = rng.integers(-32, 32, 16)
        d = f16_bits(float(rng.uniform(0.001, 0.01)))
        quants = rng.integers(-127, 128, 256)
        step = np.float32(rng.uniform(0.01, 0.05))
        isum = q6k_isum(q, scales, quants)
        D, S = f16_value(d), Fraction(float(step))
        want = f32(f32(D * S) * isum)
        slips = {f32(D * f32(S * isum)), f32(S * f32(D * isum))}
        if want in slips:
            continue
        got = O.dot_row(Q6_K, q6k_block(q, scales, d), q8_input(quants, step))
        assert bits32(got) == bits32(want), (float(got), float(want))
        return
    raise AssertionError("no input separated (d*d8)*isum from its regroupings")


# ------------------------------------------------------------------- rows

def test_a_row_of_negative_zero_terms_sums_to_negative_zero():
    # every block term -0.0: the fold from -0.0 keeps the sign, a fold from
    # +0.0 would not ((+0.0) + (-0.0) == +0.0)
    step = np.float32(0.03125)
    neg_d = f16_bits(-0.5)
    # Q6_K: every q = 32 makes isum = 0, and (d*d8) < 0 gives (d*d8)*0 = -0.0
    row6 = b"".join(q6k_block([32] * 256, [7] * 16, neg_d) for _ in range(4))
    # Q4_K: zero nibbles and mins make isum = msum = 0; d < 0 gives
    # d.mul_add(0, -(dmin*0)) = -0.0, and d8 * -0.0 = -0.0
    zero = [[0] * 32 for _ in range(8)]
    row4 = b"".join(q4k_block(neg_d, f16_bits(0.25), [5] * 8, [0] * 8, zero) for _ in range(4))
    quants = np.random.default_rng(12).integers(-127, 128, 4 * 256)
    for type_id, row in ((Q6_K, row6), (Q4_K, row4)):
        got = O.dot_row(type_id, row, q8_input(quants, step))
        assert bits32(got) == 0x80000000, (type_id, hex(bits32(got)))


def test_row_terms_are_added_in_block_order():
    # eight Q6_K blocks whose terms span magnitudes, so that the sequential
    # fold differs from a pairwise or a reversed one
    rng = np.random.default_rng(59)
    for _ in range(200):
        blocks, terms = [], []
        quants = rng.integers(-127, 128, 8 * 256)
        step = np.float32(rng.uniform(0.01, 0.05))
        for b in range(8):
            q = [int(v) for v in rng.integers(0, 64, 256)]
            scales = rng.integers(-32, 32, 16)
            d = f16_bits(float(rng.uniform(0.001, 0.01)) * (1000.0 if b % 3 == 0 else 1.0))
            blocks.append(q6k_block(q, scales, d))
            isum = q6k_isum(q, scales, quants[256 * b:256 * (b + 1)])
            terms.append(f32(f32(f16_value(d) * Fraction(float(step))) * isum))
        seq = Fraction(0)
        for t in terms:
            seq = f32(seq + t)
        rev = Fraction(0)
        for t in reversed(terms):
            rev = f32(rev + t)
        pair = terms[:]
        while len(pair) > 1:
            pair = [f32(pair[i] + pair[i + 1]) for i in range(0, len(pair), 2)]
        if seq in (rev, pair[0]):
            continue
        got = O.dot_row(Q6_K, b"".join(blocks), q8_input(quants, step))
        assert bits32(got) == bits32(seq), (float(got), float(seq))
        return
    raise AssertionError("no input separated the sequential fold from other orders")
