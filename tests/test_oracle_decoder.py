"""The CPU restatement of rusticide's decoder, pinned by the reference's own
known answers and invariants before it serves as the device decoder's checker.
"""

import numpy as np
import pytest

import oracle as O
from rusticide_amd import synth

TINY = dict(embedding_length=256, block_count=2, feed_forward_length=512, head_count=4, head_count_kv=2,
            head_dim=64, context_length=16, vocab_size=320, rope_freq_base=10000.0, rms_norm_eps=1e-5)


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_rms_norm_divides_by_root_mean_square():
    # portable/norm.rs:38-44: [1,2,3,4] / sqrt(7.5), eps 0, then x weight 1
    out = O.normalize([1, 2, 3, 4], [1, 1, 1, 1], 0.0)
    rms = np.float32(np.sqrt(np.float32(7.5)))
    assert np.array_equal(bits(out), bits(np.array([1, 2, 3, 4], np.float32) / rms))


def test_normalize_applies_the_weight_after_the_norm():
    # transformer/src/norm.rs:10-14
    x = np.array([3.0, -4.0], np.float32)
    out = O.normalize(x, [2.0, 0.5], 0.0)
    rms = np.float32(np.sqrt(np.float32(12.5)))
    assert np.array_equal(bits(out), bits(np.array([(x[0] / rms) * 2.0, (x[1] / rms) * 0.5], np.float32)))


def test_softmax_sums_to_one_and_survives_large_inputs():
    # portable/norm.rs:54-58
    assert np.array_equal(O.softmax([1000.0, 1000.0]), np.array([0.5, 0.5], np.float32))
    p = O.softmax([1.0, 2.0, 3.0])
    assert abs(float(p.sum()) - 1.0) < 1e-6 and p[2] > p[1] > p[0]


def test_rope_adjacent_known_answers():
    # portable/rope.rs:38-70
    row = O.rope_adjacent([1.0, 0.0, 1.0, 0.0], 1, 10000.0, 2)
    slow = np.float32(10000.0) ** np.float32(-2.0 / 4.0)
    np.testing.assert_allclose(row, [np.cos(1.0), np.sin(1.0), np.cos(slow), np.sin(slow)], rtol=1e-6)
    assert np.array_equal(O.rope_adjacent([1, 2, 3, 4], 0, 10000.0, 2), np.array([1, 2, 3, 4], np.float32))
    np.testing.assert_allclose(O.rope_adjacent([1.0, 0.0, 1.0, 0.0], 1, 10000.0, 1),
                               [np.cos(1.0), np.sin(1.0), 1.0, 0.0], rtol=1e-6)
    assert O.rope_adjacent([1.0, 0.0, 7.0], 1, 10000.0, 4)[2] == 7.0


def test_rope_table_is_the_rotation_the_kernel_applies():
    # the table the device reads holds exactly the angles rope_adjacent uses
    cos, sin = O.rope_table(9, 64, 10000.0)
    rng = np.random.default_rng(2)
    for pos in (0, 3, 8):
        row = rng.standard_normal(64).astype(np.float32)
        want = O.rope_adjacent(row, pos, 10000.0, 32)
        c, s = cos[pos * 32:(pos + 1) * 32], sin[pos * 32:(pos + 1) * 32]
        lo, hi = row[0::2].astype(np.float64), row[1::2].astype(np.float64)
        got = np.empty(64, np.float32)
        # fma(lo, c, -(hi*s)) and fma(hi, c, lo*s), evaluated exactly in f64
        hs = (row[1::2] * s).astype(np.float64)
        ls = (row[0::2] * s).astype(np.float64)
        got[0::2] = (lo * c.astype(np.float64) - hs).astype(np.float32)
        got[1::2] = (hi * c.astype(np.float64) + ls).astype(np.float32)
        assert np.array_equal(bits(got), bits(want))


def test_greedy_keeps_the_last_maximum_and_skips_nan():
    # sampling/src/filters.rs:37-43 (max_by keeps the last), sampler.rs:75-87
    assert O.greedy([1.0, 3.0, 3.0, 2.0]) == 2
    assert O.greedy([np.nan, 0.5, np.nan]) == 1
    assert O.greedy([-0.0, 0.0]) == 1  # total order: +0 above -0
    assert O.greedy([0.0, -0.0]) == 0
    with pytest.raises(O.DecoderError) as e:
        O.greedy([np.nan, np.nan])
    assert e.value.kind == "NO_VALID_TOKENS"
    with pytest.raises(O.DecoderError):
        O.greedy([np.inf, -np.inf])


@pytest.fixture(scope="module")
def tiny():
    return synth.decoder_model(TINY, seed=5)


def test_batches_match_one_token_at_a_time_bit_for_bit(tiny):
    # transformer/src/decoder_batch_tests.rs:50-66
    d = O.Decoder(tiny, threads=4)
    tokens = [3, 1, 4, 1, 5, 9, 2, 6]
    expected = []
    for i, t in enumerate(tokens):
        expected.append(d.forward(t, i))
    d.reset()
    first = d.forward_batch(tokens[:3], 0)
    second = d.forward_batch(tokens[3:7], 3)
    assert np.array_equal(bits(first), bits(expected[2]))
    assert np.array_equal(bits(second), bits(expected[6]))
    last = d.forward(tokens[7], 7)
    assert np.array_equal(bits(last), bits(expected[7]))
    assert not np.array_equal(bits(expected[6]), bits(expected[7]))


def test_decoder_errors_leave_the_cache_alone(tiny):
    # decoder_batch_tests.rs:74-120
    d = O.Decoder(tiny, threads=2)
    with pytest.raises(O.DecoderError) as e:
        d.forward_batch([1, TINY["vocab_size"]], 0)
    assert e.value.kind == "TOKEN_RANGE"
    with pytest.raises(O.DecoderError) as e:
        d.forward_batch(list(range(17)), 0)
    assert e.value.kind == "CONTEXT_FULL"
    d.forward_batch([1, 2], 0)
    with pytest.raises(O.DecoderError) as e:
        d.forward_batch([3], 3)
    assert e.value.kind == "CACHE_POSITION"
    with pytest.raises(O.DecoderError) as e:
        d.forward_batch([], 2)
    assert e.value.kind == "NO_TOKENS"
    # the cache still holds positions 0..2: position 2 continues it
    d.forward_batch([3], 2)


def test_generation_prefills_in_chunks_and_stops_at_the_context(tiny):
    # generate.rs:70-111: prefill chunks of 64 equal one token at a time; the
    # loop stops after the pick at the context end
    d = O.Decoder(tiny, threads=2)
    prompt = [7, 8, 9, 10, 11]
    got = d.generate_greedy(prompt, 50)
    assert len(got) == TINY["context_length"] - len(prompt) + 1
    d.reset()
    logits = None
    for i, t in enumerate(prompt):
        logits = d.forward(t, i)
    seq, pos = [], len(prompt)
    for _ in range(len(got)):
        nxt = O.greedy(logits)
        seq.append(nxt)
        if pos == TINY["context_length"]:
            break
        logits = d.forward(nxt, pos)
        pos += 1
    assert np.array_equal(got, np.array(seq, np.uint32))
    with pytest.raises(O.DecoderError):
        d.generate_greedy(list(range(16)), 3)


def test_dot_rows_known_answers():
    # float.rs:91-112: stride windows, offsets past the row or overflowing
    rows = [1.0, 2.0, 9.0, 3.0, 4.0, 9.0]
    assert O.dot_rows([1.0, 1.0], rows, 3, 0, 2.0, 2).tolist() == [1.5, 3.5]
    assert O.dot_rows([1.0], rows, 3, 2, 1.0, 2).tolist() == [9.0, 9.0]
    assert O.dot_rows([1.0], [1.0, 2.0], 2, 5, 1.0, 1).tolist() == [0.0]
    assert O.dot_rows([1.0], [1.0, 2.0], 2, 2 ** 64 - 1, 1.0, 1).tolist() == [0.0]


def test_dot_rows_scores_each_head_window_of_a_wide_row():
    # float.rs:160-172 shape: 48 values as two 24-wide rows, 12-wide heads
    rows = np.arange(1, 49, dtype=np.float32)
    q = np.ones(12, np.float32)
    for offset in (0, 12):
        want = [float(np.sum(rows[i * 24 + offset:i * 24 + offset + 12])) for i in range(2)]
        assert O.dot_rows(q, rows, 24, offset, 1.0, 2).tolist() == want


def test_mix_rows_known_answers():
    # float.rs:115-151
    rows = [1.0, 2.0, 9.0, 3.0, 4.0, 9.0]
    assert O.mix_rows([2.0, 0.5], rows, 3, 0, [10.0, 20.0]).tolist() == [13.5, 26.0]
    assert O.mix_rows([1.0, 1.0], rows, 3, 2, [0.0]).tolist() == [18.0]
    assert O.mix_rows([1.0], [1.0, 2.0], 2, 5, [5.0]).tolist() == [5.0]
    assert O.mix_rows([1.0], [1.0, 2.0], 2, 2 ** 64 - 1, [5.0]).tolist() == [5.0]
    assert O.mix_rows([1.0], [1.0, 2.0], 0, 0, [5.0]).tolist() == [6.0]


def test_mix_rows_is_fused_in_row_order():
    # float.rs:126-142: each product fused into its slot (one rounding), rows
    # in order; an unfused or reordered sum differs on these values
    rows = (np.arange(1, 49, dtype=np.float32) / np.float32(7.0)).astype(np.float32)
    w = np.float32([0.3, 0.7])
    for offset in (0, 12):
        want = np.zeros(12, np.float64)
        for i in range(2):
            seg = rows[i * 24 + offset:i * 24 + offset + 12].astype(np.float64)
            want = (seg * np.float64(w[i]) + want).astype(np.float32).astype(np.float64)  # exact product, one rounding
        got = O.mix_rows(w, rows, 24, offset, np.zeros(12, np.float32))
        assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))


def test_silu_known_answers():
    # elementwise.rs:43-56: silu(0) = 0; silu(2) = 2 / (1 + exp(-2)) in f32
    assert O.silu([0.0]).tolist() == [0.0]
    e = O.expf([-2.0])[0]
    want = np.float32(2.0) / (np.float32(1.0) + e)
    assert O.silu([2.0, 2.0]).view(np.uint32).tolist() == [np.float32(want).view(np.uint32)] * 2
    # SiLU is x * sigmoid(x): odd part plus x/2, checked in f64 on a spread
    x = np.linspace(-20, 20, 4001, dtype=np.float32)
    ref = x.astype(np.float64) / (1.0 + np.exp(-x.astype(np.float64)))
    assert np.max(np.abs(O.silu(x) - ref) / np.maximum(np.abs(ref), 1e-30)) < 4e-7
