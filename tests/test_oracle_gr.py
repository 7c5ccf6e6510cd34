"""Pin the CPU oracle's block-GR codec (and the product's host encoder) on the CPU.

Checks: hand-derived known answers (tests/golden/gr_known_answers.json),
closed-form Rice lengths and first-minimum k, the raw threshold, round trips on
random and edge-case bitmaps, agreement of the reference decoder's general
and k==3 paths, and the behaviour on streams whose one_count disagrees with
the bits (both reference decoder paths, which the GPU decoder must follow).
"""
import numpy as np
import pytest

from gr_cases import (block_from_positions, case_expected_words, case_positions, load_known_answers,
                      multi_block_dense, random_bitmap, structured_bitmap)

KATS = load_known_answers()


@pytest.mark.parametrize("case", KATS["single_block"], ids=lambda c: c["name"])
def test_known_answer_encode(oracle_mod, case):
    dense = block_from_positions(case_positions(case))
    words, offsets, meta = oracle_mod.gr_encode(dense)
    expected = case_expected_words(case, dense)
    np.testing.assert_array_equal(words, expected)
    assert offsets.tolist() == [0, expected.size]
    assert meta.tolist() == [case["meta"]]


@pytest.mark.parametrize("case", KATS["single_block"], ids=lambda c: c["name"])
@pytest.mark.parametrize("k3_fast_path", [True, False])
def test_known_answer_decode(oracle_mod, case, k3_fast_path):
    dense = block_from_positions(case_positions(case))
    words = case_expected_words(case, dense)
    offsets = np.array([0, words.size], dtype=np.int32)
    meta = np.array([case["meta"]], dtype=np.int32)
    block = oracle_mod.gr_decode_block(words, offsets, meta, 0, k3_fast_path=k3_fast_path)
    np.testing.assert_array_equal(block.view(np.int32), dense.reshape(-1))


@pytest.mark.parametrize("case", KATS["multi_block"], ids=lambda c: c["name"])
def test_known_answer_multi_block(oracle_mod, case):
    dense = multi_block_dense(case)
    words, offsets, meta = oracle_mod.gr_encode(dense)
    assert words.tolist() == case["words"]
    assert offsets.tolist() == case["offsets"]
    assert meta.tolist() == case["meta"]
    back = oracle_mod.gr_decode_dense(words, offsets, meta, case["packed_rows"], case["outfeatures"])
    np.testing.assert_array_equal(back, dense)


def _block_runs(block_words):
    pos = [w * 32 + b for w in range(128) for b in range(32) if (int(block_words[w]) >> b) & 1]
    runs, prev = [], -1
    for p in pos:
        runs.append(p - prev - 1)
        prev = p
    return runs


@pytest.mark.parametrize("p", [0.02, 0.15, 0.4])
def test_k_choice_and_length_closed_form(oracle_mod, p):
    """meta k is the first minimiser of sum(run>>k)+n(1+k); word count is ceil(bits/32)."""
    rng = np.random.default_rng(7)
    dense = random_bitmap(rng, 8, 192, p)
    words, offsets, meta = oracle_mod.gr_encode(dense)
    nob = 3
    for bi in range(meta.size):
        kb, ob = divmod(bi, nob)
        blk = np.zeros((2, 64), dtype=np.int32)
        blk[:, :] = dense[2 * kb:2 * kb + 2, 64 * ob:64 * ob + 64]
        runs = _block_runs(blk.reshape(-1).view(np.uint32))
        costs = [sum(r >> k for r in runs) + len(runs) * (1 + k) for k in range(8)]
        best = min(range(8), key=lambda k: (costs[k], k))
        nwords = offsets[bi + 1] - offsets[bi]
        if -(-costs[best] // 32) >= 128:
            assert meta[bi] == 16 and nwords == 128
        else:
            assert meta[bi] == best | (len(runs) << 8)
            assert nwords == -(-costs[best] // 32)
            assert oracle_mod.rice_bits(np.array(runs), best) == costs[best]


@pytest.mark.parametrize("p", [0.0, 0.05, 0.15, 0.3, 0.6, 0.97])
@pytest.mark.parametrize("shape", [(2, 64), (16, 896), (3, 70), (17, 130)])
def test_round_trip_random(oracle_mod, p, shape):
    rng = np.random.default_rng(int(p * 1000) + shape[0] * 7 + shape[1])
    dense = random_bitmap(rng, shape[0], shape[1], p)
    words, offsets, meta = oracle_mod.gr_encode(dense)
    back = oracle_mod.gr_decode_dense(words, offsets, meta, *shape)
    np.testing.assert_array_equal(back, dense)


@pytest.mark.parametrize("kind", ["full", "corners", "stripes", "sparse_long_runs"])
def test_round_trip_structured(oracle_mod, kind):
    rng = np.random.default_rng(3)
    dense = structured_bitmap(kind, 9, 131, rng)
    words, offsets, meta = oracle_mod.gr_encode(dense)
    np.testing.assert_array_equal(oracle_mod.gr_decode_dense(words, offsets, meta, 9, 131), dense)


@pytest.mark.parametrize("kmin,kmax", [(0, 0), (3, 3), (2, 5), (7, 7)])
def test_k_bounds_round_trip(oracle_mod, kmin, kmax):
    """The export tool's --blockgr-k-min/max (rewrite_runtime_min_checkpoint.py:228-249) still decodes."""
    rng = np.random.default_rng(11)
    dense = random_bitmap(rng, 6, 128, 0.15)
    words, offsets, meta = oracle_mod.gr_encode(dense, kmin, kmax)
    coded = meta[(meta & 16) == 0]
    assert np.all(((coded & 15) >= kmin) & ((coded & 15) <= kmax))
    np.testing.assert_array_equal(oracle_mod.gr_decode_dense(words, offsets, meta, 6, 128), dense)


def test_force_raw(oracle_mod):
    rng = np.random.default_rng(5)
    dense = random_bitmap(rng, 4, 100, 0.1)
    words, offsets, meta = oracle_mod.gr_encode(dense, force_raw=True)
    assert np.all(meta == 16) and offsets[-1] == 128 * meta.size
    np.testing.assert_array_equal(oracle_mod.gr_decode_dense(words, offsets, meta, 4, 100), dense)


def test_rice_encoder_matches_known_stream(oracle_mod):
    # runs [15]*7 at k=3 -> '01111' x 7 (see the k3_remainder_straddles_word known answer)
    out = oracle_mod.rice_encode([15] * 7, 3)
    assert out.tolist() == [0xBDEF7BDE, 7]


@pytest.mark.parametrize("k", range(8))
def test_decoder_paths_agree_on_malformed_streams(oracle_mod, k):
    """Streams whose one_count exceeds the complete codewords, truncated streams and stray bits:
    the reference's general and k==3 readers must decode identically (the GPU decoder is
    checked against these same outputs)."""
    rng = np.random.default_rng(100 + k)
    for trial in range(40):
        nwords = int(rng.integers(1, 6))
        words = rng.integers(-2**31, 2**31, size=nwords, dtype=np.int64).astype(np.int32)
        if trial % 3 == 0:
            words[-1] = 0  # trailing zero padding: an unterminated unary run
        one_count = int(rng.integers(0, 400))
        meta = np.array([k | (one_count << 8)], dtype=np.int32)
        offsets = np.array([0, nwords], dtype=np.int32)
        a = oracle_mod.gr_decode_block(words, offsets, meta, 0, k3_fast_path=True)
        b = oracle_mod.gr_decode_block(words, offsets, meta, 0, k3_fast_path=False)
        np.testing.assert_array_equal(a, b)


def test_predecode_layout(oracle_mod):
    rng = np.random.default_rng(9)
    dense = [random_bitmap(rng, 4, 128, 0.2) for _ in range(3)]
    coded = [oracle_mod.gr_encode(d) for d in dense]
    width = max(c[0].size for c in coded)
    words = np.zeros((3, width), dtype=np.int32)
    for e, c in enumerate(coded):
        words[e, : c[0].size] = c[0]
    offsets = np.stack([c[1] for c in coded])
    meta = np.stack([c[2] for c in coded])
    out = oracle_mod.gr_predecode(words, offsets, meta, np.array([2, -1, 0]), 4)
    assert out.shape == (3, 4, 128)
    assert not out[1].any()
    for slot, e in ((0, 2), (2, 0)):
        for b in range(4):
            kb, ob = divmod(b, 2)
            np.testing.assert_array_equal(out[slot, b].reshape(2, 64), dense[e][2 * kb:2 * kb + 2, 64 * ob:64 * ob + 64])
