"""Pins of the oracle's sparse split-bitmap restatement (oracle.sparse_gmap_dense, the lookup of
get_sparse_inactive_bit, TriSMoE_cuda_kernel.cu:619-637) on the CPU:
- round trip through the packer the reference's exporters use (pack_sparse_bool_matrix and the column prefix,
  pack_utils.py:32-52, restated in the oracle by column selection, an independent path);
- a scalar loop that reads one bit at a time, on a prefix that is not the running count (the kernel's
  per-row prefix, not a global column numbering, decides where a row's bits start);
- planted slips (salient and non-salient ranks swapped, the prefix ignored) that the checks above reject;
- the product's load-time conversion (checkpoint.sparse_gmap_to_dense) agrees with the oracle."""
import numpy as np
import pytest


def salient_mask(rng, rank):
    sal = rng.random(rank) < 0.07
    sal[32:64] = True          # a packed row of salient columns only
    sal[64:96] = False         # one without any
    sal[rank - 1] = True       # the partial last row ends on a salient column
    return sal


def sparse_form(oracle_mod, dense_bool, sal):
    """[N, K] split bits -> (q_gmap_sparse [rows, N], prefix [K/32 + 1]) by the exporters' packer."""
    words = oracle_mod.pack_sparse_bool_matrix(dense_bool, ~sal)
    return words, oracle_mod.sparse_prefix(~sal)


@pytest.mark.parametrize("rank,n", [(200, 37), (512, 64), (33, 5)])
def test_sparse_gmap_round_trip(oracle_mod, rank, n):
    rng = np.random.default_rng(rank + n)
    sal = salient_mask(rng, rank) if rank >= 96 else rng.random(rank) < 0.2
    dense = rng.random((n, rank)) < 0.3
    words, prefix = sparse_form(oracle_mod, dense, sal)
    c_map = oracle_mod.pack_bool_vector(sal)
    got = oracle_mod.sparse_gmap_dense(words, prefix, c_map, rank)
    want = oracle_mod.pack_bool_matrix(np.where(sal[None, :], False, dense))
    np.testing.assert_array_equal(got, want)


def scalar_lookup(words, prefix, c_map, rank):
    """get_sparse_inactive_bit one (k, n) at a time."""
    words = np.asarray(words).astype(np.uint32)
    n = words.shape[1]
    out = np.zeros((-(-rank // 32), n), dtype=np.uint32)
    for k in range(rank):
        row, b = k // 32, k % 32
        cw = int(np.uint32(c_map[row]))
        if (cw >> b) & 1:
            continue
        inactive_before = b - bin(cw & ((1 << b) - 1)).count("1")
        j = int(prefix[row]) + inactive_before
        for col in range(n):
            if (int(words[j >> 5, col]) >> (j & 31)) & 1:
                out[row, col] |= np.uint32(1 << b)
    return out.view(np.int32)


def test_sparse_gmap_matches_scalar_lookup_on_shifted_prefix(oracle_mod):
    rng = np.random.default_rng(3)
    rank, n = 160, 9
    sal = rng.random(rank) < 0.1
    c_map = oracle_mod.pack_bool_vector(sal)
    words = rng.integers(-2**31, 2**31, size=(8, n), dtype=np.int64).astype(np.int32)
    # row starts that do not follow the running count of non-salient columns (each row reads its own run)
    prefix = np.array([5, 40, 41, 100, 130, 131], dtype=np.int32)
    np.testing.assert_array_equal(oracle_mod.sparse_gmap_dense(words, prefix, c_map, rank),
                                  scalar_lookup(words, prefix, c_map, rank))


def test_planted_slips_are_caught(oracle_mod):
    """Two plausible mistakes in a restatement, each rejected by the scalar lookup or the round trip."""
    rng = np.random.default_rng(11)
    rank, n = 128, 7
    sal = salient_mask(rng, rank)
    dense = rng.random((n, rank)) < 0.4
    words, prefix = sparse_form(oracle_mod, dense, sal)
    c_map = oracle_mod.pack_bool_vector(sal)
    want = oracle_mod.pack_bool_matrix(np.where(sal[None, :], False, dense))
    # slip 1: a column's rank counted among the salient columns instead of the non-salient ones
    flipped = oracle_mod.pack_bool_vector(~sal)
    slip1 = oracle_mod.sparse_gmap_dense(words, prefix, flipped, rank)
    assert not np.array_equal(slip1, want)
    # slip 2: rows read from the start of the stream (prefix ignored)
    slip2 = oracle_mod.sparse_gmap_dense(words, np.zeros_like(prefix), c_map, rank)
    assert not np.array_equal(slip2, want)


def test_product_load_conversion_agrees(oracle_mod):
    from tris_moe_amd import checkpoint

    rng = np.random.default_rng(21)
    rank, n = 256, 48
    sal = salient_mask(rng, rank)
    dense = rng.random((n, rank)) < 0.2
    words, prefix = sparse_form(oracle_mod, dense, sal)
    c_map = oracle_mod.pack_bool_vector(sal)
    np.testing.assert_array_equal(checkpoint.sparse_gmap_to_dense(words, prefix, c_map, rank),
                                  oracle_mod.sparse_gmap_dense(words, prefix, c_map, rank))
