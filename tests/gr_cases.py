"""Shared builders for block-GR test cases (known answers and random bitmaps)."""
import json
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden" / "gr_known_answers.json"


def load_known_answers():
    return json.loads(GOLDEN.read_text())


def block_from_positions(positions) -> np.ndarray:
    """Dense packed [2, 64] int32 bitmap holding exactly one GR block with ones at flat positions."""
    words = np.zeros(128, dtype=np.uint32)
    for p in positions:
        words[p >> 5] |= np.uint32(1) << np.uint32(p & 31)
    return words.reshape(2, 64).view(np.int32)


def case_positions(case) -> list:
    if "ones_range" in case:
        lo, hi = case["ones_range"]
        return list(range(lo, hi))
    return list(case["ones"])


def case_expected_words(case, dense) -> np.ndarray:
    if case.get("raw"):
        return dense.reshape(-1).astype(np.int32)
    if "words_fill" in case:
        value, count = case["words_fill"]
        return np.full(count, value, dtype=np.int32)
    return np.asarray(case["words"], dtype=np.int32)


def multi_block_dense(case) -> np.ndarray:
    dense = np.zeros((case["packed_rows"], case["outfeatures"]), dtype=np.uint32)
    for row, col, bit in case["set_bits"]:
        dense[row, col] |= np.uint32(1) << np.uint32(bit)
    return dense.view(np.int32)


def random_bitmap(rng, packed_rows: int, n: int, p: float, rank: int | None = None) -> np.ndarray:
    """Dense packed bitmap with Bernoulli(p) bits; bits at k >= rank are cleared."""
    bits = rng.random((packed_rows * 32, n)) < p
    if rank is not None:
        bits[rank:] = False
    shifts = np.arange(32, dtype=np.uint64).reshape(1, 32, 1)
    words = (bits.reshape(packed_rows, 32, n).astype(np.uint64) << shifts).sum(axis=1).astype(np.uint32)
    return words.view(np.int32)


def structured_bitmap(kind: str, packed_rows: int, n: int, rng) -> np.ndarray:
    """Edge-case bitmaps: empty, full, single ones at block corners, dense runs."""
    dense = np.zeros((packed_rows, n), dtype=np.uint32)
    if kind == "full":
        dense[:] = 0xFFFFFFFF
    elif kind == "corners":
        dense[0, 0] = 1
        dense[-1, -1] = 0x80000000
        dense[min(1, packed_rows - 1), min(63, n - 1)] |= 0x80000000
    elif kind == "stripes":
        dense[:, ::3] = 0x55555555
    elif kind == "sparse_long_runs":
        idx = rng.choice(packed_rows * n, size=max(1, packed_rows * n // 97), replace=False)
        dense.reshape(-1)[idx] = np.uint32(1) << rng.integers(0, 32, idx.size).astype(np.uint32)
    return dense.view(np.int32)


def to_sparse(oracle_mod, payload, rank):
    """A block-GR synthetic payload (with its dense split bitmaps) in the sparse form the reference's
    TRIS_COMPACT3_BLOCK_GR=0 exporters write (pack_utils.py:32-52): non-salient columns only, per-expert rows
    zero padded to the largest."""
    E = payload["qweight1"].shape[0]
    n = payload["qweight1"].shape[2]
    forms = []
    for e in range(E):
        sal = oracle_mod.unpack_bool_vector(payload["c_map"][e], rank)
        dense = oracle_mod.unpack_bool_matrix(payload["gmap_dense"][e], rank)  # [N, K]
        forms.append((oracle_mod.pack_sparse_bool_matrix(dense, ~sal), oracle_mod.sparse_prefix(~sal)))
    rows = max(1, max(w.shape[0] for w, _ in forms))
    words = np.zeros((E, rows, n), dtype=np.int32)
    for e, (w, _) in enumerate(forms):
        words[e, : w.shape[0]] = w
    out = {k: v for k, v in payload.items() if not k.startswith("q_gmap_gr") and k != "gmap_dense"}
    out["q_gmap_sparse"] = words
    out["q_gmap_sparse_prefix"] = np.stack([pre for _, pre in forms]).astype(np.int32)
    out["compact3_use_block_gr"] = False
    return out
