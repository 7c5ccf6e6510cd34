"""Bit and half packing of the compact3 payload (format producer side).

Restates the layouts of ``utils/pack_utils.py:6-125`` and
``qlinear_cuda.py:3612-3761`` with vectorised numpy:

* bool matrix [N, K] -> int32 [ceil(K/32), N], bit k & 31 of word k // 32;
* bool vector [K] -> int32 [ceil(K/32)];
* sparse matrices keep only the active columns, compacted in k order, with a
  prefix table prefix[r] = number of active columns below 32 r;
* four fp16 values -> one int64 at bit offsets 0/16/32/48.
"""
from __future__ import annotations

import numpy as np


def pack_bool_matrix(matrix: np.ndarray) -> np.ndarray:
    m = np.asarray(matrix, dtype=bool)
    n, k = m.shape
    words = -(-k // 32)
    padded = np.zeros((n, words * 32), dtype=bool)
    padded[:, :k] = m
    packed = np.packbits(padded, axis=1, bitorder="little")          # [n, words*4] bytes, LSB first
    as_u32 = packed.reshape(n, words, 4).astype(np.uint32)
    vals = as_u32[..., 0] | (as_u32[..., 1] << 8) | (as_u32[..., 2] << 16) | (as_u32[..., 3] << 24)
    return np.ascontiguousarray(vals.T).view(np.int32)


def pack_bool_vector(values: np.ndarray) -> np.ndarray:
    return pack_bool_matrix(np.asarray(values, dtype=bool)[None, :])[:, 0].copy()


def sparse_prefix(active: np.ndarray) -> np.ndarray:
    a = np.asarray(active, dtype=bool).ravel()
    rows = -(-a.size // 32)
    padded = np.zeros(rows * 32, dtype=np.int64)
    padded[: a.size] = a
    return np.concatenate([[0], np.cumsum(padded.reshape(rows, 32).sum(axis=1))]).astype(np.int32)


def pack_sparse_bool_matrix(matrix: np.ndarray, active: np.ndarray) -> np.ndarray:
    m = np.asarray(matrix, dtype=bool)
    a = np.asarray(active, dtype=bool)
    if not a.any():
        return np.zeros((0, m.shape[0]), dtype=np.int32)
    return pack_bool_matrix(m[:, a])


def pack_half4(h0, h1, h2, h3) -> np.ndarray:
    def bits(x):
        return np.asarray(x, dtype=np.float16).view(np.uint16).astype(np.uint64)

    return (bits(h0) | (bits(h1) << np.uint64(16)) | (bits(h2) << np.uint64(32)) | (bits(h3) << np.uint64(48))).view(np.int64)


def num_gr_blocks(rank: int, outfeatures: int) -> int:
    packed_rows = -(-rank // 32)
    return -(-packed_rows // 2) * -(-outfeatures // 64)
