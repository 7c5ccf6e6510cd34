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


def pack_4bit(matrix: np.ndarray, group_size: int = 128) -> dict:
    """4-bit packed payload of a float matrix [rows, cols] with contiguous column groups (the export side
    of the packed shared backbone): per (group, row) asymmetric min/max quantisation, scale =
    (max - min) / 14 rounded to fp16, zero = round(-min / scale) in 1..15; then the reference producer's layout
    (utils/pack_utils.py:126-180): q = clamp(round(m / s + z), 0, 15) in nibble c % 8 of qweight[c // 8][r],
    (z - 1) & 0xF in nibble r % 8 of qzeros[g][r // 8], scales group-major [G, rows]."""
    m = np.asarray(matrix, dtype=np.float32)
    rows, cols = m.shape
    groups = (cols + group_size - 1) // group_size
    g_idx = (np.arange(cols) // group_size).astype(np.int32)
    pad = groups * group_size - cols
    mp = np.pad(m, ((0, 0), (0, pad)), mode="edge") if pad else m
    blocks = mp.reshape(rows, groups, group_size)
    lo = np.minimum(blocks.min(axis=2), 0.0).T   # [G, rows]; the range always holds 0
    hi = np.maximum(blocks.max(axis=2), 0.0).T
    # (max - min) / 14: one step of slack, so that rounding the zero (a shift of up to s / 2) never pushes an
    # end of the range past q = 0 or 15 and every weight stays within s / 2
    scale = ((hi - lo) / 14.0).astype(np.float16).astype(np.float32)
    scale[scale == 0] = 1.0
    zero = np.clip(np.round(-lo / scale), 0, 15)
    # a stored zero of 0 reads as 16 (the consumer adds one to (z - 1) & 0xF): use z = 1 and a scale that
    # still reaches the group's maximum at q = 15 instead
    low = zero < 1
    if low.any():
        s1 = (np.maximum(hi, scale * 0.5) / 13.5).astype(np.float16).astype(np.float32)
        scale = np.where(low, np.maximum(s1, scale), scale)
        zero = np.where(low, 1.0, zero)
    q = np.clip(np.round(m.T / scale[g_idx] + zero[g_idx]), 0, 15).astype(np.uint32)   # [cols, rows]
    qweight = np.zeros(((cols + 7) // 8, rows), dtype=np.uint32)
    for j in range(8):
        part = q[j::8]
        qweight[: part.shape[0]] |= part << np.uint32(4 * j)
    zint = ((zero.astype(np.int64) - 1) & 0xF).astype(np.uint32)   # [G, rows]
    qzeros = np.zeros((groups, (rows + 7) // 8), dtype=np.uint32)
    for j in range(8):
        part = zint[:, j::8]
        qzeros[:, : part.shape[1]] |= part << np.uint32(4 * j)
    return {"rows": rows, "cols": cols, "qweight": qweight.view(np.int32), "qzeros": qzeros.view(np.int32),
            "scales": scale.astype(np.float16), "g_idx": g_idx}
