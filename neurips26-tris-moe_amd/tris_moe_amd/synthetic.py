"""Seeded synthetic compact3 / block-GR payloads for the BASELINE configurations.

One numpy ``Generator(PCG64(seed))`` drives everything.  Per projection
(E experts, N outputs, K = rank):

* weights W ~ N(0, 0.02) rounded to fp16; sign plane qweight1 = (W >= 0);
* salient columns: the ceil(salient_frac * K) columns with the largest
  calibration-activation norm of the projection's input (the backbone output),
  jittered per expert; a second sign plane (qweight2_sparse) holds the sign of
  the first-term residual on those columns;
* split bitmap: Bernoulli(p) on non-salient positions, zeros on salient ones,
  block-GR coded by the library's encoder;
* column factors (col_pack3 halves) ~ U(0.75, 1.25); row scales (row_pack3,
  one per output and 128-column group) are the group means of |W| / factor over
  the positions each term covers, so every reconstructed weight has the
  magnitude of W.

Dict keys follow the stacked grouped payload (qlinear_cuda.py:1613-1632).
"""
from __future__ import annotations

import math

import numpy as np

from . import packing
from .configs import MoELayerSpec


def rng_for(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def _group_mean(values: np.ndarray, mask: np.ndarray, group: int, G: int) -> np.ndarray:
    """Mean of values over mask per (row, column group); groups with an empty mask use all columns."""
    n, k = values.shape
    pad = G * group - k
    v = np.pad(values, ((0, 0), (0, pad))) if pad else values
    m = np.broadcast_to(mask, values.shape)
    m = np.pad(m, ((0, 0), (0, pad))) if pad else m
    v3 = v.reshape(n, G, group)
    m3 = m.reshape(n, G, group)
    cnt = m3.sum(axis=2)
    s = np.where(m3, v3, 0.0).sum(axis=2)
    valid_cols = np.pad(np.ones(k, dtype=bool), (0, pad)).reshape(G, group)
    all_mean = np.where(valid_cols[None], v3, 0.0).sum(axis=2) / np.maximum(valid_cols.sum(axis=1), 1)[None]
    return np.where(cnt > 0, s / np.maximum(cnt, 1), all_mean).astype(np.float32)


def make_expert(rng: np.random.Generator, n: int, k: int, p: float, salient: np.ndarray, group: int = 128,
                g_idx: np.ndarray | None = None) -> dict:
    """One expert's packed compact3 tensors plus its dense split bitmap."""
    G = math.ceil(k / group)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float16).astype(np.float32)
    sign1 = w >= 0
    gmap = (rng.random((n, k), dtype=np.float32) < np.float32(p)) & ~salient[None, :]
    cf = rng.uniform(0.75, 1.25, (4, k)).astype(np.float16)
    cf32 = cf.astype(np.float32)
    absw = np.abs(w)
    a1 = _group_mean(absw / cf32[0], salient[None, :], group, G)
    gi = np.arange(k) // group
    resid = absw - a1[:, gi] * cf32[0]
    sign2 = sign1 == (resid >= 0)
    a2 = _group_mean(np.abs(resid) / cf32[1], salient[None, :], group, G)
    ad = _group_mean(absw / cf32[2], gmap, group, G)
    an = _group_mean(absw / cf32[3], ~gmap & ~salient[None, :], group, G)
    del w, absw, resid
    out = {
        "qweight1": packing.pack_bool_matrix(sign1),
        "qweight2_sparse": packing.pack_sparse_bool_matrix(sign2, salient),
        "qweight2_sparse_prefix": packing.sparse_prefix(salient),
        "c_map": packing.pack_bool_vector(salient),
        "g_idx": (gi if g_idx is None else g_idx).astype(np.int32),
        "col_pack3": packing.pack_half4(cf[0], cf[1], cf[2], cf[3]),
        "row_pack3": packing.pack_half4(a1.astype(np.float16), a2.astype(np.float16), ad.astype(np.float16),
                                        an.astype(np.float16)),
        "gmap_dense": packing.pack_bool_matrix(gmap),
    }
    return out


def salient_columns(rng: np.random.Generator, col_norm: np.ndarray, count: int) -> np.ndarray:
    score = col_norm * rng.uniform(0.8, 1.2, col_norm.shape[0])
    sal = np.zeros(col_norm.shape[0], dtype=bool)
    if count > 0:
        sal[np.argsort(-score, kind="stable")[:count]] = True
    return sal


def stack_projection(experts: list, n: int, k: int, encode, keep_dense_gmap: bool = False,
                     output_scale: np.ndarray | None = None, bias: np.ndarray | None = None) -> dict:
    """Stack per-expert tensors into the grouped payload, GR-coding each split bitmap.
    Ragged qweight2_sparse and GR word arrays are zero padded (qlinear_cuda.py:1551-1601)."""
    E = len(experts)
    packed_rows = -(-k // 32)
    coded = [encode(ex["gmap_dense"]) for ex in experts]
    max_q2 = max(ex["qweight2_sparse"].shape[0] for ex in experts)
    max_words = max(c[0].size for c in coded)
    q2 = np.zeros((E, max_q2, n), dtype=np.int32)
    words = np.zeros((E, max_words), dtype=np.int32)
    for e, ex in enumerate(experts):
        q2[e, : ex["qweight2_sparse"].shape[0]] = ex["qweight2_sparse"]
        words[e, : coded[e][0].size] = coded[e][0]
    g_idx = np.stack([ex["g_idx"] for ex in experts])
    uniform = bool(all(np.all(g[(np.arange(k) // 64) * 64] == g) for g in g_idx))
    has_scale = output_scale is not None and not np.all(output_scale == 1)
    payload = {
        "is_compact3": True,
        "qweight1": np.stack([ex["qweight1"] for ex in experts]).reshape(E, packed_rows, n),
        "qweight2_sparse": q2,
        "qweight2_sparse_prefix": np.stack([ex["qweight2_sparse_prefix"] for ex in experts]),
        "compact3_use_block_gr": True,
        "q_gmap_gr_words": words,
        "q_gmap_gr_offsets": np.stack([c[1] for c in coded]),
        "q_gmap_gr_meta": np.stack([c[2] for c in coded]),
        "c_map": np.stack([ex["c_map"] for ex in experts]),
        "g_idx": g_idx,
        "col_pack3": np.stack([ex["col_pack3"] for ex in experts]),
        "row_pack3": np.stack([ex["row_pack3"] for ex in experts]),
        "output_scale": (output_scale if output_scale is not None else np.ones((E, n))).astype(np.float16),
        "has_output_scale": bool(has_scale),
        "bias": None if bias is None else bias.astype(np.float16),
        "has_bias": bias is not None,
        "_compact3_k64_groups_uniform": uniform,
    }
    if keep_dense_gmap:
        payload["gmap_dense"] = np.stack([ex["gmap_dense"] for ex in experts])
    return payload


def make_projection(rng: np.random.Generator, num_experts: int, n: int, k: int, p: float, col_norm: np.ndarray,
                    encode, salient_frac: float = 0.05, group: int = 128, salient_counts=None,
                    keep_dense_gmap: bool = False, output_scale=None, bias=None, g_idx=None) -> dict:
    experts = []
    for e in range(num_experts):
        cnt = math.ceil(salient_frac * k) if salient_counts is None else int(salient_counts[e])
        sal = salient_columns(rng, col_norm, cnt)
        experts.append(make_expert(rng, n, k, p, sal, group, g_idx))
    return stack_projection(experts, n, k, encode, keep_dense_gmap, output_scale, bias)


def make_activations(rng: np.random.Generator, tokens: int, hidden: int, outliers: int = 4,
                     scale: float = 20.0, outlier_idx: np.ndarray | None = None) -> np.ndarray:
    """bf16-representable N(0,1) activations with `outliers` channels scaled, as float32."""
    x = rng.standard_normal((tokens, hidden), dtype=np.float32)
    if outlier_idx is None:
        outlier_idx = rng.choice(hidden, size=outliers, replace=False) if outliers else np.zeros(0, dtype=np.int64)
    x[:, outlier_idx] *= np.float32(scale)
    return bf16_round(x)


def bf16_round(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def make_layer(spec: MoELayerSpec, seed: int, encode, keep_dense_gmap: bool = False, gmap_p: float | None = None) -> dict:
    """All tensors of one synthetic MoE layer (numpy, host)."""
    rng = rng_for(seed)
    p = spec.gmap_p if gmap_p is None else gmap_p
    H, I, K, E = spec.hidden, spec.intermediate, spec.rank, spec.num_experts
    outlier_idx = rng.choice(H, size=spec.outlier_channels, replace=False) if spec.outlier_channels else None
    sv = {
        "gate": (rng.standard_normal((K, H), dtype=np.float32) * np.float32(0.02)).astype(np.float16),
        "up": (rng.standard_normal((K, H), dtype=np.float32) * np.float32(0.02)).astype(np.float16),
        "down": (rng.standard_normal((K, I), dtype=np.float32) * np.float32(0.02)).astype(np.float16),
    }
    cal_x = make_activations(rng, 64, H, spec.outlier_channels, spec.outlier_scale, outlier_idx)
    cal_m = rng.standard_normal((64, I), dtype=np.float32) * np.float32(0.1)
    norms = {
        "gate": np.linalg.norm(cal_x @ sv["gate"].astype(np.float32).T, axis=0),
        "up": np.linalg.norm(cal_x @ sv["up"].astype(np.float32).T, axis=0),
        "down": np.linalg.norm(cal_m @ sv["down"].astype(np.float32).T, axis=0),
    }
    layer = {"spec": spec, "seed": seed, "outlier_idx": outlier_idx, "backbones": sv}
    for proj, n in (("gate", I), ("up", I), ("down", H)):
        layer[proj] = make_projection(rng, E, n, K, p, norms[proj], encode, spec.salient_frac, spec.group_size,
                                      keep_dense_gmap=keep_dense_gmap)
    if spec.shared_expert_intermediate:
        Is = spec.shared_expert_intermediate
        layer["shared_expert"] = tuple(
            (rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02)).astype(np.float16)
            for shape in ((Is, H), (Is, H), (H, Is)))
        # the shared expert's gate, Linear(H, 1, bias=False) in the model dtype (bf16 values as float32), as the
        # Qwen blocks hold it (modeling_qwen2_moe.py:270, modeling_qwen3_5_moe.py:57)
        layer["shared_expert_gate"] = bf16_round(rng.standard_normal(H, dtype=np.float32) * np.float32(0.02))
    return layer


def make_inputs(spec: MoELayerSpec, tokens: int, seed: int, outlier_idx=None) -> dict:
    """Activations (bf16 values as float32) and router logits for one step."""
    rng = rng_for(seed)
    x = make_activations(rng, tokens, spec.hidden, spec.outlier_channels, spec.outlier_scale, outlier_idx)
    logits = (rng.standard_normal((tokens, spec.num_experts), dtype=np.float32) * np.float32(spec.router_std))
    return {"x": x, "router_logits": logits}


def payload_nbytes(payload: dict, experts=None) -> int:
    """Compressed bytes of the listed experts (default: all) as stored (the roofline's algorithmic
    bytes: qweight1, qweight2_sparse (+prefix), GR words (actual, unpadded) + offsets + meta,
    c_map, g_idx, col_pack3, row_pack3)."""
    E = payload["qweight1"].shape[0]
    ids = range(E) if experts is None else experts
    total = 0
    for e in ids:
        words_e = int(payload["q_gmap_gr_offsets"][e][-1])
        total += payload["qweight1"][e].nbytes + payload["qweight2_sparse"][e].nbytes
        total += payload["qweight2_sparse_prefix"][e].nbytes + 4 * words_e
        total += payload["q_gmap_gr_offsets"][e].nbytes + payload["q_gmap_gr_meta"][e].nbytes
        total += payload["c_map"][e].nbytes + payload["g_idx"][e].nbytes
        total += payload["col_pack3"][e].nbytes + payload["row_pack3"][e].nbytes
    return int(total)


def predecoded_nbytes(payload: dict, experts=None) -> int:
    """Bytes a predecoded grouped GEMM reads for the listed experts: the payload minus the GR
    stream (words, offsets, meta) plus the decoded split bitmap (128 words per GR block)."""
    E = payload["qweight1"].shape[0]
    ids = list(range(E) if experts is None else experts)
    nblk = int(payload["q_gmap_gr_meta"].shape[1])
    total = payload_nbytes(payload, ids)
    for e in ids:
        total -= 4 * int(payload["q_gmap_gr_offsets"][e][-1])
        total -= payload["q_gmap_gr_offsets"][e].nbytes + payload["q_gmap_gr_meta"][e].nbytes
        total += nblk * 128 * 4
    return int(total)


def make_ns_payload(rng: np.random.Generator, num_experts: int, infeatures: int, outfeatures: int, ranks,
                    group_size: int = 128, magnitude: float = 0.02, share_c2: bool = False) -> dict:
    """A matrix-mode null-space compensation payload (host): per expert random C2 [rank, in] and C1
    [out, rank] of the given magnitude, 4-bit packed (packing.pack_4bit) and concatenated
    (qlinear.build_grouped_ns_payload); rank 0 gives no compensation; share_c2 makes experts of equal rank
    share one C2 block."""
    from .packing import pack_4bit
    from .qlinear import build_grouped_ns_payload

    c2, c1, keys = [], [], []
    shared = {}
    for e in range(num_experts):
        r = int(ranks[e])
        if r <= 0:
            c2.append(None)
            c1.append(None)
            keys.append(("none", e))
            continue
        if share_c2 and r in shared:
            c2.append(shared[r])
        else:
            blk = pack_4bit(rng.standard_normal((r, infeatures)).astype(np.float32) * magnitude, group_size)
            shared[r] = blk
            c2.append(blk)
        keys.append(("shared", r) if share_c2 else ("local", e))
        c1.append(pack_4bit(rng.standard_normal((outfeatures, r)).astype(np.float32) * magnitude, min(r, group_size)))
    return build_grouped_ns_payload(c2, c1, infeatures, outfeatures, group_size, c2_keys=keys)
