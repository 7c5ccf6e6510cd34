"""Grouped expert runtime with the reference's Python API (``qlinear_cuda.py``), on the HIP library.

Mirrors, for the grouped block-GR expert path:

* ``build_grouped_route`` (``qlinear_cuda.py:1301-1378``) and its empty route
  (``:1242-1255``);
* ``run_grouped_structured_expert_forward`` (``:2131-2335``) and
  ``run_grouped_structured_expert_pair_forward`` (``:2338-2634``);
* ``build_grouped_precomputed_payload`` / payload resolution (``:1512-1682``);
* ``ExpertSharedMatrix`` + ``QuantLinear`` in expert_compact3 mode (mode 5):
  ``compute_shared_hidden`` (``:4454-4502``), ``forward_from_precomputed_hidden``
  (``:4504-4560``), ``can_precompute_shared`` (``:4451``), block-GR packing
  ``_pack_block_gr_gmap_tensor`` (``:3793-3859``);
* ``PackedQuantMatrix4bit`` (``:2637-2786``), the 4-bit packed backbone;
* the non-expert compact3 linear (``QuantLinear`` mode 4, ``:4238-4360``, here
  ``Compact3Linear``) and its fused launches ``run_compact3_qkv_block_gr_forward``
  (``:915-1002``) and ``run_compact3_shared_expert_gate_up_forward`` (``:1005-1098``);
* matrix-mode null-space compensation (``ns_mode == 2``) as a grouped payload:
  ``build_grouped_ns_compensation_payload`` (``:1734-1872``, here
  ``build_grouped_ns_payload``), ``run_grouped_ns_compensation_forward``
  (``:2028-2128``), ``run_grouped_ns_c1_forward`` (``:1964-2025``) and the
  ``ns_payload`` arguments of the structured forwards.

Differences that are deliberate: no CPU/dequant fallback (a missing HIP
library raises ``TrisExtensionUnavailable``); the route's segment order within
an expert is the stable flat order; the launch policy is this library's
(fused GR decode for decode-sized segments, predecode + predecoded GEMM when
segments are long), with no split-K since each workgroup covers all of K.
Null-space compensation comes from grouped payload dicts only; module lists
carry vector-mode input scales (``expert_input_scale``), not matrices.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn as nn

from . import ext
from .packing import num_gr_blocks

GROUPED_SEGMENT_M_TILE = 4
BLOCK_GR_TILE_K = 64
BLOCK_GR_TILE_OUT = 64
BLOCK_GR_PACKED_ROWS = 2
BLOCK_GR_WORDS_PER_BLOCK = 128
BLOCK_GR_META_RAW_FLAG = 1 << 4
BLOCK_GR_META_ONE_COUNT_SHIFT = 8
BLOCK_GR_MAX_K = 7
# Rows per segment above which the predecoded GEMM (one decode per block) beats
# in-kernel decode (one decode per 16-row tile).
PREDECODE_MIN_ROWS_PER_SEGMENT = 32
_PREDECODE_MAX_BYTES = 256 * 1024 * 1024

PAYLOAD_TENSOR_KEYS = ("qweight1", "qweight2_sparse", "qweight2_sparse_prefix", "q_gmap_gr_words",
                       "q_gmap_gr_offsets", "q_gmap_gr_meta", "c_map", "g_idx", "col_pack3", "row_pack3",
                       "output_scale", "bias")


# ------------------------------------------------------------------ payloads
def payload_to_device(payload: dict, device, dtype=torch.float16) -> dict:
    """Host (numpy) stacked payload -> device tensors with the reference's dtypes."""
    out = {}
    for key, val in payload.items():
        if isinstance(val, np.ndarray):
            if key in ("output_scale", "bias"):
                out[key] = torch.from_numpy(np.ascontiguousarray(val)).to(device=device, dtype=dtype)
            elif val.dtype == np.int64:
                out[key] = torch.from_numpy(np.ascontiguousarray(val)).to(device=device, dtype=torch.int64)
            else:
                out[key] = torch.from_numpy(np.ascontiguousarray(val).astype(np.int32)).to(device=device)
        else:
            out[key] = val
    return out


def _payload_has_output_scale(payload: dict) -> bool:
    scale = payload.get("output_scale")
    if not isinstance(scale, torch.Tensor) or scale.numel() == 0:
        return False
    if "has_output_scale" in payload:
        return bool(payload["has_output_scale"])
    return not bool(torch.all(scale == 1).item())


def _normalize_scalars(payload: dict) -> dict:
    """Scalars stored as 1-element tensors become Python values (grouped_payload_sidecar.py:168-190)."""
    for key in ("is_compact3", "compact3_use_block_gr", "has_output_scale", "has_bias", "_compact3_k64_groups_uniform"):
        val = payload.get(key)
        if isinstance(val, torch.Tensor) and val.numel() == 1:
            payload[key] = bool(val.reshape(-1)[0].item())
    return payload


def _k64_uniform(payload: dict) -> bool:
    if "_compact3_k64_groups_uniform" not in payload:
        g = payload["g_idx"]
        rank = int(g.size(1))
        first = g[:, (torch.arange(rank, device=g.device) // 64) * 64]
        payload["_compact3_k64_groups_uniform"] = bool(torch.equal(first, g))
    return bool(payload["_compact3_k64_groups_uniform"])


def is_sparse_payload(payload: dict) -> bool:
    """A payload whose split bitmaps are in the sparse form (compact3_use_block_gr false,
    qlinear_cuda.py:1658-1676): only the sparse kernel entry runs it."""
    return not bool(payload.get("compact3_use_block_gr", False))


def resolve_grouped_precomputed_payload(payload_or_modules, device, dtype):
    """qlinear_cuda.py:1639-1682: validate a payload dict or stack it from modules."""
    if isinstance(payload_or_modules, dict):
        payload = _normalize_scalars(payload_or_modules)
        for key in ("is_compact3", "qweight1", "c_map", "g_idx", "output_scale", "has_bias"):
            if key not in payload:
                return None
        if payload["qweight1"].device != torch.device(device) or payload["output_scale"].dtype != dtype:
            return None
        if not payload["is_compact3"]:
            return None
        if payload.get("compact3_use_block_gr", False):
            required = ("qweight2_sparse", "qweight2_sparse_prefix", "q_gmap_gr_words", "q_gmap_gr_offsets",
                        "q_gmap_gr_meta", "col_pack3", "row_pack3")
        else:  # the sparse split-bitmap form
            required = ("qweight2_sparse", "qweight2_sparse_prefix", "q_gmap_sparse", "q_gmap_sparse_prefix",
                        "col_pack3", "row_pack3")
        if any(key not in payload for key in required):
            return None
        payload["has_output_scale"] = _payload_has_output_scale(payload)
        _k64_uniform(payload)
        return payload
    return build_grouped_precomputed_payload(payload_or_modules, device, dtype)


# --------------------------------------------------------------------- route
def _empty_grouped_route(device):
    empty_int = torch.empty((0,), device=device, dtype=torch.int32)
    empty_long = torch.empty((0,), device=device, dtype=torch.long)
    return {
        "perm": empty_long,
        "grouped_token_indices": empty_long,
        "grouped_slots": empty_long,
        "grouped_expert_ids": empty_int,
        "expert_ids": empty_int,
        "segment_offsets": torch.zeros((1,), device=device, dtype=torch.int32),
        "problem_offsets": torch.zeros((1,), device=device, dtype=torch.int32),
        "total_problem_tiles": torch.zeros((1,), device="cpu", dtype=torch.int64),
        "total_problem_tiles_host": 0,
    }


def build_grouped_route(selected_experts: torch.Tensor, num_experts: int, m_tile: int = GROUPED_SEGMENT_M_TILE):
    """qlinear_cuda.py:1301-1378 on the device route kernels.  Returns None for a non-2D input and
    the empty route for an empty input or m_tile <= 0, as the reference does."""
    if selected_experts.dim() != 2:
        return None
    if m_tile <= 0 or selected_experts.numel() == 0:
        return _empty_grouped_route(selected_experts.device)
    route = ext.build_grouped_route_device(selected_experts, int(num_experts), int(m_tile))
    counts = route["counts"].to("cpu")
    num_active, total = int(counts[0]), int(counts[1])
    if num_active < 0:
        raise RuntimeError("build_grouped_route: expert id outside [0, num_experts)")
    return {
        "perm": route["perm"],
        "grouped_token_indices": route["grouped_token_indices"],
        "grouped_slots": route["grouped_slots"],
        "grouped_expert_ids": route["grouped_expert_ids"],
        "expert_ids": route["expert_ids"][:num_active].contiguous(),
        "segment_offsets": route["segment_offsets"][: num_active + 1].contiguous(),
        "problem_offsets": route["problem_offsets"][: num_active + 1].contiguous(),
        "total_problem_tiles": torch.tensor([total], dtype=torch.int64),
        "total_problem_tiles_host": total,
    }


def _route_total_problem_tiles_host(route) -> int:
    if "total_problem_tiles_host" in route:
        return int(route["total_problem_tiles_host"])
    return int(route["total_problem_tiles"].reshape(-1)[0].item())


def _coerce_grouped_route(route_or_lengths, device, expert_ids=None):
    """qlinear_cuda.py:1385-1406: a route dict, or per-expert segment lengths."""
    if isinstance(route_or_lengths, dict):
        return route_or_lengths
    lengths = torch.as_tensor(route_or_lengths, dtype=torch.long).cpu()
    if lengths.numel() == 0 or bool((lengths < 0).any()):
        return _empty_grouped_route(device)
    ids = (torch.arange(lengths.numel(), dtype=torch.int32) if expert_ids is None
           else torch.as_tensor(expert_ids, dtype=torch.int32).cpu())
    if ids.numel() != lengths.numel():
        return _empty_grouped_route(device)
    seg = torch.cat([torch.zeros(1, dtype=torch.long), torch.cumsum(lengths, 0)])
    prob = torch.cat([torch.zeros(1, dtype=torch.long),
                      torch.cumsum((lengths + GROUPED_SEGMENT_M_TILE - 1) // GROUPED_SEGMENT_M_TILE, 0)])
    return {
        "perm": torch.empty(0, dtype=torch.long, device=device),
        "grouped_token_indices": torch.empty(0, dtype=torch.long, device=device),
        "grouped_slots": torch.empty(0, dtype=torch.long, device=device),
        "grouped_expert_ids": torch.repeat_interleave(ids, lengths).to(device=device, dtype=torch.int32),
        "expert_ids": ids.to(device=device),
        "segment_offsets": seg.to(device=device, dtype=torch.int32),
        "problem_offsets": prob.to(device=device, dtype=torch.int32),
        "total_problem_tiles": prob[-1:].to(torch.int64),
        "total_problem_tiles_host": int(prob[-1]),
    }


# ------------------------------------------------------------ grouped forward
def _use_predecode(batch: int, num_segments: int, payload: dict, has_scale: bool, has_bias: bool) -> bool:
    if has_scale or has_bias or num_segments == 0:
        return False
    if batch < PREDECODE_MIN_ROWS_PER_SEGMENT * num_segments:
        return False
    rank = int(payload["g_idx"].size(1))
    n = int(payload["qweight1"].size(2))
    return num_segments * num_gr_blocks(rank, n) * BLOCK_GR_WORDS_PER_BLOCK * 4 <= _PREDECODE_MAX_BYTES


def _predecode(payload: dict, route: dict, rank: int, n: int) -> torch.Tensor:
    ids = route["expert_ids"]
    nblk = num_gr_blocks(rank, n)
    buf = torch.empty((ids.numel(), nblk, BLOCK_GR_WORDS_PER_BLOCK), dtype=torch.int32, device=ids.device)
    return ext.compact3_tris_precomputed_grouped_block_gr_predecode(
        buf, ids, payload["q_gmap_gr_words"], payload["q_gmap_gr_offsets"], payload["q_gmap_gr_meta"],
        (rank + 31) // 32, n)


def build_grouped_ns_payload(c2: list, c1: list, infeatures: int, outfeatures: int, group_size: int,
                             c2_keys: list | None = None) -> dict:
    """Host assembly of a null-space compensation payload (build_grouped_ns_compensation_payload,
    qlinear_cuda.py:1734-1872) from per-expert 4-bit packed payloads (``packing.pack_4bit`` dicts or None for
    an expert without compensation): c2[e] holds C2_e [rank_e, in], c1[e] C1_e [out, rank_e].  C2 blocks are
    concatenated along their rows (qweight / scales columns), C1 blocks along their packed rank words;
    experts with equal ``c2_keys[e]`` share one C2 block."""
    E = len(c2)
    ranks, c2_off, c2_woff, c1_woff, c1_goff = [], [], [], [], []
    c2_qw, c2_qz, c2_sc, c1_qw, c1_qz, c1_sc = [], [], [], [], [], []
    shared = {}
    tot_rank = tot_words = tot_c1_words = tot_c1_groups = 0
    in_groups = (infeatures + group_size - 1) // group_size if infeatures > 0 else 0
    for e in range(E):
        c1_woff.append(tot_c1_words)
        c1_goff.append(tot_c1_groups)
        if c2[e] is None or c1[e] is None:
            ranks.append(0)
            c2_off.append(tot_rank)
            c2_woff.append(tot_words)
            continue
        rank = int(c2[e]["rows"])
        if int(c1[e]["cols"]) != rank or int(c2[e]["cols"]) != infeatures or int(c1[e]["rows"]) != outfeatures:
            raise ValueError(f"expert {e}: C2 [{c2[e]['rows']}, {c2[e]['cols']}] / C1 [{c1[e]['rows']}, "
                             f"{c1[e]['cols']}] do not chain {infeatures} -> rank -> {outfeatures}")
        key = c2_keys[e] if c2_keys is not None else ("local", e)
        if key in shared:
            off, woff, r0 = shared[key]
            if r0 != rank:
                raise ValueError(f"expert {e}: shared C2 of rank {r0}, expert rank {rank}")
        else:
            off, woff = tot_rank, tot_words
            shared[key] = (off, woff, rank)
            c2_qw.append(np.asarray(c2[e]["qweight"], np.int32))
            c2_qz.append(np.asarray(c2[e]["qzeros"], np.int32))
            c2_sc.append(np.asarray(c2[e]["scales"], np.float16))
            tot_rank += rank
            tot_words += int(c2_qz[-1].shape[1])
        ranks.append(rank)
        c2_off.append(off)
        c2_woff.append(woff)
        c1_qw.append(np.asarray(c1[e]["qweight"], np.int32))
        c1_qz.append(np.asarray(c1[e]["qzeros"], np.int32))
        c1_sc.append(np.asarray(c1[e]["scales"], np.float16))
        tot_c1_words += int(c1_qw[-1].shape[0])
        tot_c1_groups += int(c1_qz[-1].shape[0])
    qzc = (outfeatures + 7) // 8
    return {
        "ns_rank_per_expert": np.asarray(ranks, np.int32),
        "ns_c2_rank_offsets": np.asarray(c2_off, np.int32),
        "ns_c2_rank_word_offsets": np.asarray(c2_woff, np.int32),
        "ns_c1_rank_word_offsets": np.asarray(c1_woff, np.int32),
        "ns_c1_group_offsets": np.asarray(c1_goff, np.int32),
        "max_ns_rank": max(ranks) if ranks else 0,
        "infeatures": int(infeatures),
        "outfeatures": int(outfeatures),
        "group_size": int(group_size),
        "ns_c2_qweight": np.concatenate(c2_qw, axis=1) if c2_qw else np.zeros(((infeatures + 7) // 8, 0), np.int32),
        "ns_c2_qzeros": np.concatenate(c2_qz, axis=1) if c2_qz else np.zeros((in_groups, 0), np.int32),
        "ns_c2_scales": np.concatenate(c2_sc, axis=1) if c2_sc else np.zeros((in_groups, 0), np.float16),
        "ns_c1_qweight": np.concatenate(c1_qw, axis=0) if c1_qw else np.zeros((0, outfeatures), np.int32),
        "ns_c1_qzeros": np.concatenate(c1_qz, axis=0) if c1_qz else np.zeros((0, qzc), np.int32),
        "ns_c1_scales": np.concatenate(c1_sc, axis=0) if c1_sc else np.zeros((0, outfeatures), np.float16),
    }


def validate_ns_payload(ns: dict) -> None:
    """Host check that every expert's slices lie inside the concatenated blocks (the kernels index them
    without bounds checks): raises ValueError naming the first expert that does not fit."""
    def arr(k):
        v = ns[k]
        return v.detach().cpu().numpy() if isinstance(v, torch.Tensor) else np.asarray(v)
    ranks = arr("ns_rank_per_expert").astype(np.int64)
    infeatures, outfeatures = int(ns["infeatures"]), int(ns["outfeatures"])
    gs, max_rank = int(ns["group_size"]), int(ns["max_ns_rank"])
    if max_rank > 0 and gs <= 0:
        raise ValueError("null-space payload: group_size must be positive")
    c2w, c2z, c2s = arr("ns_c2_qweight").shape, arr("ns_c2_qzeros").shape, arr("ns_c2_scales").shape
    c1w, c1z, c1s = arr("ns_c1_qweight").shape, arr("ns_c1_qzeros").shape, arr("ns_c1_scales").shape
    in_groups = (infeatures + gs - 1) // gs if gs > 0 else 0
    if max_rank > 0 and (c2w[0] != (infeatures + 7) // 8 or c2z[0] < in_groups or c2s[0] < in_groups
                         or c1w[1] != outfeatures or c1s[1] != outfeatures or c1z[1] != (outfeatures + 7) // 8):
        raise ValueError("null-space payload: block shapes do not match infeatures / outfeatures / group_size")
    off, woff = arr("ns_c2_rank_offsets"), arr("ns_c2_rank_word_offsets")
    c1wo, c1go = arr("ns_c1_rank_word_offsets"), arr("ns_c1_group_offsets")
    for e, r in enumerate(ranks):
        if r <= 0:
            continue
        egs = min(int(r), gs)
        groups = (int(r) + egs - 1) // egs
        if (r > max_rank or off[e] < 0 or off[e] + r > min(c2w[1], c2s[1]) or woff[e] < 0
                or woff[e] + (r + 7) // 8 > c2z[1] or c1wo[e] < 0 or c1wo[e] + (r + 7) // 8 > c1w[0]
                or c1go[e] < 0 or c1go[e] + groups > min(c1z[0], c1s[0])):
            raise ValueError(f"null-space payload: expert {e} (rank {int(r)}) lies outside the concatenated blocks")


def ns_payload_to_device(ns: dict, device, dtype=torch.float16) -> dict:
    """Host null-space payload -> device tensors (int32, scales in ``dtype``), scalars as Python ints;
    validated first (validate_ns_payload)."""
    validate_ns_payload(ns)
    out = {}
    for k, v in ns.items():
        if isinstance(v, (np.ndarray, torch.Tensor)):
            t = torch.as_tensor(np.ascontiguousarray(v)) if isinstance(v, np.ndarray) else v
            if t.is_floating_point():
                out[k] = t.to(device=device, dtype=dtype).contiguous()
            elif t.numel() == 1 and k in ("max_ns_rank", "infeatures", "outfeatures", "group_size"):
                out[k] = int(t.reshape(-1)[0].item())
            else:
                out[k] = t.to(device=device, dtype=torch.int32).contiguous()
        else:
            out[k] = v
    return out


def _resolve_ns_payload(ns_payload):
    """A device null-space payload with a compensation term, else None.  Module lists carry no matrix-mode
    compensation in this build (its QuantLinear holds vector-mode scales only), so they give None."""
    if ns_payload is None or isinstance(ns_payload, (list, tuple)):
        return None
    if not isinstance(ns_payload, dict) or "ns_rank_per_expert" not in ns_payload:
        raise RuntimeError("null-space payload lacks ns_rank_per_expert (build_grouped_ns_payload format)")
    return ns_payload if int(ns_payload["max_ns_rank"]) > 0 else None


def _apply_ns(out, x_grouped, route, ns):
    if ns is not None:
        ext.ns_compensation_apply_(out, x_grouped.contiguous(), route["expert_ids"], route["segment_offsets"], ns)


def _ns_route_inputs_ok(t: torch.Tensor, route) -> bool:
    if route is None or t.device.type != "cuda" or t.dtype != torch.float16 or t.dim() != 2:
        return False
    gexp = route.get("grouped_expert_ids")
    return gexp is not None and gexp.numel() == t.size(0)


def run_grouped_ns_compensation_forward(payload_or_modules, x_grouped: torch.Tensor, grouped_route_or_segment_lengths,
                                        expert_modules=None, expert_ids=None, prefer_fused_decode: bool = False):
    """qlinear_cuda.py:2028-2128: the grouped compensation C1_e . fp16(C2_e . x) per routed row as a new
    fp16 [R, out] tensor, or None when the inputs are outside the kernel contract or there is no
    matrix-mode payload (module lists carry none in this build).  prefer_fused_decode selects the
    reference's fused decode kernel there; the result is the same, and here one path serves both."""
    route = _coerce_grouped_route(grouped_route_or_segment_lengths, x_grouped.device, expert_ids=expert_ids)
    if not _ns_route_inputs_ok(x_grouped, route):
        return None
    ns = _resolve_ns_payload(payload_or_modules)
    if ns is None:
        return None
    out = torch.empty((x_grouped.size(0), int(ns["ns_c1_scales"].size(1))), dtype=torch.float16,
                      device=x_grouped.device)
    return ext.ns_compensation_apply_(out, x_grouped.contiguous(), route["expert_ids"], route["segment_offsets"], ns,
                                      accumulate=False)


def run_grouped_ns_c1_forward(payload_or_modules, hidden_grouped: torch.Tensor, grouped_route_or_segment_lengths,
                              expert_modules=None, expert_ids=None):
    """qlinear_cuda.py:1964-2025: C1_e . hidden[r][0:rank_e] per routed row for a hidden [R, max_ns_rank]
    computed elsewhere (the shared C2 projection), as a new fp16 [R, out] tensor, or None as above."""
    route = _coerce_grouped_route(grouped_route_or_segment_lengths, hidden_grouped.device, expert_ids=expert_ids)
    if not _ns_route_inputs_ok(hidden_grouped, route):
        return None
    ns = _resolve_ns_payload(payload_or_modules)
    if ns is None:
        return None
    return ext.grouped_ns_c1_forward(
        hidden_grouped.contiguous(), route["expert_ids"], route["segment_offsets"], route["problem_offsets"],
        _route_total_problem_tiles_host(route), ns["ns_rank_per_expert"], ns["ns_c1_rank_word_offsets"],
        ns["ns_c1_group_offsets"], ns["ns_c1_qweight"], ns["ns_c1_qzeros"], ns["ns_c1_scales"], int(ns["max_ns_rank"]),
        int(ns["group_size"]))


def run_grouped_structured_expert_forward(payload_or_modules, hidden_grouped: torch.Tensor, x_grouped: torch.Tensor,
                                          grouped_route_or_segment_lengths, expert_modules=None, expert_ids=None,
                                          ns_payload=None, prefer_ns_fused_decode: bool = False):
    """qlinear_cuda.py:2131-2335.  Returns fp16 [R, N] or None when the inputs are outside the
    kernel contract (non-CUDA / non-fp16 / shape mismatch), as the reference does."""
    if hidden_grouped.device.type != "cuda" or hidden_grouped.dtype != torch.float16:
        return None
    if x_grouped.device != hidden_grouped.device or x_grouped.dtype != hidden_grouped.dtype:
        return None
    if hidden_grouped.dim() != 2 or x_grouped.dim() != 2 or hidden_grouped.size(0) != x_grouped.size(0):
        return None
    route = _coerce_grouped_route(grouped_route_or_segment_lengths, hidden_grouped.device, expert_ids)
    gti = route.get("grouped_token_indices")
    if gti is not None and gti.numel() not in (0, hidden_grouped.size(0)):
        return None
    payload = resolve_grouped_precomputed_payload(payload_or_modules, hidden_grouped.device, hidden_grouped.dtype)
    if payload is None:
        return None
    ns = _resolve_ns_payload(ns_payload)
    if expert_modules is None and not isinstance(payload_or_modules, dict):
        expert_modules = payload_or_modules
    defer_bias = bool(payload["has_bias"]) and (ns_payload is not None or expert_modules is not None)
    has_bias_arg = bool(payload["has_bias"]) and not defer_bias
    bias_arg = payload["bias"] if has_bias_arg else hidden_grouped.new_empty((0, 0))
    has_scale = _payload_has_output_scale(payload)
    batch = int(hidden_grouped.size(0))
    rank = int(hidden_grouped.size(1))
    n = int(payload["qweight1"].size(2))
    total = _route_total_problem_tiles_host(route)
    uniform = _k64_uniform(payload)
    hidden_c = hidden_grouped.contiguous()
    if is_sparse_payload(payload):
        out = ext.compact3_tris_precomputed_grouped_forward(
            hidden_c, route["expert_ids"], route["segment_offsets"], route["problem_offsets"], total,
            payload["qweight1"], payload["qweight2_sparse"], payload["qweight2_sparse_prefix"],
            payload["q_gmap_sparse"], payload["q_gmap_sparse_prefix"], payload["c_map"], payload["g_idx"],
            payload["col_pack3"], payload["row_pack3"], payload["output_scale"], bias_arg, has_bias_arg)
    elif _use_predecode(batch, int(route["expert_ids"].numel()), payload, has_scale, has_bias_arg):
        decoded = _predecode(payload, route, rank, n)
        out = ext.compact3_tris_precomputed_grouped_forward_block_gr_predecoded(
            hidden_c, route["expert_ids"], route["segment_offsets"], route["problem_offsets"], total, decoded,
            payload["qweight1"], payload["qweight2_sparse"], payload["qweight2_sparse_prefix"], payload["c_map"],
            payload["g_idx"], payload["col_pack3"], payload["row_pack3"], uniform)
    else:
        out = ext.compact3_tris_precomputed_grouped_forward_block_gr(
            hidden_c, route["expert_ids"], route["segment_offsets"], route["problem_offsets"], total,
            payload["qweight1"], payload["qweight2_sparse"], payload["qweight2_sparse_prefix"],
            payload["q_gmap_gr_words"], payload["q_gmap_gr_offsets"], payload["q_gmap_gr_meta"], payload["c_map"],
            payload["g_idx"], payload["col_pack3"], payload["row_pack3"], payload["output_scale"], has_scale,
            bias_arg, has_bias_arg, uniform)
    _apply_ns(out, x_grouped, route, ns)
    if defer_bias:
        out.add_(payload["bias"].index_select(0, route["grouped_expert_ids"].to(dtype=torch.long)))
    return out


def run_grouped_structured_expert_pair_forward(payload_or_modules_a, payload_or_modules_b, hidden_a_grouped,
                                               hidden_b_grouped, x_grouped, grouped_route_or_segment_lengths,
                                               expert_modules_a=None, expert_modules_b=None, expert_ids=None,
                                               ns_payload_a=None, ns_payload_b=None):
    """qlinear_cuda.py:2338-2634: gate and up projections sharing one route, one launch.
    Returns (out_a, out_b) or (None, None) outside the kernel contract."""
    for h in (hidden_a_grouped, hidden_b_grouped):
        if h.device.type != "cuda" or h.dtype != torch.float16 or h.dim() != 2:
            return None, None
    if hidden_a_grouped.size(0) != hidden_b_grouped.size(0) or x_grouped.size(0) != hidden_a_grouped.size(0):
        return None, None
    route = _coerce_grouped_route(grouped_route_or_segment_lengths, hidden_a_grouped.device, expert_ids)
    pa = resolve_grouped_precomputed_payload(payload_or_modules_a, hidden_a_grouped.device, hidden_a_grouped.dtype)
    pb = resolve_grouped_precomputed_payload(payload_or_modules_b, hidden_b_grouped.device, hidden_b_grouped.dtype)
    if pa is None or pb is None:
        return None, None
    if is_sparse_payload(pa) or is_sparse_payload(pb):
        # no pair entry for sparse split bitmaps: one launch per projection (qlinear_cuda.py:2381-2411)
        out_a = run_grouped_structured_expert_forward(pa, hidden_a_grouped, x_grouped, route, expert_modules_a,
                                                      ns_payload=ns_payload_a)
        out_b = run_grouped_structured_expert_forward(pb, hidden_b_grouped, x_grouped, route, expert_modules_b,
                                                      ns_payload=ns_payload_b)
        return out_a, out_b
    ns_a = _resolve_ns_payload(ns_payload_a)
    ns_b = _resolve_ns_payload(ns_payload_b)
    if expert_modules_a is None and not isinstance(payload_or_modules_a, dict):
        expert_modules_a = payload_or_modules_a
    if expert_modules_b is None and not isinstance(payload_or_modules_b, dict):
        expert_modules_b = payload_or_modules_b
    defer_a = bool(pa["has_bias"]) and (ns_payload_a is not None or expert_modules_a is not None)
    defer_b = bool(pb["has_bias"]) and (ns_payload_b is not None or expert_modules_b is not None)
    empty = hidden_a_grouped.new_empty((0, 0))
    bias_a = pa["bias"] if pa["has_bias"] and not defer_a else empty
    bias_b = pb["bias"] if pb["has_bias"] and not defer_b else empty
    scale_a = _payload_has_output_scale(pa)
    scale_b = _payload_has_output_scale(pb)
    batch = int(hidden_a_grouped.size(0))
    total = _route_total_problem_tiles_host(route)
    uniform = _k64_uniform(pa) and _k64_uniform(pb)
    nseg = int(route["expert_ids"].numel())
    ha = hidden_a_grouped.contiguous()
    hb = hidden_b_grouped.contiguous()
    if (_use_predecode(batch, nseg, pa, scale_a, bias_a.numel() > 0)
            and _use_predecode(batch, nseg, pb, scale_b, bias_b.numel() > 0)):
        da = _predecode(pa, route, int(ha.size(1)), int(pa["qweight1"].size(2)))
        db = _predecode(pb, route, int(hb.size(1)), int(pb["qweight1"].size(2)))
        out_a, out_b = ext.compact3_tris_precomputed_grouped_dual_forward_block_gr_predecoded(
            ha, hb, route["expert_ids"], route["segment_offsets"], route["problem_offsets"], total,
            da, pa["qweight1"], pa["qweight2_sparse"], pa["qweight2_sparse_prefix"], pa["c_map"], pa["g_idx"],
            pa["col_pack3"], pa["row_pack3"], db, pb["qweight1"], pb["qweight2_sparse"],
            pb["qweight2_sparse_prefix"], pb["c_map"], pb["g_idx"], pb["col_pack3"], pb["row_pack3"], uniform)
    else:
        out_a, out_b = ext.compact3_tris_precomputed_grouped_dual_forward_block_gr(
            ha, hb, route["expert_ids"], route["segment_offsets"], route["problem_offsets"], total,
            pa["qweight1"], pa["qweight2_sparse"], pa["qweight2_sparse_prefix"], pa["q_gmap_gr_words"],
            pa["q_gmap_gr_offsets"], pa["q_gmap_gr_meta"], pa["c_map"], pa["g_idx"], pa["col_pack3"],
            pa["row_pack3"], pa["output_scale"], scale_a, bias_a,
            pb["qweight1"], pb["qweight2_sparse"], pb["qweight2_sparse_prefix"], pb["q_gmap_gr_words"],
            pb["q_gmap_gr_offsets"], pb["q_gmap_gr_meta"], pb["c_map"], pb["g_idx"], pb["col_pack3"],
            pb["row_pack3"], pb["output_scale"], scale_b, bias_b, uniform)
    if ns_a is not None or ns_b is not None:
        ext.ns_compensation_pair_apply_(out_a, out_b, x_grouped.contiguous(), route["expert_ids"],
                                        route["segment_offsets"], ns_a, ns_b)
    gexp = route["grouped_expert_ids"].to(dtype=torch.long)
    if defer_a:
        out_a.add_(pa["bias"].index_select(0, gexp))
    if defer_b:
        out_b.add_(pb["bias"].index_select(0, gexp))
    return out_a, out_b


# --------------------------------------------------------------- modules
def pack_block_gr_gmap_tensor(packed: torch.Tensor, force_raw: bool = False, fixed_k=None, k_min=None, k_max=None):
    """tools/rewrite_runtime_min_checkpoint.py:252-347 (and QuantLinear._pack_block_gr_gmap_tensor):
    dense packed split bitmap [packed_rows, N] -> (words, offsets, meta) int32 tensors on packed.device."""
    if fixed_k is not None:
        if k_min is not None or k_max is not None:
            raise ValueError("--blockgr-k cannot be combined with --blockgr-k-min/--blockgr-k-max")
        if not 0 <= fixed_k <= BLOCK_GR_MAX_K:
            raise ValueError(f"--blockgr-k must be in [0, {BLOCK_GR_MAX_K}], got {fixed_k}")
        lo, hi = fixed_k, fixed_k
    elif k_min is None and k_max is None:
        lo, hi = 0, BLOCK_GR_MAX_K
    elif k_min is None or k_max is None:
        raise ValueError("--blockgr-k-min and --blockgr-k-max must be provided together")
    else:
        if not 0 <= k_min <= k_max <= BLOCK_GR_MAX_K:
            raise ValueError(f"--blockgr-k-min/--blockgr-k-max must satisfy 0 <= min <= max <= {BLOCK_GR_MAX_K}")
        lo, hi = k_min, k_max
    if packed.numel() == 0:
        empty = torch.zeros((0,), dtype=torch.int32, device=packed.device)
        return empty, empty, empty
    words, offsets, meta = ext.gr_encode(packed.detach().to("cpu", torch.int32), lo, hi, force_raw)
    dev = packed.device
    return (torch.from_numpy(words).to(dev), torch.from_numpy(offsets).to(dev), torch.from_numpy(meta).to(dev))


class PackedQuantMatrix4bit(nn.Module):
    """qlinear_cuda.py:2637-2786: a 4-bit packed matrix [rows, cols] (the shared backbone SV of real
    checkpoints): qweight int32 [ceil(cols/8), rows], qzeros int32 [G, ceil(rows/8)], scales [G, rows],
    g_idx int32 [cols]; W[r][c] = (q - z) * s (see ``ext.packed4_dequant``).

    ``project`` computes x . W^T on the GPU: the fused 4-bit kernel for uniform groups below
    ``ext.BACKBONE_LIBRARY_MIN_ROWS`` rows, else the cached dequantised matrix through the fp16 path."""

    def __init__(self, weight_dtype=torch.float16):
        super().__init__()
        self.register_buffer("qweight", torch.zeros((0, 0), dtype=torch.int32))
        self.register_buffer("qzeros", torch.zeros((0, 0), dtype=torch.int32))
        self.register_buffer("scales", torch.zeros((0, 0), dtype=weight_dtype))
        self.register_buffer("g_idx", torch.zeros((0,), dtype=torch.int32))
        self.register_buffer("rows", torch.zeros((), dtype=torch.int32))
        self.register_buffer("cols", torch.zeros((), dtype=torch.int32))
        self._rows_host = 0
        self._cols_host = 0
        self._group_size = 0
        self._cached_weight = None
        self._cached_weight_key = None

    def _apply(self, fn):
        super()._apply(fn)
        self.invalidate_cache()
        return self

    def invalidate_cache(self):
        self._cached_weight = None
        self._cached_weight_key = None

    def set_empty(self):
        self.set_quantized(torch.zeros((0, 0), dtype=torch.int32), torch.zeros((0, 0), dtype=torch.int32),
                           torch.zeros((0, 0), dtype=self.scales.dtype), torch.zeros((0,), dtype=torch.int32), 0, 0)

    def is_quantized(self) -> bool:
        return self.qweight.numel() > 0 and self._rows_host > 0 and self._cols_host > 0

    def set_quantized(self, qweight, qzeros, scales, g_idx, rows=None, cols=None):
        """qlinear_cuda.py:2726-2743; rows default to scales.shape[1], cols to g_idx.numel()."""
        def as_t(v):
            return torch.as_tensor(np.ascontiguousarray(v)) if isinstance(v, np.ndarray) else v
        self.qweight = as_t(qweight).to(torch.int32).contiguous()
        self.qzeros = as_t(qzeros).to(torch.int32).contiguous()
        self.scales = as_t(scales).to(dtype=self.scales.dtype).contiguous()
        self.g_idx = as_t(g_idx).to(torch.int32).contiguous()
        n_rows = int(rows.item()) if isinstance(rows, torch.Tensor) else rows
        n_cols = int(cols.item()) if isinstance(cols, torch.Tensor) else cols
        if n_rows is None:
            n_rows = self.scales.shape[1] if self.scales.dim() == 2 else 0
        if n_cols is None:
            n_cols = self.g_idx.numel()
        self.rows = torch.tensor(int(n_rows), dtype=torch.int32)
        self.cols = torch.tensor(int(n_cols), dtype=torch.int32)
        self._rows_host = int(n_rows)
        self._cols_host = int(n_cols)
        self._group_size = ext.uniform_group_size(self.g_idx) if self.g_idx.numel() else 0
        self.invalidate_cache()
        return self

    def set_from_payload(self, payload, device=None):
        """qlinear_cuda.py:2745-2759 (a payload of build_packed_4bit_payload, utils/pack_utils.py:126-180)."""
        if payload is None or not isinstance(payload, dict) or "qweight" not in payload:
            self.set_empty()
            return self
        self.set_quantized(payload["qweight"], payload["qzeros"], payload["scales"], payload["g_idx"],
                           payload.get("rows"), payload.get("cols"))
        if device is not None:
            self.to(device)
        return self

    @property
    def group_size(self) -> int:
        return self._group_size

    def matrix(self) -> ext.Packed4Matrix:
        return ext.Packed4Matrix(self.qweight, self.qzeros, self.scales, self.g_idx, self._rows_host,
                                 self._cols_host, self._group_size)

    def dequantize(self, device, dtype) -> torch.Tensor:
        """qlinear_cuda.py:2761-2786 on the GPU (fp16: the HIP kernel, bit for bit; cached)."""
        device = torch.device(device)
        key = (device.type, device.index, dtype)
        if self._cached_weight is not None and self._cached_weight_key == key:
            return self._cached_weight
        if self._rows_host == 0 or self._cols_host == 0:
            w = torch.zeros((self._rows_host, self._cols_host), device=device, dtype=dtype)
        else:
            if self.qweight.device != device:
                self.to(device)
            w = ext.packed4_dequant(self.matrix())
            if dtype != torch.float16:
                w = w.to(dtype)
        self._cached_weight = w
        self._cached_weight_key = key
        return w

    def fused_ok(self, tokens: int) -> bool:
        return self._group_size > 0 and tokens < ext.BACKBONE_LIBRARY_MIN_ROWS

    def project(self, x: torch.Tensor, in_scale: torch.Tensor | None = None,
                row_index: torch.Tensor | None = None) -> torch.Tensor:
        """hidden = fp16(x[row_index] * in_scale) . W^T (compute_shared_hidden with a packed SV,
        qlinear_cuda.py:4487-4494)."""
        tokens = int(row_index.numel()) if row_index is not None else int(x.size(0))
        if self.fused_ok(tokens):
            return ext.packed4_backbone_linear(x, self.matrix(), in_scale=in_scale, row_index=row_index)
        return ext.backbone_linear(x, self.dequantize(x.device, torch.float16), in_scale=in_scale,
                                   row_index=row_index)


def shared_projection(x: torch.Tensor, sv, in_scale: torch.Tensor | None = None,
                      row_index: torch.Tensor | None = None) -> torch.Tensor:
    """The shared backbone of one projection: sv is an fp16 SV [rank, in] or a PackedQuantMatrix4bit."""
    if isinstance(sv, PackedQuantMatrix4bit):
        return sv.project(x, in_scale=in_scale, row_index=row_index)
    return ext.backbone_linear(x, sv, in_scale=in_scale, row_index=row_index)


def shared_projection_pair(x: torch.Tensor, sv_a, sv_b, row_index: torch.Tensor | None = None,
                           in_scale_a: torch.Tensor | None = None, in_scale_b: torch.Tensor | None = None):
    """Gate and up backbones of the same rows, each with its own ns_mode == 1 input scale (or None): one launch
    for two fp16 matrices or two fused-capable packed matrices of one shape, else two projections."""
    tokens = int(row_index.numel()) if row_index is not None else int(x.size(0))
    if isinstance(sv_a, torch.Tensor) and isinstance(sv_b, torch.Tensor):
        return ext.backbone_linear_pair(x, sv_a, sv_b, row_index=row_index, in_scale_a=in_scale_a,
                                        in_scale_b=in_scale_b)
    if (isinstance(sv_a, PackedQuantMatrix4bit) and isinstance(sv_b, PackedQuantMatrix4bit)
            and sv_a.fused_ok(tokens) and sv_b.fused_ok(tokens) and sv_a.group_size == sv_b.group_size
            and (sv_a._rows_host, sv_a._cols_host) == (sv_b._rows_host, sv_b._cols_host)
            and sv_a.scales.shape == sv_b.scales.shape):
        return ext.packed4_backbone_linear_pair(x, sv_a.matrix(), sv_b.matrix(), row_index=row_index,
                                                in_scale_a=in_scale_a, in_scale_b=in_scale_b)
    return (shared_projection(x, sv_a, in_scale=in_scale_a, row_index=row_index),
            shared_projection(x, sv_b, in_scale=in_scale_b, row_index=row_index))


class ExpertSharedMatrix(nn.Module):
    """qlinear_cuda.py:2787-2968: the shared backbone SV [rank, in] of one (layer, projection), either fp16
    (``shared_sv``) or 4-bit packed (``shared_sv_quant``)."""

    def __init__(self, shared_sv=None):
        super().__init__()
        self.register_buffer("shared_sv", torch.zeros((0, 0), dtype=torch.float16))
        self.shared_sv_quant = PackedQuantMatrix4bit()
        if shared_sv is not None:
            self.set_shared_sv(shared_sv)

    def set_shared_sv(self, payload):
        """qlinear_cuda.py:2944-2953: a packed payload dict (with ``qweight``) or an fp16 matrix."""
        if isinstance(payload, dict) and "qweight" in payload:
            self.shared_sv = torch.zeros((0, 0), dtype=torch.float16)
            self.shared_sv_quant.set_from_payload(payload)  # the payload's tensors keep their device
        else:
            self.shared_sv_quant.set_empty()
            self.shared_sv = torch.as_tensor(payload).to(dtype=torch.float16).contiguous()
        return self

    def get_shared_sv(self, device, dtype):
        if self.shared_sv_quant.is_quantized():
            return self.shared_sv_quant.dequantize(device, dtype)
        sv = self.shared_sv
        if sv.device != torch.device(device) or sv.dtype != dtype:
            sv = sv.to(device=device, dtype=dtype).contiguous()
        return sv

    def backbone(self, device):
        """What shared_projection takes: the packed matrix (moved to device) or the fp16 SV."""
        if self.shared_sv_quant.is_quantized():
            if self.shared_sv_quant.qweight.device != torch.device(device):
                self.shared_sv_quant.to(device)
            return self.shared_sv_quant
        return self.get_shared_sv(device, torch.float16)


class QuantLinear(nn.Module):
    """Expert compact3 linear (mode 5) with its shared backbone: W = B_e . SV.

    Holds one expert's packed tensors (``expert_*`` buffers, qlinear_cuda.py:2971+) and its
    block-GR split bitmap; ``forward(x) = forward_from_precomputed_hidden(compute_shared_hidden(x), x)``.
    """

    QUANT_TYPE = "hip"

    def __init__(self, infeatures: int, outfeatures: int, rank: int, shared: ExpertSharedMatrix, bias=None,
                 expert_input_scale=None):
        super().__init__()
        self.infeatures = infeatures
        self.outfeatures = outfeatures
        self.rank = rank
        self._shared_matrix_module = shared
        self._mode_host = 5
        self._ns_mode_host = 1 if expert_input_scale is not None else 0
        self.register_buffer("expert_input_scale", expert_input_scale)
        self.register_buffer("bias", bias)
        self.register_buffer("ns_vector_row", torch.ones(outfeatures, dtype=torch.float16))

    def load_expert_payload(self, tensors: dict):
        """Set the expert_* buffers from one expert's packed tensors (host numpy or torch)."""
        for key in ("qweight1", "qweight2_sparse", "qweight2_sparse_prefix", "c_map", "g_idx", "col_pack3",
                    "row_pack3"):
            val = tensors[key]
            t = torch.as_tensor(np.ascontiguousarray(val)) if isinstance(val, np.ndarray) else val
            self.register_buffer("expert_" + key, t.clone())
        if "gmap_dense" in tensors:
            dense = torch.as_tensor(np.ascontiguousarray(tensors["gmap_dense"]))
            words, offsets, meta = pack_block_gr_gmap_tensor(dense)
        else:
            words, offsets, meta = (torch.as_tensor(tensors[k]) for k in ("q_gmap_gr_words", "q_gmap_gr_offsets",
                                                                           "q_gmap_gr_meta"))
        self.register_buffer("expert_q_gmap_gr_words", words)
        self.register_buffer("expert_q_gmap_gr_offsets", offsets)
        self.register_buffer("expert_q_gmap_gr_meta", meta)
        return self

    def can_precompute_shared(self) -> bool:
        return self._mode_host == 5 and self._shared_matrix_module is not None

    def compute_shared_hidden(self, x: torch.Tensor):
        """hidden = (x * s_in) . SV^T (qlinear_cuda.py:4454-4502, fp16 backbone branch)."""
        if not self.can_precompute_shared():
            return None
        shape = x.shape[:-1]
        xb = x.reshape(-1, x.shape[-1]).contiguous()
        sv = self._shared_matrix_module.backbone(xb.device)
        rank = sv._rows_host if isinstance(sv, PackedQuantMatrix4bit) else sv.shape[0]
        if xb.shape[0] == 0:
            return xb.new_empty((0, rank)).reshape(shape + (rank,))
        scale = None
        if self._ns_mode_host == 1:
            scale = self.expert_input_scale.to(device=xb.device, dtype=xb.dtype).contiguous()
        hidden = shared_projection(xb, sv, in_scale=scale)
        return hidden.reshape(shape + (hidden.shape[-1],))

    def _single_payload(self, device, dtype) -> dict:
        key = (str(device), dtype)
        cache = getattr(self, "_payload_cache", None)
        if cache is not None and cache[0] == key:
            return cache[1]
        payload = build_grouped_precomputed_payload([self], device, dtype)
        self._payload_cache = (key, payload)
        return payload

    def forward_from_precomputed_hidden(self, hidden: torch.Tensor, x_base: torch.Tensor):
        """qlinear_cuda.py:4504-4560 for one expert: a one-segment grouped call."""
        out_shape = hidden.shape[:-1] + (self.outfeatures,)
        hf = hidden.reshape(-1, hidden.shape[-1]).contiguous()
        xf = x_base.reshape(-1, x_base.shape[-1]).contiguous()
        if hf.shape[0] == 0:
            return hf.new_empty((0, self.outfeatures)).reshape(out_shape)
        payload = self._single_payload(hf.device, hf.dtype)
        # ns_vector_row is the payload's output_scale, applied in the kernel epilogue.
        out = run_grouped_structured_expert_forward(payload, hf, xf, [hf.shape[0]])
        if out is None:
            raise RuntimeError("QuantLinear.forward_from_precomputed_hidden: grouped kernel rejected the inputs")
        return out.reshape(out_shape)

    def forward(self, x: torch.Tensor):
        hidden = self.compute_shared_hidden(x)
        return self.forward_from_precomputed_hidden(hidden, x)


# ------------------------------------------------------------------ non-expert compact3 linears
COMPACT3_MODULE_KEYS = ("qweight1", "qweight2_sparse", "qweight2_sparse_prefix", "q_gmap_gr_words",
                        "q_gmap_gr_offsets", "q_gmap_gr_meta", "c_map", "g_idx", "col_pack3", "row_pack3")


class Compact3Linear(nn.Module):
    """A non-expert compact3 linear (the reference's QuantLinear in compact3 mode 4, qlinear_cuda.py:4238-4360):
    y = fp16((x' . W^T + C1 . (C2 . x)) * output_scale + bias) with W the block-GR compact3 matrix over the
    full input width, x' = fp16(x * input_scale) when an input scale is set, the null-space term when packed
    C1 / C2 matrices are set.  Attention projections and dense (shared-expert) MLPs use it."""

    def __init__(self, infeatures: int, outfeatures: int):
        super().__init__()
        self.infeatures = int(infeatures)
        self.outfeatures = int(outfeatures)
        self._mode_host = 4
        self._ns_mode_host = 0
        for key in COMPACT3_MODULE_KEYS:
            self.register_buffer(key, torch.empty(0, dtype=torch.int64 if key.endswith("pack3") else torch.int32))
        self.register_buffer("input_scale", None)
        self.register_buffer("output_scale", None)
        self.register_buffer("bias", None)
        self.ns_c1 = None
        self.ns_c2 = None

    def load_tensors(self, tensors: dict):
        """Set the packed buffers from host arrays or tensors (the module's checkpoint keys); optional
        input_scale, output_scale, bias, and ns_c1 / ns_c2 as pack_4bit dicts (qweight, qzeros, scales, g_idx)."""
        conv = lambda v, dt: v.to(dtype=dt) if isinstance(v, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(v)).to(dt)
        for key in COMPACT3_MODULE_KEYS:
            setattr(self, key, conv(tensors[key], torch.int64 if key.endswith("pack3") else torch.int32))
        for key in ("input_scale", "output_scale", "bias"):
            if tensors.get(key) is not None:
                setattr(self, key, conv(tensors[key], torch.float16))
        for key in ("ns_c1", "ns_c2"):
            if tensors.get(key) is not None:
                setattr(self, key, {k: conv(v, torch.float16 if k == "scales" else torch.int32)
                                    for k, v in tensors[key].items()})
        self._ns_mode_host = 2 if self.ns_c1 is not None and self.ns_c2 is not None else 0
        return self

    def _apply(self, fn, *args, **kwargs):
        super()._apply(fn, *args, **kwargs)
        for key in ("ns_c1", "ns_c2"):
            d = getattr(self, key)
            if d is not None:
                setattr(self, key, {k: fn(v) for k, v in d.items()})
        return self

    def _compact3_k64_groups_uniform(self) -> bool:
        g = self.g_idx.reshape(1, -1)
        rank = int(g.size(1))
        return bool(torch.equal(g[:, (torch.arange(rank, device=g.device) // 64) * 64], g)) if rank else True

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape[:-1] + (self.outfeatures,)
        x2 = x.reshape(-1, self.infeatures).to(torch.float16).contiguous()
        empty = x2.new_empty((0,))
        ns = self._ns_mode_host == 2
        c1, c2 = (self.ns_c1, self.ns_c2) if ns else ({}, {})
        y = ext.compact3_linear_forward(
            x2, *[getattr(self, key) for key in COMPACT3_MODULE_KEYS[:3]], empty, empty,
            *[getattr(self, key) for key in COMPACT3_MODULE_KEYS[3:]],
            self.input_scale if self.input_scale is not None else empty,
            self.output_scale if self.output_scale is not None else empty,
            self.bias if self.bias is not None else empty,
            self.input_scale is not None, self.output_scale is not None, self.bias is not None,
            *[c1.get(k, empty) for k in ("qweight", "qzeros", "scales", "g_idx")],
            *[c2.get(k, empty) for k in ("qweight", "qzeros", "scales", "g_idx")], ns, 1, False,
            self._compact3_k64_groups_uniform())
        return y.reshape(shape)


def _plain_compact3(module, outfeatures=None, allow_bias=False) -> bool:
    """The fused Q/K/V and gate/up launches take modules without scales or a null-space term
    (qlinear_cuda.py:873-912)."""
    return (isinstance(module, Compact3Linear) and module._ns_mode_host == 0 and module.input_scale is None
            and module.output_scale is None and (allow_bias or module.bias is None)
            and (outfeatures is None or module.outfeatures == outfeatures))


def run_compact3_qkv_block_gr_forward(q_proj, k_proj, v_proj, hidden_states: torch.Tensor):
    """qlinear_cuda.py:915-1002: (q, k, v) of one input through the fused Q/K/V binding, or None when the
    modules or the input fall outside it (the caller then runs the three modules)."""
    if hidden_states.device.type != "cuda" or hidden_states.dtype != torch.float16:
        return None
    if hidden_states.shape[-1] != getattr(q_proj, "infeatures", None):
        return None
    n = getattr(q_proj, "outfeatures", None)
    if not all(_plain_compact3(m, n, allow_bias=True) for m in (q_proj, k_proj, v_proj)):
        return None
    shape = hidden_states.shape[:-1] + (n,)
    x = hidden_states.reshape(-1, hidden_states.shape[-1]).contiguous()
    empty = x.new_empty((0,))
    args = []
    for m in (q_proj, k_proj, v_proj):
        args += [getattr(m, key) for key in COMPACT3_MODULE_KEYS] + [m.bias if m.bias is not None else empty]
    fused = ext.compact3_qkv_linear_forward(x, *args, 1, all(m._compact3_k64_groups_uniform()
                                                            for m in (q_proj, k_proj, v_proj)))
    return tuple(fused[i].reshape(shape) for i in range(3))


def run_compact3_shared_expert_gate_up_forward(gate_proj, up_proj, hidden_states: torch.Tensor):
    """qlinear_cuda.py:1005-1098: (gate, up) of one input through the dual binding, or None as above."""
    if hidden_states.device.type != "cuda" or hidden_states.dtype != torch.float16:
        return None
    if hidden_states.shape[-1] != getattr(gate_proj, "infeatures", None):
        return None
    n = getattr(gate_proj, "outfeatures", None)
    if not (_plain_compact3(gate_proj, n) and _plain_compact3(up_proj, n)):
        return None
    shape = hidden_states.shape[:-1] + (n,)
    x = hidden_states.reshape(-1, hidden_states.shape[-1]).contiguous()
    fused = ext.compact3_dual_linear_forward(x, *[getattr(gate_proj, k) for k in COMPACT3_MODULE_KEYS],
                                             *[getattr(up_proj, k) for k in COMPACT3_MODULE_KEYS], 1,
                                             gate_proj._compact3_k64_groups_uniform()
                                             and up_proj._compact3_k64_groups_uniform())
    return fused[0].reshape(shape), fused[1].reshape(shape)


def build_grouped_precomputed_payload(modules, device, dtype):
    """qlinear_cuda.py:1512-1636: stack per-expert buffers (zero-padding ragged qweight2_sparse and
    GR words) into the grouped payload dict."""
    if len(modules) == 0:
        return None
    for m in modules:
        if not isinstance(m, QuantLinear) or m._mode_host != 5:
            return None
    dev = torch.device(device)

    def stack(name, dt=torch.int32, pad_rows=False, pad_cols=False):
        ts = [getattr(m, "expert_" + name).to(device=dev, dtype=dt) for m in modules]
        if pad_rows:
            rows = max(int(t.shape[0]) for t in ts)
            ts = [torch.nn.functional.pad(t, (0, 0, 0, rows - int(t.shape[0]))) for t in ts]
        if pad_cols:
            cols = max(int(t.shape[0]) for t in ts)
            ts = [torch.nn.functional.pad(t, (0, cols - int(t.shape[0]))) for t in ts]
        return torch.stack(ts, 0).contiguous()

    output_scale = torch.stack([m.ns_vector_row.to(device=dev, dtype=dtype) for m in modules], 0).contiguous()
    if output_scale.numel() > 0 and bool(torch.all(output_scale == 0).item()):
        output_scale = torch.ones_like(output_scale)
    has_bias = any(m.bias is not None for m in modules)
    bias = None
    if has_bias:
        bias = torch.stack([m.bias.to(device=dev, dtype=dtype) if m.bias is not None
                            else torch.zeros(m.outfeatures, device=dev, dtype=dtype) for m in modules], 0)
    payload = {
        "is_compact3": True,
        "qweight1": stack("qweight1"),
        "qweight2_sparse": stack("qweight2_sparse", pad_rows=True),
        "qweight2_sparse_prefix": stack("qweight2_sparse_prefix"),
        "compact3_use_block_gr": True,
        "q_gmap_gr_words": stack("q_gmap_gr_words", pad_cols=True),
        "q_gmap_gr_offsets": stack("q_gmap_gr_offsets"),
        "q_gmap_gr_meta": stack("q_gmap_gr_meta"),
        "c_map": stack("c_map"),
        "g_idx": stack("g_idx"),
        "col_pack3": stack("col_pack3", torch.int64),
        "row_pack3": stack("row_pack3", torch.int64),
        "output_scale": output_scale,
        "has_output_scale": not bool(torch.all(output_scale == 1).item()),
        "bias": bias,
        "has_bias": has_bias,
    }
    _k64_uniform(payload)
    return payload
