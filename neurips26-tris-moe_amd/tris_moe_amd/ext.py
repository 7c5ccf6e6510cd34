"""Drop-in for the reference's native module ``autogptq_TriS_cuda`` on the grouped expert path.

Every function keeps the pybind name, argument order and defaults of
``TriSMoE_cuda.cpp:1138-1430`` for the block-GR paths and returns
freshly allocated torch tensors exactly as the reference does, but computes
through the gfx950 HIP kernels of libtris_moe_hip.so (C ABI, via ctypes).
Argument contracts mirror the reference's ``CHECK_*`` / ``TORCH_CHECK``
macros (``TriSMoE_cuda_kernel.cu:49-54``, ``:9789-9842``) and raise
``RuntimeError`` like them.  All work is enqueued on torch's current stream of
the input's device.

Besides the grouped expert entry points, the module has the 4-bit packed
backbone (``packed4_linear_forward``), the grouped null-space compensation
(``grouped_ns_*``) and the non-expert compact3 linears
(``compact3_linear_forward``, ``compact3_qkv_linear_forward``,
``compact3_dual_linear_forward``) for block-GR payloads; a sparse split-bitmap
payload raises RuntimeError, which the reference's callers treat as "kernel
unavailable" (convert it to block-GR at load).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import TRIS_COMPACT3_KERNEL_ABI_VERSION, TrisPayload  # noqa: F401

BLOCK_GR_TILE_K = 64
BLOCK_GR_TILE_OUT = 64
BLOCK_GR_PACKED_ROWS = 2
BLOCK_GR_WORDS_PER_BLOCK = 128


def _stream(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _ptr(t):
    if t is None or t.numel() == 0:
        return None
    return ctypes.c_void_p(t.data_ptr())


def _check_cuda(name, t, dtype, dims=None, device=None):
    if not isinstance(t, torch.Tensor):
        raise RuntimeError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if device is not None and t.device != device:
        raise RuntimeError(f"{name} must be on {device}")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")
    if t.dtype != dtype:
        raise RuntimeError(f"{name} must be {dtype}")
    if dims is not None and t.dim() != dims:
        raise RuntimeError(f"{name} must be {dims}D")


def _host_tiles(total_problem_tiles) -> int:
    if isinstance(total_problem_tiles, torch.Tensor):
        if total_problem_tiles.device.type != "cpu":
            raise RuntimeError("total_problem_tiles must be a CPU tensor")
        if total_problem_tiles.numel() != 1:
            raise RuntimeError("total_problem_tiles must contain one value")
        return int(total_problem_tiles.reshape(-1)[0].item())
    return int(total_problem_tiles)


def _num_gr_blocks(packed_rows: int, outfeatures: int) -> int:
    return -(-packed_rows // BLOCK_GR_PACKED_ROWS) * -(-outfeatures // BLOCK_GR_TILE_OUT)


def make_payload_struct(rank, qweight1, qweight2_sparse, qweight2_sparse_prefix, q_gmap_gr_words, q_gmap_gr_offsets,
                        q_gmap_gr_meta, c_map, g_idx, col_pack3, row_pack3, output_scale, has_output_scale, bias,
                        has_bias, use_uniform_k64_groups, device, need_gr=True, who="grouped payload"):
    """Validate one projection's stacked payload (kernel.cu:9789-9842) and pack the C descriptor."""
    _check_cuda("qweight1", qweight1, torch.int32, 3, device)
    _check_cuda("qweight2_sparse", qweight2_sparse, torch.int32, 3, device)
    _check_cuda("qweight2_sparse_prefix", qweight2_sparse_prefix, torch.int32, 2, device)
    _check_cuda("c_map", c_map, torch.int32, 2, device)
    _check_cuda("g_idx", g_idx, torch.int32, 2, device)
    _check_cuda("col_pack3", col_pack3, torch.int64, 2, device)
    _check_cuda("row_pack3", row_pack3, torch.int64, 3, device)
    num_experts = int(qweight1.size(0))
    packed_rows = (rank + 31) // 32
    outfeatures = int(qweight1.size(2))
    num_groups = int(row_pack3.size(2))
    nblk = _num_gr_blocks(packed_rows, outfeatures)
    if int(qweight1.size(1)) != packed_rows:
        raise RuntimeError(f"{who}: qweight1 packed height mismatch")
    if int(qweight2_sparse.size(0)) != num_experts or int(qweight2_sparse.size(2)) != outfeatures:
        raise RuntimeError(f"{who}: qweight2_sparse shape mismatch")
    if tuple(qweight2_sparse_prefix.shape) != (num_experts, packed_rows + 1):
        raise RuntimeError(f"{who}: qweight2 prefix mismatch")
    if tuple(c_map.shape) != (num_experts, packed_rows):
        raise RuntimeError(f"{who}: c_map mismatch")
    if tuple(g_idx.shape) != (num_experts, rank):
        raise RuntimeError(f"{who}: g_idx mismatch")
    if tuple(col_pack3.shape) != (num_experts, rank):
        raise RuntimeError(f"{who}: col_pack3 mismatch")
    if int(row_pack3.size(0)) != num_experts or int(row_pack3.size(1)) != outfeatures:
        raise RuntimeError(f"{who}: row_pack3 mismatch")
    words_stride = 0
    if need_gr:
        _check_cuda("q_gmap_gr_words", q_gmap_gr_words, torch.int32, 2, device)
        _check_cuda("q_gmap_gr_offsets", q_gmap_gr_offsets, torch.int32, 2, device)
        _check_cuda("q_gmap_gr_meta", q_gmap_gr_meta, torch.int32, 2, device)
        if (int(q_gmap_gr_words.size(0)) != num_experts or int(q_gmap_gr_offsets.size(0)) != num_experts
                or int(q_gmap_gr_meta.size(0)) != num_experts):
            raise RuntimeError(f"{who}: block-GR expert mismatch")
        if int(q_gmap_gr_offsets.size(1)) != nblk + 1:
            raise RuntimeError(f"{who}: q_gmap_gr_offsets shape mismatch")
        if int(q_gmap_gr_meta.size(1)) != nblk:
            raise RuntimeError(f"{who}: q_gmap_gr_meta shape mismatch")
        words_stride = int(q_gmap_gr_words.size(1))
    if has_output_scale:
        _check_cuda("output_scale", output_scale, torch.float16, 2, device)
        if tuple(output_scale.shape) != (num_experts, outfeatures):
            raise RuntimeError(f"{who}: output_scale mismatch")
    if has_bias:
        _check_cuda("bias", bias, torch.float16, 2, device)
        if tuple(bias.shape) != (num_experts, outfeatures):
            raise RuntimeError(f"{who}: bias mismatch")
    s = TrisPayload()
    s.num_experts = num_experts
    s.rank = rank
    s.outfeatures = outfeatures
    s.num_groups = num_groups
    s.qweight2_sparse_rows = int(qweight2_sparse.size(1))
    s.gr_words_stride = words_stride
    s.qweight1 = qweight1.data_ptr()
    s.qweight2_sparse = qweight2_sparse.data_ptr() if qweight2_sparse.numel() else None
    s.qweight2_sparse_prefix = qweight2_sparse_prefix.data_ptr()
    if need_gr:
        s.q_gmap_gr_words = q_gmap_gr_words.data_ptr() if q_gmap_gr_words.numel() else None
        s.q_gmap_gr_offsets = q_gmap_gr_offsets.data_ptr()
        s.q_gmap_gr_meta = q_gmap_gr_meta.data_ptr() if q_gmap_gr_meta.numel() else None
    s.c_map = c_map.data_ptr()
    s.g_idx = g_idx.data_ptr()
    s.col_pack3 = col_pack3.data_ptr()
    s.row_pack3 = row_pack3.data_ptr() if row_pack3.numel() else None
    s.output_scale = output_scale.data_ptr() if has_output_scale else None
    s.bias = bias.data_ptr() if has_bias else None
    s.has_output_scale = int(bool(has_output_scale))
    s.has_bias = int(bool(has_bias))
    s.use_uniform_k64_groups = int(bool(use_uniform_k64_groups))
    return s


def _check_route(hidden, expert_ids, segment_offsets, problem_offsets):
    _check_cuda("hidden", hidden, torch.float16, 2)
    dev = hidden.device
    _check_cuda("expert_ids", expert_ids, torch.int32, 1, dev)
    _check_cuda("segment_offsets", segment_offsets, torch.int32, 1, dev)
    _check_cuda("problem_offsets", problem_offsets, torch.int32, 1, dev)
    if segment_offsets.size(0) != expert_ids.size(0) + 1:
        raise RuntimeError("segment_offsets must be 1D [segments + 1]")
    if problem_offsets.size(0) != expert_ids.size(0) + 1:
        raise RuntimeError("problem_offsets must be 1D [segments + 1]")


# ------------------------------------------------------------------ route
def build_grouped_route(selected_experts: torch.Tensor, num_experts: int, m_tile: int):
    """TriSMoE_cuda.cpp:741-793: returns [perm, grouped_token_indices, grouped_slots, expert_ids,
    segment_offsets, problem_offsets, total_problem_tiles(CPU int64 [1])].

    The kernels build everything on the device; as in the reference, one
    device->host copy fetches the active-expert and tile counts to size the
    returned tensors.  ``build_grouped_route_device`` skips that copy."""
    out = build_grouped_route_device(selected_experts, num_experts, m_tile)
    counts = out["counts"].to("cpu")
    num_active, total = int(counts[0]), int(counts[1])
    if num_active < 0:
        raise RuntimeError("selected_experts contains an expert id outside [0, num_experts)")
    return [
        out["perm"],
        out["grouped_token_indices"],
        out["grouped_slots"],
        out["expert_ids"][:num_active].contiguous(),
        out["segment_offsets"][: num_active + 1].contiguous(),
        out["problem_offsets"][: num_active + 1].contiguous(),
        torch.tensor([total], dtype=torch.int64),
    ]


def build_grouped_route_device(selected_experts: torch.Tensor, num_experts: int, m_tile: int = 4) -> dict:
    """Route metadata padded to num_experts segments, with no host synchronisation."""
    if not isinstance(selected_experts, torch.Tensor) or selected_experts.device.type != "cuda":
        raise RuntimeError("selected_experts must be a CUDA tensor")
    if selected_experts.dim() != 2:
        raise RuntimeError("selected_experts must be 2D [tokens, top_k]")
    if num_experts < 0:
        raise RuntimeError("num_experts must be non-negative")
    if m_tile <= 0:
        raise RuntimeError("m_tile must be positive")
    sel = selected_experts.contiguous().to(torch.int64)
    dev = sel.device
    t, k = int(sel.size(0)), int(sel.size(1))
    r = t * k
    long_opts = dict(device=dev, dtype=torch.int64)
    int_opts = dict(device=dev, dtype=torch.int32)
    perm = torch.empty(r, **long_opts)
    gti = torch.empty(r, **long_opts)
    gsl = torch.empty(r, **long_opts)
    gexp = torch.empty(r, **int_opts)
    expert_ids = torch.empty(max(num_experts, 0), **int_opts)
    seg = torch.empty(num_experts + 1, **int_opts)
    prob = torch.empty(num_experts + 1, **int_opts)
    counts = torch.empty(2, **int_opts)
    inv = torch.empty(r, **int_opts)
    lib = _lib.load()
    _lib.check(lib.tris_build_grouped_route(_ptr(sel), t, k, num_experts, m_tile, _ptr(perm), _ptr(gti), _ptr(gsl),
                                            _ptr(gexp), _ptr(expert_ids), _ptr(seg), _ptr(prob), _ptr(counts),
                                            _ptr(inv), _stream(sel)), "build_grouped_route")
    return {"perm": perm, "grouped_token_indices": gti, "grouped_slots": gsl, "grouped_expert_ids": gexp,
            "expert_ids": expert_ids, "segment_offsets": seg, "problem_offsets": prob, "counts": counts,
            "inverse_perm": inv}


ROUTE_TOPK_MAX_ROWS = 2048     # tokens * top_k for tris_route_topk_grouped
ROUTE_TOPK_MAX_EXPERTS = 1024
ROUTE_TOPK_MAX_K = 16


def _route_topk_outputs(router_logits: torch.Tensor, top_k: int, who: str):
    """Validated logits and the fused router's output tensors: (logits, dict of outputs)."""
    _check_cuda("router_logits", router_logits, torch.float32, 2)
    logits = router_logits.contiguous()
    t, e = int(logits.size(0)), int(logits.size(1))
    k = int(top_k)
    if t * k > ROUTE_TOPK_MAX_ROWS or e > ROUTE_TOPK_MAX_EXPERTS or k > ROUTE_TOPK_MAX_K or k > e or k <= 0:
        raise RuntimeError(f"{who}: batch outside the one-workgroup limits")
    dev = logits.device
    r = t * k
    long_opts = dict(device=dev, dtype=torch.int64)
    int_opts = dict(device=dev, dtype=torch.int32)
    w16 = torch.empty((t, k), device=dev, dtype=torch.float16)
    w32 = torch.empty((t, k), device=dev, dtype=torch.float32)
    sel = torch.empty((t, k), **long_opts)
    perm = torch.empty(r, **long_opts)
    gti = torch.empty(r, **long_opts)
    gsl = torch.empty(r, **long_opts)
    gexp = torch.empty(r, **int_opts)
    expert_ids = torch.empty(e, **int_opts)
    seg = torch.empty(e + 1, **int_opts)
    prob = torch.empty(e + 1, **int_opts)
    counts = torch.empty(2, **int_opts)
    inv = torch.empty(r, **int_opts)
    return logits, {"perm": perm, "grouped_token_indices": gti, "grouped_slots": gsl, "grouped_expert_ids": gexp,
                    "expert_ids": expert_ids, "segment_offsets": seg, "problem_offsets": prob, "counts": counts,
                    "inverse_perm": inv, "routing_weights_f16": w16, "routing_weights": w32,
                    "selected_experts": sel}


def _route_topk_args(logits, out, top_k, renormalize, m_tile):
    t, e = int(logits.size(0)), int(logits.size(1))
    return (_ptr(logits), t, e, int(top_k), int(bool(renormalize)), int(m_tile), _ptr(out["routing_weights_f16"]),
            _ptr(out["routing_weights"]), _ptr(out["selected_experts"]), _ptr(out["perm"]),
            _ptr(out["grouped_token_indices"]), _ptr(out["grouped_slots"]), _ptr(out["grouped_expert_ids"]),
            _ptr(out["expert_ids"]), _ptr(out["segment_offsets"]), _ptr(out["problem_offsets"]),
            _ptr(out["counts"]), _ptr(out["inverse_perm"]))


def route_topk_ok(router_logits: torch.Tensor, top_k: int) -> bool:
    """tris_route_topk takes these logits: fp32 [T, E] on the GPU, E <= ROUTE_TOPK_MAX_EXPERTS, 0 < top_k <=
    min(E, ROUTE_TOPK_MAX_K)."""
    if not isinstance(router_logits, torch.Tensor) or router_logits.device.type != "cuda":
        return False
    if router_logits.dtype != torch.float32 or router_logits.dim() != 2:
        return False
    e = int(router_logits.size(1))
    return 0 < top_k <= min(e, ROUTE_TOPK_MAX_K) and e <= ROUTE_TOPK_MAX_EXPERTS


def route_topk(router_logits: torch.Tensor, top_k: int, renormalize: bool):
    """Router softmax / top-k / renormalisation and the fp16 cast (modeling_mixtral.py:548-555) in one launch
    for any batch (tris_route_topk).  Returns (routing_weights fp32 [T, k], selected_experts int64 [T, k],
    routing_weights fp16 [T, k])."""
    if not route_topk_ok(router_logits, top_k):
        raise RuntimeError("route_topk: fp32 [tokens, experts] logits on the GPU, experts <= "
                           f"{ROUTE_TOPK_MAX_EXPERTS}, 0 < top_k <= min(experts, {ROUTE_TOPK_MAX_K})")
    logits = router_logits.contiguous()
    t, e = int(logits.size(0)), int(logits.size(1))
    w32 = torch.empty((t, top_k), dtype=torch.float32, device=logits.device)
    w16 = torch.empty((t, top_k), dtype=torch.float16, device=logits.device)
    sel = torch.empty((t, top_k), dtype=torch.int64, device=logits.device)
    _lib.check(_lib.load().tris_route_topk(_ptr(logits), t, e, top_k, int(bool(renormalize)), _ptr(w16), _ptr(w32),
                                           _ptr(sel), _stream(logits)), "route_topk")
    return w32, sel, w16


def route_topk_grouped(router_logits: torch.Tensor, top_k: int, renormalize: bool, m_tile: int = 4) -> dict:
    """Router softmax / top-k / renormalisation (modeling_mixtral.py:548-555) and the padded grouped
    route in one launch, for decode-sized batches (an extension; see build_grouped_route_device).
    Returns the route dict plus routing_weights_f16 [T, k], routing_weights [T, k] fp32 and
    selected_experts [T, k] int64."""
    logits, out = _route_topk_outputs(router_logits, top_k, "route_topk_grouped")
    _lib.check(_lib.load().tris_route_topk_grouped(*_route_topk_args(logits, out, top_k, renormalize, m_tile),
                                                   _stream(logits)), "route_topk_grouped")
    return out


ROUTE_BACKBONE_MAX_TOKENS = 64  # tokens of tris_route_topk_backbone


class BackbonePending:
    """Gate/up backbone outputs launched beside the router (route_topk_backbone_pair) whose split-K slice
    reduction may still be outstanding: pass it as ``backbone`` to grouped_block_gr_predecode_multi (or to
    finish_backbone) on the same stream before out_a / out_b are read."""

    __slots__ = ("job", "out_a", "out_b", "keep")

    def __init__(self, job, out_a, out_b, keep):
        self.job, self.out_a, self.out_b, self.keep = job, out_a, out_b, keep


def route_topk_backbone_ok(x: torch.Tensor, sv_a, sv_b, in_scale_a=None, in_scale_b=None) -> bool:
    """True when route_topk_backbone_pair can run this backbone pair: fp16 SV matrices of one shape over x's
    columns, 16-byte aligned, at most ROUTE_BACKBONE_MAX_TOKENS tokens."""
    if not (isinstance(sv_a, torch.Tensor) and isinstance(sv_b, torch.Tensor)):
        return False
    if x.dtype != torch.float16 or x.dim() != 2 or not x.is_contiguous() or x.data_ptr() % 16:
        return False
    if int(x.size(0)) > ROUTE_BACKBONE_MAX_TOKENS or int(x.size(0)) == 0:
        return False
    for sv in (sv_a, sv_b):
        if (sv.dtype != torch.float16 or sv.dim() != 2 or not sv.is_contiguous() or sv.data_ptr() % 16
                or sv.device != x.device):
            return False
    if sv_a.shape != sv_b.shape or int(sv_a.size(1)) != int(x.size(1)) or int(x.size(1)) == 0:
        return False
    for sc in (in_scale_a, in_scale_b):
        if sc is not None and (sc.dtype != torch.float16 or sc.numel() != x.size(1) or not sc.is_contiguous()
                               or sc.data_ptr() % 16):
            return False
    return True


def route_topk_backbone_pair(router_logits: torch.Tensor, top_k: int, renormalize: bool, m_tile: int,
                             x: torch.Tensor, sv_a: torch.Tensor, sv_b: torch.Tensor,
                             in_scale_a: torch.Tensor | None = None, in_scale_b: torch.Tensor | None = None,
                             split: int = 0, out_a_hi: torch.Tensor | None = None,
                             out_b_hi: torch.Tensor | None = None):
    """route_topk_grouped and the gate/up backbones of the same tokens (backbone_linear_pair without a row
    index) in one launch (tris_route_topk_backbone, an extension).  Returns (route dict, BackbonePending): the
    backbone's split-K reduction is left for the predecode launch.  split > 0: sv_a / sv_b are two stacked
    projections each; the pending outputs hold columns [0, split) and out_a_hi / out_b_hi (fp16
    [tokens, rank - split], given) receive columns [split, rank)."""
    if not route_topk_backbone_ok(x, sv_a, sv_b, in_scale_a, in_scale_b):
        raise RuntimeError("route_topk_backbone_pair: backbone pair outside the merged launch's conditions")
    logits, out = _route_topk_outputs(router_logits, top_k, "route_topk_backbone_pair")
    if int(x.size(0)) != int(logits.size(0)):
        raise RuntimeError("route_topk_backbone_pair: x and router_logits differ in tokens")
    tokens, in_f, rank = int(x.size(0)), int(x.size(1)), int(sv_a.size(0))
    lo = split if split > 0 else rank
    if split > 0:
        if not 0 < split < rank:
            raise RuntimeError("route_topk_backbone_pair: split outside (0, rank)")
        for name, t in (("out_a_hi", out_a_hi), ("out_b_hi", out_b_hi)):
            _check_cuda(name, t, torch.float16, 2, x.device)
            if tuple(t.shape) != (tokens, rank - split) or not t.is_contiguous():
                raise RuntimeError(f"route_topk_backbone_pair: {name} must be a contiguous [{tokens}, {rank - split}]")
    out_a = torch.empty((tokens, lo), dtype=torch.float16, device=x.device)
    out_b = torch.empty((tokens, lo), dtype=torch.float16, device=x.device)
    lib = _lib.load()
    nbytes = int(lib.tris_backbone_pair_workspace_bytes(tokens, in_f, rank))
    # a buffer of this call's own, held by the BackbonePending until the launch that reduces the partial sums
    # has been enqueued (on this stream, so the allocator reuses it only after that launch): pending calls on
    # other streams, or a second call before the first is reduced, each keep their own partial sums
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=x.device)
    job = _lib.TrisBackbonePairJob(_ptr(x), tokens, in_f, _ptr(sv_a), _ptr(sv_b), rank, _ptr(in_scale_a),
                                   _ptr(in_scale_b), _ptr(out_a), _ptr(out_b), _ptr(ws), int(ws.numel()),
                                   _ptr(out_a_hi) if split > 0 else None, _ptr(out_b_hi) if split > 0 else None,
                                   int(split))
    _lib.check(lib.tris_route_topk_backbone(*_route_topk_args(logits, out, top_k, renormalize, m_tile),
                                            ctypes.byref(job), 1, _stream(logits)), "route_topk_backbone_pair")
    return out, BackbonePending(job, out_a, out_b, (x, sv_a, sv_b, in_scale_a, in_scale_b, ws, out_a_hi, out_b_hi))


ROUTE_WAVE_MAX_ROWS = 64     # tokens * top_k of the one-wavefront route (tris_route_predecode_multi_reduce)
ROUTE_WAVE_MAX_EXPERTS = 8
ROUTER_BACKBONE_MAX_HIDDEN = 8192  # hidden of tris_router_backbone


def router_backbone_ok(x: torch.Tensor, weight: torch.Tensor, sv_a, sv_b, in_scale_a=None, in_scale_b=None) -> bool:
    """True when router_backbone_pair can run: bf16 activations and router weight (router_linear_ok), at most
    ROUTE_BACKBONE_MAX_TOKENS tokens and ROUTER_BACKBONE_MAX_HIDDEN columns, and fp16 backbones of one shape over
    x's columns (16-byte aligned, optional fp16 input scales)."""
    if not router_linear_ok(x, weight) or x.dtype != torch.bfloat16:
        return False
    if int(x.size(0)) > ROUTE_BACKBONE_MAX_TOKENS or int(x.size(1)) > ROUTER_BACKBONE_MAX_HIDDEN:
        return False
    return route_topk_backbone_ok(x.view(torch.float16), sv_a, sv_b, in_scale_a, in_scale_b)


def router_backbone_pair(x: torch.Tensor, weight: torch.Tensor, sv_a: torch.Tensor, sv_b: torch.Tensor,
                         in_scale_a: torch.Tensor | None = None, in_scale_b: torch.Tensor | None = None):
    """router_linear and the gate/up backbones of the same tokens in one launch (tris_router_backbone, an
    extension): returns (router_logits bf16 [T, E], the logits as fp32, x16, BackbonePending).  The backbones
    read x's bf16 values as fp16 (x16's bits); their split-K reduction is left for route_predecode_multi or
    grouped_block_gr_predecode_multi (backbone=)."""
    if not router_backbone_ok(x, weight, sv_a, sv_b, in_scale_a, in_scale_b):
        raise RuntimeError("router_backbone_pair: inputs outside the merged launch's conditions")
    tokens, hidden, experts, rank = int(x.size(0)), int(x.size(1)), int(weight.size(0)), int(sv_a.size(0))
    dev = x.device
    logits = torch.empty((tokens, experts), dtype=torch.bfloat16, device=dev)
    logits32 = torch.empty((tokens, experts), dtype=torch.float32, device=dev)
    x16 = torch.empty((tokens, hidden), dtype=torch.float16, device=dev)
    out_a = torch.empty((tokens, rank), dtype=torch.float16, device=dev)
    out_b = torch.empty((tokens, rank), dtype=torch.float16, device=dev)
    lib = _lib.load()
    nbytes = int(lib.tris_backbone_pair_workspace_bytes(tokens, hidden, rank))
    # this call's own partial sums, held by the BackbonePending until the reducing launch is enqueued
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=dev)
    job = _lib.TrisBackbonePairJob(_ptr(x), tokens, hidden, _ptr(sv_a), _ptr(sv_b), rank, _ptr(in_scale_a),
                                   _ptr(in_scale_b), _ptr(out_a), _ptr(out_b), _ptr(ws), int(ws.numel()))
    _lib.check(lib.tris_router_backbone(_ptr(x), _ptr(weight), tokens, hidden, experts, _ptr(logits), _ptr(logits32),
                                        _ptr(x16), ctypes.byref(job), _stream(x)), "router_backbone_pair")
    return logits, logits32, x16, BackbonePending(job, out_a, out_b, (x, weight, sv_a, sv_b, in_scale_a, in_scale_b,
                                                                      ws, x16))


def route_predecode_ok(router_logits: torch.Tensor, top_k: int) -> bool:
    """The one-wavefront route of route_predecode_multi takes these fp32 [T, E] logits: T * top_k <= 64,
    E <= 8."""
    if not isinstance(router_logits, torch.Tensor) or router_logits.dim() != 2:
        return False
    t, e = int(router_logits.size(0)), int(router_logits.size(1))
    return (router_logits.dtype == torch.float32 and 0 < t and 0 < top_k <= e and t * top_k <= ROUTE_WAVE_MAX_ROWS
            and e <= ROUTE_WAVE_MAX_EXPERTS)


def route_predecode_multi(router_logits: torch.Tensor, top_k: int, renormalize: bool, m_tile: int, jobs,
                          backbone: BackbonePending | None = None, decode_all: bool = False) -> dict:
    """route_topk_grouped and grouped_block_gr_predecode_multi of the same route in one launch
    (tris_route_predecode_multi_reduce, an extension): jobs as grouped_block_gr_predecode_multi takes them, each
    buffer [min(E, T * top_k), blocks, 128], or none (the route and the backbone's reduction alone, for the
    GEMMs that decode the bitmaps themselves); ``backbone``: a BackbonePending reduced in the same launch.
    decode_all: decode every expert into slot e for expert e (tris_route_predecode_all_reduce; buffers
    [E, blocks, 128], read by the ``decoded_by_expert`` GEMMs).  Returns the route dict of route_topk_grouped."""
    if not route_predecode_ok(router_logits, top_k):
        raise RuntimeError("route_predecode_multi: logits outside the one-wavefront route (T * top_k <= "
                           f"{ROUTE_WAVE_MAX_ROWS}, E <= {ROUTE_WAVE_MAX_EXPERTS})")
    if not 0 <= len(jobs) <= _lib.MAX_PREDECODE_JOBS:
        raise RuntimeError(f"route_predecode_multi: 0 to {_lib.MAX_PREDECODE_JOBS} predecode jobs")
    logits, out = _route_topk_outputs(router_logits, top_k, "route_predecode_multi")
    t, e = int(logits.size(0)), int(logits.size(1))
    slots = e if decode_all else min(e, t * int(top_k))
    dev = logits.device
    arr = (_lib.TrisPredecodeJob * len(jobs))()
    keep = []
    for q, (buf, words, offsets, meta, packed_rows, outfeatures) in enumerate(jobs):
        _check_cuda("decoded_q_gmap_words", buf, torch.int32, None, dev)
        _check_cuda("q_gmap_gr_words", words, torch.int32, 2, dev)
        _check_cuda("q_gmap_gr_offsets", offsets, torch.int32, 2, dev)
        _check_cuda("q_gmap_gr_meta", meta, torch.int32, 2, dev)
        nblk = _num_gr_blocks(int(packed_rows), int(outfeatures))
        if buf.numel() != slots * nblk * BLOCK_GR_WORDS_PER_BLOCK:
            raise RuntimeError("decoded_q_gmap_words must hold [E, blocks, 128] words" if decode_all else
                               "decoded_q_gmap_words must hold [min(E, T * top_k), blocks, 128] words")
        if int(offsets.size(1)) != nblk + 1 or int(meta.size(1)) != nblk:
            raise RuntimeError("q_gmap_gr_offsets/meta shape mismatch")
        if words.numel() == 0:
            words = torch.zeros((max(int(offsets.size(0)), 1), 1), dtype=torch.int32, device=dev)
        keep.append(words)
        arr[q] = _lib.TrisPredecodeJob(_ptr(buf), _ptr(words), _ptr(offsets), _ptr(meta), int(offsets.size(0)),
                                       int(words.size(1)), int(packed_rows), int(outfeatures))
    bb = ctypes.byref(backbone.job) if backbone is not None else None
    lib = _lib.load()
    if decode_all:
        _lib.check(lib.tris_route_predecode_all_reduce(
            *_route_topk_args(logits, out, top_k, renormalize, m_tile), arr if jobs else None, len(jobs), bb,
            _stream(logits)), "route_predecode_multi")
    else:
        _lib.check(lib.tris_route_predecode_multi_reduce(
            *_route_topk_args(logits, out, top_k, renormalize, m_tile), arr if jobs else None, len(jobs), slots, bb,
            _stream(logits)), "route_predecode_multi")
    return out


def finish_backbone(pending: BackbonePending):
    """Run a BackbonePending's outstanding reduction alone (when no predecode launch follows); returns
    (out_a, out_b)."""
    _lib.check(_lib.load().tris_grouped_block_gr_predecode_multi_reduce(
        None, 0, None, 0, ctypes.byref(pending.job), _stream(pending.out_a)), "finish_backbone")
    return pending.out_a, pending.out_b


# ----------------------------------------------------------- grouped GEMMs
def compact3_tris_precomputed_grouped_forward_block_gr(hidden, expert_ids, segment_offsets, problem_offsets,
                                                       total_problem_tiles, qweight1, qweight2_sparse,
                                                       qweight2_sparse_prefix, q_gmap_gr_words, q_gmap_gr_offsets,
                                                       q_gmap_gr_meta, c_map, g_idx, col_pack3, row_pack3,
                                                       output_scale, has_output_scale, bias, has_bias,
                                                       use_uniform_k64_groups=False):
    """TriSMoE_cuda.cpp:1018-1063 -> tris_grouped_forward_block_gr."""
    _check_route(hidden, expert_ids, segment_offsets, problem_offsets)
    total = _host_tiles(total_problem_tiles)
    rank = int(hidden.size(1))
    pay = make_payload_struct(rank, qweight1, qweight2_sparse, qweight2_sparse_prefix, q_gmap_gr_words,
                              q_gmap_gr_offsets, q_gmap_gr_meta, c_map, g_idx, col_pack3, row_pack3, output_scale,
                              has_output_scale, bias, has_bias, use_uniform_k64_groups, hidden.device)
    out = torch.zeros((hidden.size(0), pay.outfeatures), dtype=torch.float16, device=hidden.device)
    _lib.check(_lib.load().tris_grouped_forward_block_gr(
        _ptr(hidden), int(hidden.size(0)), _ptr(expert_ids), _ptr(segment_offsets), _ptr(problem_offsets),
        int(expert_ids.size(0)), total, ctypes.byref(pay), _ptr(out), _stream(hidden)),
        "compact3_tris_precomputed_grouped_forward_block_gr")
    return out


def compact3_tris_precomputed_grouped_forward(hidden, expert_ids, segment_offsets, problem_offsets,
                                              total_problem_tiles, qweight1, qweight2_sparse, qweight2_sparse_prefix,
                                              q_gmap_sparse, q_gmap_sparse_prefix, c_map, g_idx, col_pack3,
                                              row_pack3, output_scale, bias, has_bias):
    """TriSMoE_cuda.cpp:795-832 (sparse split bitmaps) -> tris_grouped_forward_sparse.  output_scale fp16 [E, N]
    is always applied, as the reference's sparse kernels do (kernel.cu:4051-4064)."""
    _check_route(hidden, expert_ids, segment_offsets, problem_offsets)
    total = _host_tiles(total_problem_tiles)
    rank = int(hidden.size(1))
    _check_cuda("q_gmap_sparse", q_gmap_sparse, torch.int32, 3, hidden.device)
    _check_cuda("q_gmap_sparse_prefix", q_gmap_sparse_prefix, torch.int32, 2, hidden.device)
    pay = make_payload_struct(rank, qweight1, qweight2_sparse, qweight2_sparse_prefix, None, None, None, c_map, g_idx,
                              col_pack3, row_pack3, output_scale, True, bias, has_bias, False, hidden.device,
                              need_gr=False)
    packed_rows = (rank + 31) // 32
    if int(q_gmap_sparse.size(0)) != pay.num_experts or int(q_gmap_sparse.size(2)) != pay.outfeatures:
        raise RuntimeError("compact3 grouped q_gmap_sparse shape mismatch")
    if tuple(q_gmap_sparse_prefix.shape) != (pay.num_experts, packed_rows + 1):
        raise RuntimeError("compact3 grouped q_gmap prefix mismatch")
    out = torch.zeros((hidden.size(0), pay.outfeatures), dtype=torch.float16, device=hidden.device)
    _lib.check(_lib.load().tris_grouped_forward_sparse(
        _ptr(hidden), int(hidden.size(0)), _ptr(expert_ids), _ptr(segment_offsets), _ptr(problem_offsets),
        int(expert_ids.size(0)), total, ctypes.byref(pay), _ptr(q_gmap_sparse), _ptr(q_gmap_sparse_prefix),
        int(q_gmap_sparse.size(1)), _ptr(out), _stream(hidden)), "compact3_tris_precomputed_grouped_forward")
    return out


def compact3_tris_precomputed_grouped_dual_forward_block_gr(
        hidden_a, hidden_b, expert_ids, segment_offsets, problem_offsets, total_problem_tiles,
        qweight1_a, qweight2_sparse_a, qweight2_sparse_prefix_a, q_gmap_gr_words_a, q_gmap_gr_offsets_a,
        q_gmap_gr_meta_a, c_map_a, g_idx_a, col_pack3_a, row_pack3_a, output_scale_a, has_output_scale_a, bias_a,
        qweight1_b, qweight2_sparse_b, qweight2_sparse_prefix_b, q_gmap_gr_words_b, q_gmap_gr_offsets_b,
        q_gmap_gr_meta_b, c_map_b, g_idx_b, col_pack3_b, row_pack3_b, output_scale_b, has_output_scale_b, bias_b,
        use_uniform_k64_groups=False):
    """TriSMoE_cuda.cpp:1065-1136 -> tris_grouped_dual_forward_block_gr.  has_bias = bias.numel() > 0
    (kernel.cu:10330-10331)."""
    _check_route(hidden_a, expert_ids, segment_offsets, problem_offsets)
    _check_cuda("hidden_b", hidden_b, torch.float16, 2, hidden_a.device)
    if hidden_b.size(0) != hidden_a.size(0):
        raise RuntimeError("hidden_a/hidden_b batch mismatch")
    total = _host_tiles(total_problem_tiles)
    has_bias_a = isinstance(bias_a, torch.Tensor) and bias_a.numel() > 0
    has_bias_b = isinstance(bias_b, torch.Tensor) and bias_b.numel() > 0
    pa = make_payload_struct(int(hidden_a.size(1)), qweight1_a, qweight2_sparse_a, qweight2_sparse_prefix_a,
                             q_gmap_gr_words_a, q_gmap_gr_offsets_a, q_gmap_gr_meta_a, c_map_a, g_idx_a, col_pack3_a,
                             row_pack3_a, output_scale_a, has_output_scale_a, bias_a, has_bias_a,
                             use_uniform_k64_groups, hidden_a.device, who="grouped payload a")
    pb = make_payload_struct(int(hidden_b.size(1)), qweight1_b, qweight2_sparse_b, qweight2_sparse_prefix_b,
                             q_gmap_gr_words_b, q_gmap_gr_offsets_b, q_gmap_gr_meta_b, c_map_b, g_idx_b, col_pack3_b,
                             row_pack3_b, output_scale_b, has_output_scale_b, bias_b, has_bias_b,
                             use_uniform_k64_groups, hidden_a.device, who="grouped payload b")
    out_a = torch.zeros((hidden_a.size(0), pa.outfeatures), dtype=torch.float16, device=hidden_a.device)
    out_b = torch.zeros((hidden_b.size(0), pb.outfeatures), dtype=torch.float16, device=hidden_a.device)
    _lib.check(_lib.load().tris_grouped_dual_forward_block_gr(
        _ptr(hidden_a), _ptr(hidden_b), int(hidden_a.size(0)), _ptr(expert_ids), _ptr(segment_offsets),
        _ptr(problem_offsets), int(expert_ids.size(0)), total, ctypes.byref(pa), ctypes.byref(pb), _ptr(out_a),
        _ptr(out_b), _stream(hidden_a)), "compact3_tris_precomputed_grouped_dual_forward_block_gr")
    return [out_a, out_b]


def compact3_tris_precomputed_grouped_block_gr_predecode(decoded_q_gmap_words, expert_ids, q_gmap_gr_words,
                                                         q_gmap_gr_offsets, q_gmap_gr_meta, packed_rows, outfeatures):
    """TriSMoE_cuda.cpp:836-853 (kernel.cu:8980-9029): decode into the caller's buffer and return it."""
    _check_cuda("decoded_q_gmap_words", decoded_q_gmap_words, torch.int32, None)
    dev = decoded_q_gmap_words.device
    _check_cuda("expert_ids", expert_ids, torch.int32, 1, dev)
    _check_cuda("q_gmap_gr_words", q_gmap_gr_words, torch.int32, 2, dev)
    _check_cuda("q_gmap_gr_offsets", q_gmap_gr_offsets, torch.int32, 2, dev)
    _check_cuda("q_gmap_gr_meta", q_gmap_gr_meta, torch.int32, 2, dev)
    nblk = _num_gr_blocks(int(packed_rows), int(outfeatures))
    num_active = int(expert_ids.size(0))
    if decoded_q_gmap_words.numel() != num_active * nblk * BLOCK_GR_WORDS_PER_BLOCK:
        raise RuntimeError("decoded_q_gmap_words must hold [active, blocks, 128] words")
    if int(q_gmap_gr_offsets.size(1)) != nblk + 1 or int(q_gmap_gr_meta.size(1)) != nblk:
        raise RuntimeError("q_gmap_gr_offsets/meta shape mismatch")
    words = q_gmap_gr_words
    if words.numel() == 0:
        words = torch.zeros((max(int(q_gmap_gr_offsets.size(0)), 1), 1), dtype=torch.int32, device=dev)
    _lib.check(_lib.load().tris_grouped_block_gr_predecode(
        _ptr(decoded_q_gmap_words), _ptr(expert_ids), num_active, _ptr(words), _ptr(q_gmap_gr_offsets),
        _ptr(q_gmap_gr_meta), int(q_gmap_gr_offsets.size(0)), int(words.size(1)), int(packed_rows),
        int(outfeatures), _stream(decoded_q_gmap_words)),
        "compact3_tris_precomputed_grouped_block_gr_predecode")
    return decoded_q_gmap_words


def grouped_block_gr_predecode_multi(jobs, expert_ids, backbone: BackbonePending | None = None):
    """Predecode several projections' GR streams for the same routed experts in one launch (an
    extension batching TriSMoE_cuda.cpp:836-853).  jobs: sequence of (decoded_buffer,
    q_gmap_gr_words, q_gmap_gr_offsets, q_gmap_gr_meta, packed_rows, outfeatures); each buffer is
    filled as compact3_tris_precomputed_grouped_block_gr_predecode would fill it and returned.
    ``backbone``: a BackbonePending whose slice reduction runs in the same launch
    (tris_grouped_block_gr_predecode_multi_reduce)."""
    if len(jobs) > _lib.MAX_PREDECODE_JOBS:
        raise RuntimeError(f"at most {_lib.MAX_PREDECODE_JOBS} predecode jobs per launch")
    _check_cuda("expert_ids", expert_ids, torch.int32, 1)
    dev = expert_ids.device
    num_active = int(expert_ids.size(0))
    arr = (_lib.TrisPredecodeJob * max(len(jobs), 1))()
    keep = []
    for q, (buf, words, offsets, meta, packed_rows, outfeatures) in enumerate(jobs):
        _check_cuda("decoded_q_gmap_words", buf, torch.int32, None, dev)
        _check_cuda("q_gmap_gr_words", words, torch.int32, 2, dev)
        _check_cuda("q_gmap_gr_offsets", offsets, torch.int32, 2, dev)
        _check_cuda("q_gmap_gr_meta", meta, torch.int32, 2, dev)
        nblk = _num_gr_blocks(int(packed_rows), int(outfeatures))
        if buf.numel() != num_active * nblk * BLOCK_GR_WORDS_PER_BLOCK:
            raise RuntimeError("decoded_q_gmap_words must hold [active, blocks, 128] words")
        if int(offsets.size(1)) != nblk + 1 or int(meta.size(1)) != nblk:
            raise RuntimeError("q_gmap_gr_offsets/meta shape mismatch")
        if words.numel() == 0:
            words = torch.zeros((max(int(offsets.size(0)), 1), 1), dtype=torch.int32, device=dev)
        keep.append(words)
        arr[q] = _lib.TrisPredecodeJob(_ptr(buf), _ptr(words), _ptr(offsets), _ptr(meta), int(offsets.size(0)),
                                       int(words.size(1)), int(packed_rows), int(outfeatures))
    if backbone is not None:
        _lib.check(_lib.load().tris_grouped_block_gr_predecode_multi_reduce(
            arr, len(jobs), _ptr(expert_ids), num_active, ctypes.byref(backbone.job), _stream(expert_ids)),
            "grouped_block_gr_predecode_multi")
        return [j[0] for j in jobs]
    _lib.check(_lib.load().tris_grouped_block_gr_predecode_multi(arr, len(jobs), _ptr(expert_ids), num_active,
                                                                 _stream(expert_ids)),
               "grouped_block_gr_predecode_multi")
    return [j[0] for j in jobs]


def compact3_tris_precomputed_grouped_forward_block_gr_predecoded(hidden, expert_ids, segment_offsets,
                                                                  problem_offsets, total_problem_tiles,
                                                                  decoded_q_gmap_words, qweight1, qweight2_sparse,
                                                                  qweight2_sparse_prefix, c_map, g_idx, col_pack3,
                                                                  row_pack3, use_uniform_k64_groups=False,
                                                                  out=None, decoded_by_expert=False):
    """TriSMoE_cuda.cpp:855-889 (no output scale / bias, as the reference's NoScaleNoBias kernel).
    ``out``: optional [rows, N] fp16 buffer; rows outside every segment are left as they are
    (the default buffer is zero-filled, as the reference's).  decoded_by_expert: the decoded bitmaps hold every
    expert, slot e for expert e (tris_grouped_forward_block_gr_predecoded_experts, an extension)."""
    _check_route(hidden, expert_ids, segment_offsets, problem_offsets)
    total = _host_tiles(total_problem_tiles)
    pay = make_payload_struct(int(hidden.size(1)), qweight1, qweight2_sparse, qweight2_sparse_prefix, None, None,
                              None, c_map, g_idx, col_pack3, row_pack3, None, False, None, False,
                              use_uniform_k64_groups, hidden.device, need_gr=False)
    _check_predecoded(decoded_q_gmap_words, expert_ids, pay, hidden.device, decoded_by_expert)
    out = _out_buffer(out, hidden.size(0), pay.outfeatures, hidden.device)
    if decoded_by_expert:
        _lib.check(_lib.load().tris_grouped_forward_block_gr_predecoded_experts(
            _ptr(hidden), None, None, 0, int(hidden.size(0)), _ptr(expert_ids), _ptr(segment_offsets),
            int(expert_ids.size(0)), total, _ptr(decoded_q_gmap_words), None, ctypes.byref(pay), None, _ptr(out), None,
            _stream(hidden)), "compact3_tris_precomputed_grouped_forward_block_gr_predecoded")
        return out
    _lib.check(_lib.load().tris_grouped_forward_block_gr_predecoded(
        _ptr(hidden), int(hidden.size(0)), _ptr(expert_ids), _ptr(segment_offsets), _ptr(problem_offsets),
        int(expert_ids.size(0)), total, _ptr(decoded_q_gmap_words), ctypes.byref(pay), _ptr(out), _stream(hidden)),
        "compact3_tris_precomputed_grouped_forward_block_gr_predecoded")
    return out


def _out_buffer(out, rows, cols, device):
    if out is None:
        return torch.zeros((rows, cols), dtype=torch.float16, device=device)
    _check_cuda("out", out, torch.float16, 2, device)
    if tuple(out.shape) != (int(rows), int(cols)):
        raise RuntimeError(f"out must be [{int(rows)}, {int(cols)}]")
    return out


def _gather_rows(row_index, hidden_a, hidden_b):
    """Grouped row count: hidden's rows, or row_index's length when the rows are gathered (then both
    hidden tensors must hold the same rows)."""
    if row_index is None:
        return int(hidden_a.size(0))
    _check_cuda("row_index", row_index, torch.int64, 1, hidden_a.device)
    if int(hidden_b.size(0)) != int(hidden_a.size(0)):
        raise RuntimeError("gathered hidden_a and hidden_b must have the same rows")
    return int(row_index.size(0))


def _check_predecoded(decoded, expert_ids, pay, device, by_expert=False):
    _check_cuda("decoded_q_gmap_words", decoded, torch.int32, None, device)
    nblk = _num_gr_blocks((pay.rank + 31) // 32, pay.outfeatures)
    if by_expert:
        if decoded.numel() < int(pay.num_experts) * nblk * BLOCK_GR_WORDS_PER_BLOCK:
            raise RuntimeError("decoded_q_gmap_words is smaller than [experts, blocks, 128]")
    elif decoded.numel() < int(expert_ids.size(0)) * nblk * BLOCK_GR_WORDS_PER_BLOCK:
        raise RuntimeError("decoded_q_gmap_words is smaller than [segments, blocks, 128]")


def compact3_tris_precomputed_grouped_dual_forward_block_gr_predecoded(
        hidden_a, hidden_b, expert_ids, segment_offsets, problem_offsets, total_problem_tiles,
        decoded_q_gmap_words_a, qweight1_a, qweight2_sparse_a, qweight2_sparse_prefix_a, c_map_a, g_idx_a,
        col_pack3_a, row_pack3_a, decoded_q_gmap_words_b, qweight1_b, qweight2_sparse_b, qweight2_sparse_prefix_b,
        c_map_b, g_idx_b, col_pack3_b, row_pack3_b, use_uniform_k64_groups=False, out_a=None, out_b=None,
        row_index=None, decoded_by_expert=False):
    """TriSMoE_cuda.cpp:922-974.  ``out_a`` / ``out_b`` as ``out`` of the single-projection call.
    ``row_index``: optional int64 [batch] (the route's grouped_token_indices): grouped row r reads row
    row_index[r] of per-token hidden_a / hidden_b (tris_grouped_dual_forward_block_gr_predecoded_rows, an
    extension; the MFMA kernel's payload conditions apply).  decoded_by_expert: as in the single-projection
    call."""
    _check_route(hidden_a, expert_ids, segment_offsets, problem_offsets)
    _check_cuda("hidden_b", hidden_b, torch.float16, 2, hidden_a.device)
    batch = _gather_rows(row_index, hidden_a, hidden_b)
    total = _host_tiles(total_problem_tiles)
    pa = make_payload_struct(int(hidden_a.size(1)), qweight1_a, qweight2_sparse_a, qweight2_sparse_prefix_a, None,
                             None, None, c_map_a, g_idx_a, col_pack3_a, row_pack3_a, None, False, None, False,
                             use_uniform_k64_groups, hidden_a.device, need_gr=False, who="grouped payload a")
    pb = make_payload_struct(int(hidden_b.size(1)), qweight1_b, qweight2_sparse_b, qweight2_sparse_prefix_b, None,
                             None, None, c_map_b, g_idx_b, col_pack3_b, row_pack3_b, None, False, None, False,
                             use_uniform_k64_groups, hidden_a.device, need_gr=False, who="grouped payload b")
    _check_predecoded(decoded_q_gmap_words_a, expert_ids, pa, hidden_a.device, decoded_by_expert)
    _check_predecoded(decoded_q_gmap_words_b, expert_ids, pb, hidden_a.device, decoded_by_expert)
    out_a = _out_buffer(out_a, batch, pa.outfeatures, hidden_a.device)
    out_b = _out_buffer(out_b, batch, pb.outfeatures, hidden_a.device)
    if decoded_by_expert:
        _lib.check(_lib.load().tris_grouped_forward_block_gr_predecoded_experts(
            _ptr(hidden_a), _ptr(hidden_b), _ptr(row_index), int(hidden_a.size(0)), batch, _ptr(expert_ids),
            _ptr(segment_offsets), int(expert_ids.size(0)), total, _ptr(decoded_q_gmap_words_a),
            _ptr(decoded_q_gmap_words_b), ctypes.byref(pa), ctypes.byref(pb), _ptr(out_a), _ptr(out_b),
            _stream(hidden_a)), "compact3_tris_precomputed_grouped_dual_forward_block_gr_predecoded")
        return [out_a, out_b]
    if row_index is not None:
        _lib.check(_lib.load().tris_grouped_dual_forward_block_gr_predecoded_rows(
            _ptr(hidden_a), _ptr(hidden_b), _ptr(row_index), int(hidden_a.size(0)), batch, _ptr(expert_ids),
            _ptr(segment_offsets), int(expert_ids.size(0)), total, _ptr(decoded_q_gmap_words_a),
            _ptr(decoded_q_gmap_words_b), ctypes.byref(pa), ctypes.byref(pb), _ptr(out_a), _ptr(out_b),
            _stream(hidden_a)), "compact3_tris_precomputed_grouped_dual_forward_block_gr_predecoded")
        return [out_a, out_b]
    _lib.check(_lib.load().tris_grouped_dual_forward_block_gr_predecoded(
        _ptr(hidden_a), _ptr(hidden_b), int(hidden_a.size(0)), _ptr(expert_ids), _ptr(segment_offsets),
        _ptr(problem_offsets), int(expert_ids.size(0)), total, _ptr(decoded_q_gmap_words_a),
        _ptr(decoded_q_gmap_words_b), ctypes.byref(pa), ctypes.byref(pb), _ptr(out_a), _ptr(out_b),
        _stream(hidden_a)), "compact3_tris_precomputed_grouped_dual_forward_block_gr_predecoded")
    return [out_a, out_b]


def compact3_tris_precomputed_grouped_swiglu_forward_block_gr_predecoded(
        hidden_gate, hidden_up, expert_ids, segment_offsets, problem_offsets, total_problem_tiles,
        decoded_q_gmap_words_gate, qweight1_gate, qweight2_sparse_gate, qweight2_sparse_prefix_gate, c_map_gate,
        g_idx_gate, col_pack3_gate, row_pack3_gate, decoded_q_gmap_words_up, qweight1_up, qweight2_sparse_up,
        qweight2_sparse_prefix_up, c_map_up, g_idx_up, col_pack3_up, row_pack3_up, out=None, row_index=None):
    """fp16(silu(gate) * up) of the dual predecoded GEMM (TriSMoE_cuda.cpp:922-974) fused with the
    SwiGLU product of modeling_mixtral.py:496 (an extension with no reference entry point; needs
    uniform 64-column groups).  ``row_index`` as in the dual call."""
    _check_route(hidden_gate, expert_ids, segment_offsets, problem_offsets)
    _check_cuda("hidden_up", hidden_up, torch.float16, 2, hidden_gate.device)
    batch = _gather_rows(row_index, hidden_gate, hidden_up)
    total = _host_tiles(total_problem_tiles)
    pg = make_payload_struct(int(hidden_gate.size(1)), qweight1_gate, qweight2_sparse_gate,
                             qweight2_sparse_prefix_gate, None, None, None, c_map_gate, g_idx_gate, col_pack3_gate,
                             row_pack3_gate, None, False, None, False, True, hidden_gate.device, need_gr=False,
                             who="gate payload")
    pu = make_payload_struct(int(hidden_up.size(1)), qweight1_up, qweight2_sparse_up, qweight2_sparse_prefix_up,
                             None, None, None, c_map_up, g_idx_up, col_pack3_up, row_pack3_up, None, False, None,
                             False, True, hidden_gate.device, need_gr=False, who="up payload")
    _check_predecoded(decoded_q_gmap_words_gate, expert_ids, pg, hidden_gate.device)
    _check_predecoded(decoded_q_gmap_words_up, expert_ids, pu, hidden_gate.device)
    out = _out_buffer(out, batch, pg.outfeatures, hidden_gate.device)
    if row_index is not None:
        _lib.check(_lib.load().tris_grouped_swiglu_forward_block_gr_predecoded_rows(
            _ptr(hidden_gate), _ptr(hidden_up), _ptr(row_index), int(hidden_gate.size(0)), batch, _ptr(expert_ids),
            _ptr(segment_offsets), int(expert_ids.size(0)), total, _ptr(decoded_q_gmap_words_gate),
            _ptr(decoded_q_gmap_words_up), ctypes.byref(pg), ctypes.byref(pu), _ptr(out), _stream(hidden_gate)),
            "compact3_tris_precomputed_grouped_swiglu_forward_block_gr_predecoded")
        return out
    _lib.check(_lib.load().tris_grouped_swiglu_forward_block_gr_predecoded(
        _ptr(hidden_gate), _ptr(hidden_up), int(hidden_gate.size(0)), _ptr(expert_ids), _ptr(segment_offsets),
        _ptr(problem_offsets), int(expert_ids.size(0)), total, _ptr(decoded_q_gmap_words_gate),
        _ptr(decoded_q_gmap_words_up), ctypes.byref(pg), ctypes.byref(pu), _ptr(out), _stream(hidden_gate)),
        "compact3_tris_precomputed_grouped_swiglu_forward_block_gr_predecoded")
    return out


def _segments_total(segment_offsets) -> int:
    return int(segment_offsets.numel()) - 1


def compact3_tris_precomputed_grouped_forward_block_gr_predecoded_hybrid(
        hidden, expert_ids, segment_offsets, full_problem_offsets, full_problem_tiles, tail_problem_offsets,
        tail_problem_tiles, decoded_q_gmap_words, qweight1, qweight2_sparse, qweight2_sparse_prefix, c_map, g_idx,
        col_pack3, row_pack3, use_uniform_k64_groups=False):
    """TriSMoE_cuda.cpp:891-920.  The reference splits full 16-row tiles (tensor cores) from tail
    tiles; here one kernel covers every row of every segment, so the split metadata only bounds
    the launch and the result is the predecoded GEMM."""
    total = _host_tiles(full_problem_tiles) + _host_tiles(tail_problem_tiles) + _segments_total(segment_offsets)
    return compact3_tris_precomputed_grouped_forward_block_gr_predecoded(
        hidden, expert_ids, segment_offsets, full_problem_offsets, total, decoded_q_gmap_words, qweight1,
        qweight2_sparse, qweight2_sparse_prefix, c_map, g_idx, col_pack3, row_pack3, use_uniform_k64_groups)


def compact3_tris_precomputed_grouped_dual_forward_block_gr_predecoded_hybrid(
        hidden_a, hidden_b, expert_ids, segment_offsets, full_problem_offsets, full_problem_tiles,
        tail_problem_offsets, tail_problem_tiles, decoded_q_gmap_words_a, qweight1_a, qweight2_sparse_a,
        qweight2_sparse_prefix_a, c_map_a, g_idx_a, col_pack3_a, row_pack3_a, decoded_q_gmap_words_b, qweight1_b,
        qweight2_sparse_b, qweight2_sparse_prefix_b, c_map_b, g_idx_b, col_pack3_b, row_pack3_b,
        use_uniform_k64_groups=False):
    """TriSMoE_cuda.cpp:976-1016 (see the single-projection hybrid)."""
    total = _host_tiles(full_problem_tiles) + _host_tiles(tail_problem_tiles) + _segments_total(segment_offsets)
    return compact3_tris_precomputed_grouped_dual_forward_block_gr_predecoded(
        hidden_a, hidden_b, expert_ids, segment_offsets, full_problem_offsets, total, decoded_q_gmap_words_a,
        qweight1_a, qweight2_sparse_a, qweight2_sparse_prefix_a, c_map_a, g_idx_a, col_pack3_a, row_pack3_a,
        decoded_q_gmap_words_b, qweight1_b, qweight2_sparse_b, qweight2_sparse_prefix_b, c_map_b, g_idx_b,
        col_pack3_b, row_pack3_b, use_uniform_k64_groups)


# ---------------------------------------------- verification / helper entry points
# ------------------------------------------------------------------ in-kernel-decode MFMA GEMMs (decode sizes)
def decode_payload_ok(p: dict) -> bool:
    """The payload suits the decode kernels: the GR stream, uniform 64-column groups, no sparse-only form, and
    rank a multiple of 256 up to 512."""
    rank = int(p["g_idx"].size(1))
    return bool(p.get("_compact3_k64_groups_uniform", False)) and rank % 256 == 0 and 0 < rank <= 512 and \
        p.get("q_gmap_gr_words") is not None


MFMA_MAX_GROUPS = 8  # row-scale groups the MFMA kernel stages whole per output tile


def mfma_payload_ok(p: dict) -> bool:
    """The payload suits the predecoded MFMA kernel (the one that can gather its rows through a row index):
    uniform 64-column groups, rank a multiple of 64, at most MFMA_MAX_GROUPS groups and 32-bit buffer offsets
    per expert."""
    rank = int(p["g_idx"].size(1))
    n = int(p["qweight1"].size(2))
    groups = int(p["row_pack3"].size(2))
    packed_rows = (rank + 31) // 32
    limit = 1 << 31
    return (bool(p.get("_compact3_k64_groups_uniform", False)) and rank > 0 and rank % 64 == 0
            and 1 <= groups <= MFMA_MAX_GROUPS and packed_rows * n * 4 < limit
            and int(p["qweight2_sparse"].size(1)) * n * 4 < limit and n * groups * 8 < limit
            and ((packed_rows + 1) // 2) * ((n + 63) // 64) * 128 * 4 < limit)


def _decode_struct(p: dict, device):
    rank = int(p["g_idx"].size(1))
    bias = p["bias"] if p.get("has_bias") else None
    return make_payload_struct(rank, p["qweight1"], p["qweight2_sparse"], p["qweight2_sparse_prefix"],
                               p["q_gmap_gr_words"], p["q_gmap_gr_offsets"], p["q_gmap_gr_meta"], p["c_map"],
                               p["g_idx"], p["col_pack3"], p["row_pack3"], p["output_scale"],
                               bool(p.get("has_output_scale", False)), bias, bool(p.get("has_bias", False)),
                               bool(p.get("_compact3_k64_groups_uniform", False)), device, who="decode payload")


def _decode_route_args(hidden, expert_ids, segment_offsets, row_index, batch):
    dev = hidden.device
    _check_cuda("hidden", hidden, torch.float16, 2, dev)
    _check_cuda("expert_ids", expert_ids, torch.int32, 1, dev)
    _check_cuda("segment_offsets", segment_offsets, torch.int32, 1, dev)
    if segment_offsets.numel() != expert_ids.numel() + 1:
        raise RuntimeError("segment_offsets must hold segments + 1 entries")
    if row_index is not None:
        _check_cuda("row_index", row_index, torch.int64, 1, dev)
        if row_index.numel() != batch:
            raise RuntimeError("row_index must hold one entry per grouped row")
    elif int(hidden.size(0)) != batch:
        raise RuntimeError("without row_index hidden must hold one row per grouped row")


def grouped_decode_forward(hidden: torch.Tensor, payload: dict, expert_ids: torch.Tensor,
                           segment_offsets: torch.Tensor, batch: int, row_index: torch.Tensor | None = None,
                           out: torch.Tensor | None = None) -> torch.Tensor:
    """tris_grouped_decode_forward_block_gr: fp16 [batch, N] of the grouped rows (rows outside every segment
    left as they are in ``out``)."""
    _decode_route_args(hidden, expert_ids, segment_offsets, row_index, batch)
    st = _decode_struct(payload, hidden.device)
    out = _out_buffer(out, batch, st.outfeatures, hidden.device)
    _lib.check(_lib.load().tris_grouped_decode_forward_block_gr(
        _ptr(hidden), _ptr(row_index), int(hidden.size(0)), batch, _ptr(expert_ids), _ptr(segment_offsets),
        int(expert_ids.numel()), ctypes.byref(st), _ptr(out), _stream(hidden)), "tris_grouped_decode_forward_block_gr")
    return out


def grouped_decode_pair_forward(hidden_a: torch.Tensor, hidden_b: torch.Tensor, payload_a: dict, payload_b: dict,
                                expert_ids: torch.Tensor, segment_offsets: torch.Tensor, batch: int,
                                row_index: torch.Tensor | None = None, swiglu: bool = False, out_a=None, out_b=None):
    """tris_grouped_decode_pair_forward_block_gr: (out_a, out_b) fp16 [batch, N], or with swiglu one output
    fp16(silu(g) * u)."""
    _decode_route_args(hidden_a, expert_ids, segment_offsets, row_index, batch)
    _check_cuda("hidden_b", hidden_b, torch.float16, 2, hidden_a.device)
    if hidden_b.shape != hidden_a.shape:
        raise RuntimeError("hidden_a and hidden_b must have one shape")
    sa = _decode_struct(payload_a, hidden_a.device)
    sb = _decode_struct(payload_b, hidden_a.device)
    out_a = _out_buffer(out_a, batch, sa.outfeatures, hidden_a.device)
    if not swiglu:
        out_b = _out_buffer(out_b, batch, sb.outfeatures, hidden_a.device)
    _lib.check(_lib.load().tris_grouped_decode_pair_forward_block_gr(
        _ptr(hidden_a), _ptr(hidden_b), _ptr(row_index), int(hidden_a.size(0)), batch, _ptr(expert_ids),
        _ptr(segment_offsets), int(expert_ids.numel()), ctypes.byref(sa), ctypes.byref(sb), _ptr(out_a),
        _ptr(out_b) if not swiglu else None, int(bool(swiglu)), _stream(hidden_a)),
        "tris_grouped_decode_pair_forward_block_gr")
    return out_a if swiglu else (out_a, out_b)


def compact3_dequant(payload_tensors: dict, rank: int, expert_ids: torch.Tensor, use_uniform_k64_groups=False):
    """Dense fp16 weights [num, N, rank] of the listed experts (GPU verification kernel)."""
    dev = expert_ids.device
    pay = make_payload_struct(rank, payload_tensors["qweight1"], payload_tensors["qweight2_sparse"],
                              payload_tensors["qweight2_sparse_prefix"], payload_tensors["q_gmap_gr_words"],
                              payload_tensors["q_gmap_gr_offsets"], payload_tensors["q_gmap_gr_meta"],
                              payload_tensors["c_map"], payload_tensors["g_idx"], payload_tensors["col_pack3"],
                              payload_tensors["row_pack3"], None, False, None, False, use_uniform_k64_groups, dev)
    ids = expert_ids.to(torch.int32).contiguous()
    out = torch.empty((ids.numel(), pay.outfeatures, rank), dtype=torch.float16, device=dev)
    _lib.check(_lib.load().tris_compact3_dequant(ctypes.byref(pay), _ptr(ids), ids.numel(), _ptr(out), _stream(ids)),
               "tris_compact3_dequant")
    return out


def gr_decode_dense(q_gmap_gr_words, q_gmap_gr_offsets, q_gmap_gr_meta, expert_ids, packed_rows, outfeatures):
    """Dense packed split bitmaps [num, packed_rows, N] int32 of the listed experts."""
    dev = q_gmap_gr_offsets.device
    ids = expert_ids.to(torch.int32).contiguous()
    words = q_gmap_gr_words
    if words.numel() == 0:
        words = torch.zeros((max(int(q_gmap_gr_offsets.size(0)), 1), 1), dtype=torch.int32, device=dev)
    out = torch.zeros((ids.numel(), packed_rows, outfeatures), dtype=torch.int32, device=dev)
    _lib.check(_lib.load().tris_gr_decode_dense(_ptr(words), _ptr(q_gmap_gr_offsets), _ptr(q_gmap_gr_meta),
                                                int(q_gmap_gr_offsets.size(0)), int(words.size(1)), _ptr(ids),
                                                ids.numel(), packed_rows, outfeatures, _ptr(out), _stream(ids)),
               "tris_gr_decode_dense")
    return out


def backbone_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Scratch for one backbone call's split-K partial sums (no initial contents needed), taken from the
    caching allocator on the current stream: calls on different streams (the shared expert runs beside the
    routed path) never share it, and its reuse is ordered after the call's reduction on that stream."""
    return torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)


# From this many rows on, and with more than BACKBONE_LIBRARY_MIN_ELEMS activation elements (rows x
# in_features), the backbone is a plain dense GEMM better served by the library GEMM (hipBLASLt through
# F.linear, as the reference's compute_shared_hidden, qlinear_cuda.py:4454-4502); otherwise the decode-shaped
# split-K MFMA kernel of tris_backbone_linear.  Measured on MI355X (kernel vs library, us): in 2048 pair at
# 256 rows 12.7 vs 16.4; in 512 at 256 rows 7.3 vs 16.7, at 512 rows 8.1 vs 5.4; in 4096 pair at 256 rows
# 25.3 vs 18.0; in 14336 at 128 rows 23.0 vs 14.6.
BACKBONE_LIBRARY_MIN_ROWS = 256
BACKBONE_LIBRARY_MIN_ELEMS = 1 << 19


# Rows from which a backbone with rank a multiple of 128 and in_features of 32 goes to the tiled split-K GEMM of
# tris_backbone_linear[_pair] (256 x 128 workgroup tiles) instead of the library GEMM.  Measured on MI355X at the
# C2 prefill shapes: the gate/up pair over 2048 tokens 35 us (+ 15.6 us for the reduction that writes the routed
# rows) against the library's 2 x 22 us plus two 5.5 us row gathers; 4096 x 14336 -> 512 91 us + 19.7 us against
# 105.6 us.
BACKBONE_GEMM_MIN_ROWS = 512
# Workgroups the tiled GEMM's launch must have to take a shape (it fills the GPU from 512; with few, long
# workgroups, as for the A3B layer's short rows, the library GEMM is faster).
BACKBONE_GEMM_MIN_WORKGROUPS = 256


def _gemm_workgroups(rows: int, in_features: int, rank: int, tile_m: int = 256, tile_n: int = 128,
                     target: int = 512) -> int:
    """Workgroups of one projection of the tiled GEMM (backbone_gemm_slices / backbone_wide_slice_k in
    tris_backbone.hip): row tiles x column tiles x K slices (at least 16 stages of 32 columns each, at most 16)."""
    tiles = -(-rows // tile_m) * -(-rank // tile_n)
    slices = max(1, min(-(-target // tiles), in_features // 512, 16))
    return tiles * slices


def _backbone_gemm_ok(rows: int, in_features: int, rank: int) -> bool:
    return (rows >= BACKBONE_GEMM_MIN_ROWS and rank % 128 == 0 and rank > 0 and in_features % 32 == 0
            and in_features > 0 and _gemm_workgroups(rows, in_features, rank) >= BACKBONE_GEMM_MIN_WORKGROUPS)


def _backbone_use_library(rows: int, in_features: int, rank: int = 0) -> bool:
    return (rows >= BACKBONE_LIBRARY_MIN_ROWS and rows * in_features > BACKBONE_LIBRARY_MIN_ELEMS
            and not _backbone_gemm_ok(rows, in_features, rank))


def _backbone_library(x, svs, in_scales, row_index):
    """One library GEMM per projection; in_scales: one fp16 input scale (or None) per projection."""
    outs = []
    for sv, sc in zip(svs, in_scales):
        if row_index is not None and x.size(0) < row_index.numel():
            # more routed rows than tokens (top-k > 1): project each token once, then gather the projected rows
            xs = x * sc if sc is not None else x
            outs.append(torch.nn.functional.linear(xs, sv).index_select(0, row_index))
            continue
        xs = x.index_select(0, row_index) if row_index is not None else x
        if sc is not None:
            xs = xs * sc  # fp16 products, as x * ns_col
        outs.append(torch.nn.functional.linear(xs, sv))
    return outs


def backbone_linear(x: torch.Tensor, sv: torch.Tensor, in_scale: torch.Tensor | None = None,
                    row_index: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """hidden = fp16(x[row_index] * in_scale) @ sv^T with fp32 accumulation (compute_shared_hidden).  out: an
    fp16 [rows, rank] buffer to write (e.g. one owned by another stream), else a new tensor."""
    _check_cuda("x", x, torch.float16, 2)
    _check_cuda("shared_sv", sv, torch.float16, 2, x.device)
    if sv.size(1) != x.size(1):
        raise RuntimeError("shared_sv in-features mismatch")
    tokens = int(row_index.numel()) if row_index is not None else int(x.size(0))
    if row_index is not None:
        _check_cuda("row_index", row_index, torch.int64, 1, x.device)
    if in_scale is not None:
        _check_cuda("in_scale", in_scale, torch.float16, 1, x.device)
    rank, in_f = int(sv.size(0)), int(sv.size(1))
    if out is not None:
        _check_cuda("out", out, torch.float16, 2, x.device)
        if tuple(out.shape) != (tokens, rank):
            raise RuntimeError("backbone_linear: out must be [rows, rank]")
    if _backbone_use_library(tokens, in_f, rank):
        res = _backbone_library(x, (sv,), (in_scale,), row_index)[0]
        return res if out is None else out.copy_(res)
    if row_index is not None and x.size(0) < tokens and _backbone_gemm_ok(int(x.size(0)), in_f, rank):
        # more routed rows than tokens: project each token once, then gather the projected rows
        res = backbone_linear(x, sv, in_scale=in_scale).index_select(0, row_index)
        return res if out is None else out.copy_(res)
    if out is None:
        out = torch.empty((tokens, rank), dtype=torch.float16, device=x.device)
    lib = _lib.load()
    ws = backbone_workspace(x.device, int(lib.tris_backbone_workspace_bytes(tokens, in_f, rank)))
    _lib.check(lib.tris_backbone_linear(_ptr(x), tokens, in_f, _ptr(row_index), _ptr(sv), rank, _ptr(in_scale),
                                        _ptr(out), _ptr(ws), int(ws.numel()), _stream(x)), "tris_backbone_linear")
    return out


class BackbonePartials:
    """The fp32 split-K partial sums [slices, rows, rank] of a backbone projection whose reduction was left to its
    consumer (backbone_linear_deferred): grouped_forward_block_gr_predecoded_partials takes them in place of the
    projection's rows.  Holds the call's workspace until then."""

    __slots__ = ("partials", "slices", "rows", "rank")

    def __init__(self, partials: torch.Tensor, slices: int, rows: int, rank: int):
        self.partials, self.slices, self.rows, self.rank = partials, slices, rows, rank


# Rows up to which backbone_linear_deferred leaves the reduction to the consumer (decode batches; the tiled
# GEMM's shapes start far above).
BACKBONE_DEFERRED_MAX_ROWS = 64


def backbone_linear_deferred(x: torch.Tensor, sv: torch.Tensor, in_scale: torch.Tensor | None = None):
    """backbone_linear of x's rows with its split-K reduction left to the consumer (tris_backbone_linear_deferred,
    an extension): a BackbonePartials when the plan splits K, else the fp16 [rows, rank] projection (also for
    shapes past BACKBONE_DEFERRED_MAX_ROWS, which backbone_linear projects).  The partial sums' reduction gives
    backbone_linear's bits."""
    _check_cuda("x", x, torch.float16, 2)
    _check_cuda("shared_sv", sv, torch.float16, 2, x.device)
    if sv.size(1) != x.size(1):
        raise RuntimeError("shared_sv in-features mismatch")
    if in_scale is not None:
        _check_cuda("in_scale", in_scale, torch.float16, 1, x.device)
    rows, in_f, rank = int(x.size(0)), int(sv.size(1)), int(sv.size(0))
    if rows == 0 or rows > BACKBONE_DEFERRED_MAX_ROWS or _backbone_use_library(rows, in_f, rank):
        return backbone_linear(x, sv, in_scale=in_scale)
    out = torch.empty((rows, rank), dtype=torch.float16, device=x.device)
    lib = _lib.load()
    ws = backbone_workspace(x.device, int(lib.tris_backbone_workspace_bytes(rows, in_f, rank)))
    slices = ctypes.c_int32(0)
    _lib.check(lib.tris_backbone_linear_deferred(_ptr(x), rows, in_f, None, _ptr(sv), rank, _ptr(in_scale), _ptr(out),
                                                 _ptr(ws), int(ws.numel()), ctypes.byref(slices), _stream(x)),
               "tris_backbone_linear_deferred")
    n = int(slices.value)
    if n <= 1:
        return out
    part = ws[: n * rows * rank * 4].view(torch.float32).view(n, rows, rank)
    return BackbonePartials(part, n, rows, rank)


PARTIALS_GEMM_MAX_ROWS = 4  # rows grouped_forward_block_gr_predecoded_partials takes (its 4-row kernel instances)


def partials_gemm_ok(payload: dict) -> bool:
    """True when grouped_forward_block_gr_predecoded_partials takes a projection's payload dict: rank <= 512, a
    multiple of 64, and at most 8 row-scale groups (the MFMA kernel's staging of one chunk)."""
    rank = int(payload["g_idx"].size(1))
    return 0 < rank <= 512 and rank % 64 == 0 and int(payload["row_pack3"].size(2)) <= 8


def grouped_forward_block_gr_predecoded_partials(hidden: BackbonePartials, expert_ids, segment_offsets,
                                                 total_problem_tiles, decoded_q_gmap_words, qweight1,
                                                 qweight2_sparse, qweight2_sparse_prefix, c_map, g_idx, col_pack3,
                                                 row_pack3, use_uniform_k64_groups=True, out=None,
                                                 decoded_by_expert=False):
    """compact3_tris_precomputed_grouped_forward_block_gr_predecoded over the rows a deferred backbone projection
    leaves as partial sums (tris_grouped_forward_block_gr_predecoded_partials, an extension): the GEMM's staging
    adds the slices as backbone_linear's reduction would, so the output is that GEMM's over backbone_linear's
    output, bit for bit, without the reduction's launch."""
    if not isinstance(hidden, BackbonePartials):
        raise RuntimeError("grouped_forward_block_gr_predecoded_partials: hidden must be a BackbonePartials")
    if hidden.rows > PARTIALS_GEMM_MAX_ROWS:
        raise RuntimeError(f"grouped_forward_block_gr_predecoded_partials: at most {PARTIALS_GEMM_MAX_ROWS} rows")
    dev = hidden.partials.device
    _check_cuda("expert_ids", expert_ids, torch.int32, 1, dev)
    _check_cuda("segment_offsets", segment_offsets, torch.int32, 1, dev)
    if segment_offsets.size(0) != expert_ids.size(0) + 1:
        raise RuntimeError("segment_offsets must be 1D [segments + 1]")
    total = _host_tiles(total_problem_tiles)
    pay = make_payload_struct(hidden.rank, qweight1, qweight2_sparse, qweight2_sparse_prefix, None, None, None,
                              c_map, g_idx, col_pack3, row_pack3, None, False, None, False, use_uniform_k64_groups,
                              dev, need_gr=False)
    _check_predecoded(decoded_q_gmap_words, expert_ids, pay, dev, decoded_by_expert)
    out = _out_buffer(out, hidden.rows, pay.outfeatures, dev)
    _lib.check(_lib.load().tris_grouped_forward_block_gr_predecoded_partials(
        _ptr(hidden.partials), hidden.slices, hidden.rows, _ptr(expert_ids), _ptr(segment_offsets),
        int(expert_ids.size(0)), total, _ptr(decoded_q_gmap_words), ctypes.byref(pay), _ptr(out),
        1 if decoded_by_expert else 0, _stream(hidden.partials)), "grouped_forward_block_gr_predecoded_partials")
    return out


def grouped_forward_block_gr_predecoded_partials_combine(hidden: BackbonePartials, expert_ids, segment_offsets,
                                                         total_problem_tiles, decoded_q_gmap_words, qweight1,
                                                         qweight2_sparse, qweight2_sparse_prefix, c_map, g_idx,
                                                         col_pack3, row_pack3, inverse_perm, routing_weights_f16,
                                                         out_dtype=torch.bfloat16, use_uniform_k64_groups=True,
                                                         decoded_by_expert=False):
    """grouped_forward_block_gr_predecoded_partials for one token routed to two experts with the routed combine in
    the same launch (tris_grouped_forward_block_gr_predecoded_partials_combine, an extension): returns the token's
    [1, N] output in out_dtype (bf16 or fp16), moe_combine's over the GEMM's rows bit for bit."""
    if not isinstance(hidden, BackbonePartials) or hidden.rows != 2:
        raise RuntimeError("the one-token combine takes the partial sums of 2 routed rows")
    if out_dtype not in (torch.bfloat16, torch.float16):
        raise RuntimeError("out_dtype must be bfloat16 or float16")
    dev = hidden.partials.device
    _check_cuda("expert_ids", expert_ids, torch.int32, 1, dev)
    _check_cuda("segment_offsets", segment_offsets, torch.int32, 1, dev)
    _check_cuda("inverse_perm", inverse_perm, torch.int32, 1, dev)
    _check_cuda("routing_weights_f16", routing_weights_f16, torch.float16, None, dev)
    if int(expert_ids.numel()) != 2 or int(segment_offsets.numel()) != 3:
        raise RuntimeError("the one-token combine takes 2 segments")
    if int(inverse_perm.numel()) != 2 or int(routing_weights_f16.numel()) != 2:
        raise RuntimeError("the one-token combine takes a top-2 route of one token")
    total = _host_tiles(total_problem_tiles)
    pay = make_payload_struct(hidden.rank, qweight1, qweight2_sparse, qweight2_sparse_prefix, None, None, None,
                              c_map, g_idx, col_pack3, row_pack3, None, False, None, False, use_uniform_k64_groups,
                              dev, need_gr=False)
    _check_predecoded(decoded_q_gmap_words, expert_ids, pay, dev, decoded_by_expert)
    out = torch.empty((1, pay.outfeatures), dtype=out_dtype, device=dev)
    w16 = routing_weights_f16.contiguous()
    _lib.check(_lib.load().tris_grouped_forward_block_gr_predecoded_partials_combine(
        _ptr(hidden.partials), hidden.slices, _ptr(expert_ids), _ptr(segment_offsets), total,
        _ptr(decoded_q_gmap_words), ctypes.byref(pay), _ptr(inverse_perm), _ptr(w16),
        1 if out_dtype == torch.bfloat16 else 0, _ptr(out), 1 if decoded_by_expert else 0, _stream(hidden.partials)),
        "grouped_forward_block_gr_predecoded_partials_combine")
    return out


def backbone_linear_pair(x: torch.Tensor, sv_a: torch.Tensor, sv_b: torch.Tensor,
                         row_index: torch.Tensor | None = None, in_scale_a: torch.Tensor | None = None,
                         in_scale_b: torch.Tensor | None = None):
    """(fp16(x[row_index] * in_scale_a) @ sv_a^T, fp16(x[row_index] * in_scale_b) @ sv_b^T) in one launch: the
    gate and up backbones, each with its own ns_mode == 1 input scale (or None)."""
    _check_cuda("x", x, torch.float16, 2)
    _check_cuda("shared_sv_a", sv_a, torch.float16, 2, x.device)
    _check_cuda("shared_sv_b", sv_b, torch.float16, 2, x.device)
    if sv_a.shape != sv_b.shape or sv_a.size(1) != x.size(1):
        raise RuntimeError("backbone pair shape mismatch")
    tokens = int(row_index.numel()) if row_index is not None else int(x.size(0))
    if row_index is not None:
        _check_cuda("row_index", row_index, torch.int64, 1, x.device)
    for name, sc in (("in_scale_a", in_scale_a), ("in_scale_b", in_scale_b)):
        if sc is not None:
            _check_cuda(name, sc, torch.float16, 1, x.device)
            if sc.numel() != x.size(1):
                raise RuntimeError(f"{name} must hold in_features values")
    rank, in_f = int(sv_a.size(0)), int(sv_a.size(1))
    if _backbone_use_library(tokens, in_f, rank):
        out_a, out_b = _backbone_library(x, (sv_a, sv_b), (in_scale_a, in_scale_b), row_index)
        return out_a, out_b
    if row_index is not None and x.size(0) < tokens and _backbone_gemm_ok(int(x.size(0)), in_f, rank):
        # more routed rows than tokens: project each token once, then gather the projected rows
        out_a, out_b = backbone_linear_pair(x, sv_a, sv_b, in_scale_a=in_scale_a, in_scale_b=in_scale_b)
        return out_a.index_select(0, row_index), out_b.index_select(0, row_index)
    out_a = torch.empty((tokens, rank), dtype=torch.float16, device=x.device)
    out_b = torch.empty((tokens, rank), dtype=torch.float16, device=x.device)
    lib = _lib.load()
    ws = backbone_workspace(x.device, int(lib.tris_backbone_pair_workspace_bytes(tokens, in_f, rank)))
    _lib.check(lib.tris_backbone_linear_pair(_ptr(x), tokens, in_f, _ptr(row_index), _ptr(sv_a), _ptr(sv_b), rank,
                                             _ptr(in_scale_a), _ptr(in_scale_b), _ptr(out_a), _ptr(out_b), _ptr(ws),
                                             int(ws.numel()), _stream(x)),
               "tris_backbone_linear_pair")
    return out_a, out_b


def backbone_scatter_ok(tokens: int, sv_a, sv_b) -> bool:
    """True when backbone_linear_pair_scatter can run: two fp16 SV matrices of one shape that the tiled GEMM takes
    (tokens >= 512, rank a multiple of 128, in_features of 32)."""
    if not all(isinstance(sv, torch.Tensor) and sv.dtype == torch.float16 and sv.dim() == 2 and sv.is_contiguous()
               and sv.data_ptr() % 16 == 0 for sv in (sv_a, sv_b)):
        return False
    rank, in_f = int(sv_a.size(0)), int(sv_a.size(1))
    return sv_a.shape == sv_b.shape and _backbone_gemm_ok(tokens, in_f, rank)


def backbone_linear_pair_scatter(x: torch.Tensor, sv_a: torch.Tensor, sv_b: torch.Tensor, inverse_perm: torch.Tensor,
                                 top_k: int, out_rows: int, in_scale_a: torch.Tensor | None = None,
                                 in_scale_b: torch.Tensor | None = None):
    """The gate and up backbones of the tokens x written to their routed rows (tris_backbone_linear_pair_scatter,
    an extension): out[inverse_perm[t * top_k + j]] = fp16(x[t] * in_scale) @ sv^T, the rows the reference's
    compute_shared_hidden gives for x[perm] (qlinear_cuda.py:4454-4502), with each token projected once and no
    gathered copy of the rows.  Returns two fp16 [out_rows, rank] tensors (rows no slot names are unset)."""
    _check_cuda("x", x, torch.float16, 2)
    _check_cuda("shared_sv_a", sv_a, torch.float16, 2, x.device)
    _check_cuda("shared_sv_b", sv_b, torch.float16, 2, x.device)
    _check_cuda("inverse_perm", inverse_perm, torch.int32, 1, x.device)
    if sv_a.shape != sv_b.shape or sv_a.size(1) != x.size(1):
        raise RuntimeError("backbone pair shape mismatch")
    tokens = int(x.size(0))
    if inverse_perm.numel() != tokens * top_k:
        raise RuntimeError("inverse_perm must hold tokens * top_k entries")
    for name, sc in (("in_scale_a", in_scale_a), ("in_scale_b", in_scale_b)):
        if sc is not None:
            _check_cuda(name, sc, torch.float16, 1, x.device)
            if sc.numel() != x.size(1):
                raise RuntimeError(f"{name} must hold in_features values")
    rank, in_f = int(sv_a.size(0)), int(sv_a.size(1))
    out_a = torch.empty((out_rows, rank), dtype=torch.float16, device=x.device)
    out_b = torch.empty((out_rows, rank), dtype=torch.float16, device=x.device)
    lib = _lib.load()
    ws = backbone_workspace(x.device, int(lib.tris_backbone_scatter_workspace_bytes(tokens, in_f, rank, 2)))
    _lib.check(lib.tris_backbone_linear_pair_scatter(_ptr(x), tokens, in_f, _ptr(sv_a), _ptr(sv_b), rank,
                                                     _ptr(in_scale_a), _ptr(in_scale_b), _ptr(inverse_perm), int(top_k),
                                                     int(out_rows), _ptr(out_a), _ptr(out_b), _ptr(ws),
                                                     int(ws.numel()), _stream(x)),
               "tris_backbone_linear_pair_scatter")
    return out_a, out_b


SWIGLU_BACKBONE_MAX_ROWS = 128  # rows of one row group of tris_backbone_swiglu_linear's decode kernel
# rows of its four row groups, for a rank that is not a multiple of 512 (a multiple takes the tiled GEMM above
# SWIGLU_BACKBONE_MAX_ROWS); each group reads the projection again.  Measured on MI355X at the A3B shape (256
# routed rows, in 512, rank 256): one launch in place of the SwiGLU product and a backbone launch
SWIGLU_BACKBONE_GROUPED_MAX_ROWS = 512


def backbone_swiglu_ok(gate: torch.Tensor, sv, in_scale: torch.Tensor | None = None) -> bool:
    """True when backbone_swiglu_linear should run: an fp16 SV matrix, a multiple of 32 columns, 16-byte aligned
    contiguous tensors, and either at most SWIGLU_BACKBONE_MAX_ROWS rows or a prefill-size batch whose rank is a
    multiple of 512 (the tiled GEMM's full-rank tiles; the C entry takes any rank of 128s above 128 rows)."""
    if not isinstance(sv, torch.Tensor) or sv.dtype != torch.float16 or sv.dim() != 2 or not sv.is_contiguous():
        return False
    if gate.dim() != 2 or int(gate.size(1)) % 32 != 0:
        return False
    rows, in_f, rank = int(gate.size(0)), int(gate.size(1)), int(sv.size(0))
    # above one row group of the decode kernel: a rank of 512s takes the tiled GEMM's 128 x 512 tiles (which need
    # enough workgroups); any other rank, the decode kernel's row groups up to SWIGLU_BACKBONE_GROUPED_MAX_ROWS
    if rows > SWIGLU_BACKBONE_MAX_ROWS and rank % 512 == 0 and (rows < BACKBONE_GEMM_MIN_ROWS or _gemm_workgroups(
            rows, in_f, rank, tile_m=128, tile_n=512, target=256) < BACKBONE_GEMM_MIN_WORKGROUPS // 2):
        return False
    if rows > SWIGLU_BACKBONE_GROUPED_MAX_ROWS and rank % 512 != 0:
        return False
    if int(sv.size(1)) != int(gate.size(1)) or sv.data_ptr() % 16 or gate.data_ptr() % 16:
        return False
    return in_scale is None or (in_scale.dtype == torch.float16 and in_scale.numel() == gate.size(1)
                                and in_scale.is_contiguous() and in_scale.data_ptr() % 16 == 0)


def backbone_swiglu_linear(gate: torch.Tensor, up: torch.Tensor, sv: torch.Tensor,
                           in_scale: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """fp16(act_fn(gate) * up [* in_scale]) @ sv^T in one projection with the product formed in its operand
    staging (tris_backbone_swiglu_linear, an extension): the down backbone of a SwiGLU layer without the
    intermediate tensor.  The product is swiglu_mul's, bit for bit."""
    _check_cuda("gate", gate, torch.float16, 2)
    _check_cuda("up", up, torch.float16, 2, gate.device)
    _check_cuda("shared_sv", sv, torch.float16, 2, gate.device)
    if up.shape != gate.shape or int(sv.size(1)) != int(gate.size(1)):
        raise RuntimeError("backbone_swiglu_linear: shape mismatch")
    if in_scale is not None:
        _check_cuda("in_scale", in_scale, torch.float16, 1, gate.device)
    rows, in_f, rank = int(gate.size(0)), int(gate.size(1)), int(sv.size(0))
    if out is None:
        out = torch.empty((rows, rank), dtype=torch.float16, device=gate.device)
    else:
        _check_cuda("out", out, torch.float16, 2, gate.device)
        if tuple(out.shape) != (rows, rank):
            raise RuntimeError("backbone_swiglu_linear: out must be [rows, rank]")
    lib = _lib.load()
    ws = backbone_workspace(gate.device, int(lib.tris_backbone_swiglu_workspace_bytes(rows, in_f, rank)))
    _lib.check(lib.tris_backbone_swiglu_linear(_ptr(gate), _ptr(up), rows, in_f, _ptr(sv), rank, _ptr(in_scale),
                                               _ptr(out), _ptr(ws), int(ws.numel()), _stream(gate)),
               "tris_backbone_swiglu_linear")
    return out


def backbone_swiglu_linear_split(gate: torch.Tensor, up: torch.Tensor, sv: torch.Tensor, split: int,
                                 in_scale: torch.Tensor | None = None, out: torch.Tensor | None = None,
                                 out_hi: torch.Tensor | None = None):
    """backbone_swiglu_linear of two stacked projections, its output split by columns
    (tris_backbone_swiglu_linear_split, an extension): returns (out [rows, split], out_hi [rows, rank - split]).
    On the decode kernel only: at most SWIGLU_BACKBONE_MAX_ROWS rows, or SWIGLU_BACKBONE_GROUPED_MAX_ROWS for a
    rank that is not a multiple of 512."""
    _check_cuda("gate", gate, torch.float16, 2)
    _check_cuda("up", up, torch.float16, 2, gate.device)
    _check_cuda("shared_sv", sv, torch.float16, 2, gate.device)
    if up.shape != gate.shape or int(sv.size(1)) != int(gate.size(1)):
        raise RuntimeError("backbone_swiglu_linear_split: shape mismatch")
    if in_scale is not None:
        _check_cuda("in_scale", in_scale, torch.float16, 1, gate.device)
    rows, in_f, rank = int(gate.size(0)), int(gate.size(1)), int(sv.size(0))
    if not 0 < int(split) < rank:
        raise RuntimeError("backbone_swiglu_linear_split: split outside (0, rank)")
    bufs = []
    for name, t, cols in (("out", out, int(split)), ("out_hi", out_hi, rank - int(split))):
        if t is None:
            t = torch.empty((rows, cols), dtype=torch.float16, device=gate.device)
        else:
            _check_cuda(name, t, torch.float16, 2, gate.device)
            if tuple(t.shape) != (rows, cols) or not t.is_contiguous():
                raise RuntimeError(f"backbone_swiglu_linear_split: {name} must be a contiguous [{rows}, {cols}]")
        bufs.append(t)
    lib = _lib.load()
    ws = backbone_workspace(gate.device, int(lib.tris_backbone_swiglu_workspace_bytes(rows, in_f, rank)))
    _lib.check(lib.tris_backbone_swiglu_linear_split(_ptr(gate), _ptr(up), rows, in_f, _ptr(sv), rank, _ptr(in_scale),
                                                     _ptr(bufs[0]), _ptr(bufs[1]), int(split), _ptr(ws),
                                                     int(ws.numel()), _stream(gate)),
               "tris_backbone_swiglu_linear_split")
    return bufs[0], bufs[1]


# ----------------------------------------------------------------------------------------- 4-bit backbone
class Packed4Matrix:
    """Device tensors of one 4-bit packed matrix (PackedQuantMatrix4bit buffers, qlinear_cuda.py:2637-2786):
    qweight int32 [ceil(cols/8), rows], qzeros int32 [G, ceil(rows/8)], scales fp16 [G, rows], g_idx int32
    [cols]; group_size > 0 when g_idx[c] == c // group_size (a multiple of 8), else 0."""

    __slots__ = ("qweight", "qzeros", "scales", "g_idx", "rows", "cols", "group_size")

    def __init__(self, qweight, qzeros, scales, g_idx, rows: int, cols: int, group_size: int):
        self.qweight, self.qzeros, self.scales, self.g_idx = qweight, qzeros, scales, g_idx
        self.rows, self.cols, self.group_size = int(rows), int(cols), int(group_size)

    def c_struct(self):
        return _lib.TrisPacked4(_ptr(self.qweight), _ptr(self.qzeros), _ptr(self.scales), _ptr(self.g_idx),
                                self.rows, self.cols, int(self.scales.size(0)), self.group_size)


def uniform_group_size(g_idx) -> int:
    """The group size when g_idx[c] == c // size for every column and size is a multiple of 8 (one group:
    cols rounded up to 8), else 0.  Read on the host once per matrix, as the reference's
    resolve_packed4_fast_config reads g_idx (TriSMoE_cuda_kernel.cu:8044-8048)."""
    import numpy as np

    g = g_idx.detach().to("cpu").numpy() if isinstance(g_idx, torch.Tensor) else np.asarray(g_idx)
    g = g.astype(np.int64).reshape(-1)
    cols = int(g.size)
    if cols == 0 or g[0] != 0:
        return 0
    nz = np.flatnonzero(g != 0)
    if nz.size == 0:
        return (cols + 7) // 8 * 8
    size = int(nz[0])
    if size % 8 != 0 or not np.array_equal(g, np.arange(cols) // size):
        return 0
    return size


def _check_packed4(m: Packed4Matrix, device):
    _check_cuda("qweight", m.qweight, torch.int32, 2, device)
    _check_cuda("qzeros", m.qzeros, torch.int32, 2, device)
    _check_cuda("scales", m.scales, torch.float16, 2, device)
    if m.g_idx is not None:
        _check_cuda("g_idx", m.g_idx, torch.int32, 1, device)
    if (m.qweight.size(0) != (m.cols + 7) // 8 or m.qweight.size(1) != m.rows or m.scales.size(1) != m.rows
            or m.qzeros.size(1) != (m.rows + 7) // 8 or m.qzeros.size(0) != m.scales.size(0)):
        raise RuntimeError("packed 4-bit matrix: inconsistent qweight / qzeros / scales shapes")


def packed4_dequant(m: Packed4Matrix) -> torch.Tensor:
    """fp16 [rows, cols] = PackedQuantMatrix4bit.dequantize (qlinear_cuda.py:2761-2786), bit for bit."""
    dev = m.qweight.device
    _check_packed4(m, dev)
    if m.g_idx is None:
        raise RuntimeError("packed4_dequant needs g_idx")
    out = torch.empty((m.rows, m.cols), dtype=torch.float16, device=dev)
    st = m.c_struct()
    _lib.check(_lib.load().tris_packed4_dequant(ctypes.byref(st), _ptr(out), _stream(out)), "tris_packed4_dequant")
    return out


def packed4_backbone_linear(x: torch.Tensor, m: Packed4Matrix, in_scale: torch.Tensor | None = None,
                            row_index: torch.Tensor | None = None) -> torch.Tensor:
    """hidden = fp16(x[row_index] * in_scale) . SV^T straight from the packed matrix (uniform groups)."""
    _check_cuda("x", x, torch.float16, 2)
    _check_packed4(m, x.device)
    if x.size(1) != m.cols:
        raise RuntimeError("packed backbone in-features mismatch")
    tokens = int(row_index.numel()) if row_index is not None else int(x.size(0))
    if row_index is not None:
        _check_cuda("row_index", row_index, torch.int64, 1, x.device)
    if in_scale is not None:
        _check_cuda("in_scale", in_scale, torch.float16, 1, x.device)
    out = torch.empty((tokens, m.rows), dtype=torch.float16, device=x.device)
    lib = _lib.load()
    ws = backbone_workspace(x.device, int(lib.tris_backbone_workspace_bytes(tokens, m.cols, m.rows)))
    st = m.c_struct()
    _lib.check(lib.tris_packed4_backbone_linear(_ptr(x), tokens, _ptr(row_index), ctypes.byref(st), _ptr(in_scale),
                                                _ptr(out), _ptr(ws), int(ws.numel()), _stream(x)),
               "tris_packed4_backbone_linear")
    return out


def packed4_backbone_linear_pair(x: torch.Tensor, ma: Packed4Matrix, mb: Packed4Matrix,
                                 row_index: torch.Tensor | None = None, in_scale_a: torch.Tensor | None = None,
                                 in_scale_b: torch.Tensor | None = None):
    """The gate and up packed backbones of the same rows in one launch, each with its own input scale (or None);
    the same bits as two single calls."""
    _check_cuda("x", x, torch.float16, 2)
    _check_packed4(ma, x.device)
    _check_packed4(mb, x.device)
    if x.size(1) != ma.cols or (ma.rows, ma.cols) != (mb.rows, mb.cols):
        raise RuntimeError("packed backbone pair shape mismatch")
    tokens = int(row_index.numel()) if row_index is not None else int(x.size(0))
    if row_index is not None:
        _check_cuda("row_index", row_index, torch.int64, 1, x.device)
    for name, sc in (("in_scale_a", in_scale_a), ("in_scale_b", in_scale_b)):
        if sc is not None:
            _check_cuda(name, sc, torch.float16, 1, x.device)
            if sc.numel() != x.size(1):
                raise RuntimeError(f"{name} must hold in_features values")
    out_a = torch.empty((tokens, ma.rows), dtype=torch.float16, device=x.device)
    out_b = torch.empty((tokens, mb.rows), dtype=torch.float16, device=x.device)
    lib = _lib.load()
    ws = backbone_workspace(x.device, int(lib.tris_backbone_pair_workspace_bytes(tokens, ma.cols, ma.rows)))
    sa, sb = ma.c_struct(), mb.c_struct()
    _lib.check(lib.tris_packed4_backbone_linear_pair(_ptr(x), tokens, _ptr(row_index), ctypes.byref(sa),
                                                     ctypes.byref(sb), _ptr(in_scale_a), _ptr(in_scale_b),
                                                     _ptr(out_a), _ptr(out_b), _ptr(ws), int(ws.numel()), _stream(x)),
               "tris_packed4_backbone_linear_pair")
    return out_a, out_b


def packed4_linear_forward(input: torch.Tensor, qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
                           g_idx: torch.Tensor, group_size: int | None = None) -> torch.Tensor:
    """The extension's packed4_linear_forward(input, qweight, qzeros, scales, g_idx) (TriSMoE_cuda.cpp binding
    of TriSMoE_cuda_kernel.cu:8023-8137): fp16 [batch, cols] -> [batch, rows].  Uniform groups take the fused
    kernel below BACKBONE_LIBRARY_MIN_ROWS rows; otherwise the matrix is dequantised and projected in fp16
    (the reference's non-fast kernels and its Python fallback, qlinear_cuda.py:4490-4494).  group_size: the
    uniform group size if known (else read from g_idx on the host)."""
    _check_cuda("input", input, torch.float16, 2)
    cols = int(g_idx.numel())
    if input.size(1) != cols:
        raise RuntimeError("packed4_linear_forward: input columns != g_idx length")
    gs = uniform_group_size(g_idx) if group_size is None else int(group_size)
    m = Packed4Matrix(qweight, qzeros, scales, g_idx, int(qweight.size(1)), cols, gs)
    if input.size(0) == 0 or m.rows == 0:
        return torch.zeros((int(input.size(0)), m.rows), dtype=torch.float16, device=input.device)
    if gs > 0 and input.size(0) < BACKBONE_LIBRARY_MIN_ROWS:
        return packed4_backbone_linear(input, m)
    return backbone_linear(input, packed4_dequant(m))


# ----------------------------------------------------------------- null-space compensation
NS_PAYLOAD_TENSORS = ("ns_rank_per_expert", "ns_c2_rank_offsets", "ns_c2_rank_word_offsets", "ns_c1_rank_word_offsets",
                      "ns_c1_group_offsets", "ns_c2_qweight", "ns_c2_qzeros", "ns_c2_scales", "ns_c1_qweight",
                      "ns_c1_qzeros", "ns_c1_scales")


def _ns_struct(ns: dict, infeatures: int, device):
    for k in ("ns_rank_per_expert", "ns_c2_rank_offsets", "ns_c2_rank_word_offsets", "ns_c1_rank_word_offsets",
              "ns_c1_group_offsets"):
        _check_cuda(k, ns[k], torch.int32, 1, device)
    for k in ("ns_c2_qweight", "ns_c2_qzeros", "ns_c1_qweight", "ns_c1_qzeros"):
        _check_cuda(k, ns[k], torch.int32, 2, device)
    for k in ("ns_c2_scales", "ns_c1_scales"):
        _check_cuda(k, ns[k], torch.float16, 2, device)
    E = int(ns["ns_rank_per_expert"].numel())
    if any(int(ns[k].numel()) != E for k in ("ns_c2_rank_offsets", "ns_c2_rank_word_offsets",
                                             "ns_c1_rank_word_offsets", "ns_c1_group_offsets")):
        raise RuntimeError("null-space payload: per-expert offset vectors differ in length")
    if int(ns["ns_c2_qweight"].size(0)) != (infeatures + 7) // 8:
        raise RuntimeError("null-space payload: ns_c2_qweight rows != ceil(infeatures / 8)")
    return _lib.TrisNsPayload(*[_ptr(ns[k]) for k in NS_PAYLOAD_TENSORS], E, int(infeatures),
                              int(ns["ns_c1_scales"].size(1)), int(ns["max_ns_rank"]), int(ns["group_size"]),
                              int(ns["ns_c2_qweight"].size(1)), int(ns["ns_c2_qzeros"].size(1)))


def ns_compensation_apply_(out: torch.Tensor, x_grouped: torch.Tensor, expert_ids: torch.Tensor,
                           segment_offsets: torch.Tensor, ns: dict, accumulate: bool = True) -> torch.Tensor:
    """out[r] = fp16(out[r] + C1_e . fp16(C2_e . x_grouped[r])) for every routed row (accumulate), or the
    compensation alone: the grouped null-space term of run_grouped_structured_expert_forward
    (qlinear_cuda.py:2322-2334) on the HIP kernels."""
    _check_cuda("x_grouped", x_grouped, torch.float16, 2)
    dev = x_grouped.device
    _check_cuda("out", out, torch.float16, 2, dev)
    _check_cuda("expert_ids", expert_ids, torch.int32, 1, dev)
    _check_cuda("segment_offsets", segment_offsets, torch.int32, 1, dev)
    st = _ns_struct(ns, int(x_grouped.size(1)), dev)
    batch = int(x_grouped.size(0))
    if out.size(0) != batch or out.size(1) != st.outfeatures:
        raise RuntimeError("null-space compensation: out must be [batch, outfeatures]")
    x_grouped = _aligned16(x_grouped)
    lib = _lib.load()
    nseg = int(expert_ids.numel())
    ws = ns_workspace(dev, int(lib.tris_grouped_ns_workspace_bytes(batch, nseg, st.infeatures, st.max_ns_rank)))
    _lib.check(lib.tris_grouped_ns_compensation_forward(
        _ptr(x_grouped), batch, _ptr(expert_ids), _ptr(segment_offsets), nseg, ctypes.byref(st), _ptr(ws),
        int(ws.numel()), _ptr(out), int(bool(accumulate)), _stream(x_grouped)), "tris_grouped_ns_compensation_forward")
    return out


def ns_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Scratch for one null-space compensation call's split-K partial sums, from the caching allocator on the
    current stream (the layer runs compensation terms on side streams beside the backbones), so concurrent
    calls never share it."""
    return torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)


def _aligned16(x: torch.Tensor) -> torch.Tensor:
    """x itself when its data starts on a 16-byte boundary (the kernels' vector loads), else a copy."""
    return x if x.data_ptr() % 16 == 0 else x.clone()


def ns_compensation_pair_apply_(out_a, out_b, x: torch.Tensor, expert_ids: torch.Tensor,
                                segment_offsets: torch.Tensor, ns_a, ns_b, accumulate: bool = True,
                                row_index: torch.Tensor | None = None) -> tuple:
    """ns_compensation_apply_ for two payloads over the same rows (the gate and up projections) in one pair
    of launches; the same values as two single calls.  A payload given as None (and its out) is skipped.
    With row_index (int64 [batch], the route's grouped_token_indices), x is the ungrouped input [T, in] and
    grouped row r reads x[row_index[r]]: the gather x.index_select(0, grouped_token_indices) of
    qlinear_cuda.py:2322-2334 done inside the kernel."""
    if ns_a is None or ns_b is None:
        x_g = x if row_index is None else x.index_select(0, row_index)
        for o, ns in ((out_a, ns_a), (out_b, ns_b)):
            if ns is not None:
                ns_compensation_apply_(o, x_g, expert_ids, segment_offsets, ns, accumulate)
        return out_a, out_b
    _check_cuda("x", x, torch.float16, 2)
    dev = x.device
    _check_cuda("out_a", out_a, torch.float16, 2, dev)
    _check_cuda("out_b", out_b, torch.float16, 2, dev)
    _check_cuda("expert_ids", expert_ids, torch.int32, 1, dev)
    _check_cuda("segment_offsets", segment_offsets, torch.int32, 1, dev)
    batch = int(out_a.size(0))
    if row_index is not None:
        _check_cuda("row_index", row_index, torch.int64, 1, dev)
        if int(row_index.numel()) != batch:
            raise RuntimeError("row_index must hold one input row per grouped row")
    elif int(x.size(0)) != batch:
        raise RuntimeError("null-space compensation: x_grouped must have one row per output row")
    in_f = int(x.size(1))
    sa, sb = _ns_struct(ns_a, in_f, dev), _ns_struct(ns_b, in_f, dev)
    for o, st in ((out_a, sa), (out_b, sb)):
        if o.size(0) != batch or o.size(1) != st.outfeatures:
            raise RuntimeError("null-space compensation: out must be [batch, outfeatures]")
    x = _aligned16(x)
    lib = _lib.load()
    nseg = int(expert_ids.numel())
    ws = ns_workspace(dev, int(lib.tris_grouped_ns_pair_workspace_bytes(batch, nseg, in_f, sa.max_ns_rank,
                                                                        sb.max_ns_rank)))
    _lib.check(lib.tris_grouped_ns_compensation_pair_forward(
        _ptr(x), int(x.size(0)), _ptr(row_index), batch, _ptr(expert_ids), _ptr(segment_offsets), nseg,
        ctypes.byref(sa), ctypes.byref(sb), _ptr(ws), int(ws.numel()), _ptr(out_a), _ptr(out_b),
        int(bool(accumulate)), _stream(x)), "tris_grouped_ns_compensation_pair_forward")
    return out_a, out_b


def grouped_ns_compensation_forward(x_grouped, expert_ids, segment_offsets, problem_offsets, total_problem_tiles,
                                    ns_rank_per_expert, ns_c2_rank_offsets, ns_c2_rank_word_offsets,
                                    ns_c1_rank_word_offsets, ns_c1_group_offsets, ns_c2_qweight, ns_c2_qzeros,
                                    ns_c2_scales, ns_c1_qweight, ns_c1_qzeros, ns_c1_scales, max_ns_rank: int,
                                    group_size: int, decode_phase: bool = False) -> torch.Tensor:
    """The extension's grouped_ns_compensation_forward (TriSMoE_cuda_kernel.cu:1208-2145; called at
    qlinear_cuda.py:2103-2124): fp16 [batch, out] compensation C1_e . (C2_e . x) per routed row."""
    ns = {"ns_rank_per_expert": ns_rank_per_expert, "ns_c2_rank_offsets": ns_c2_rank_offsets,
          "ns_c2_rank_word_offsets": ns_c2_rank_word_offsets, "ns_c1_rank_word_offsets": ns_c1_rank_word_offsets,
          "ns_c1_group_offsets": ns_c1_group_offsets, "ns_c2_qweight": ns_c2_qweight, "ns_c2_qzeros": ns_c2_qzeros,
          "ns_c2_scales": ns_c2_scales, "ns_c1_qweight": ns_c1_qweight, "ns_c1_qzeros": ns_c1_qzeros,
          "ns_c1_scales": ns_c1_scales, "max_ns_rank": int(max_ns_rank), "group_size": int(group_size)}
    out = torch.empty((int(x_grouped.size(0)), int(ns_c1_scales.size(1))), dtype=torch.float16,
                      device=x_grouped.device)
    return ns_compensation_apply_(out, x_grouped, expert_ids, segment_offsets, ns, accumulate=False)


def grouped_ns_compensation_fused_decode_forward(x_grouped, expert_ids, segment_offsets, problem_offsets,
                                                 total_problem_tiles, ns_rank_per_expert, ns_c2_rank_offsets,
                                                 ns_c2_rank_word_offsets, ns_c1_rank_word_offsets,
                                                 ns_c1_group_offsets, ns_c2_qweight, ns_c2_qzeros, ns_c2_scales,
                                                 ns_c1_qweight, ns_c1_qzeros, ns_c1_scales, max_ns_rank: int,
                                                 group_size: int) -> torch.Tensor:
    """The extension's grouped_ns_compensation_fused_decode_forward (TriSMoE_cuda.cpp:456-496,
    kernel.cu:8676-8776): the same compensation as grouped_ns_compensation_forward, which the reference
    computes with one fused launch at decode.  Here both names run the decode-shaped split-K kernels."""
    return grouped_ns_compensation_forward(
        x_grouped, expert_ids, segment_offsets, problem_offsets, total_problem_tiles, ns_rank_per_expert,
        ns_c2_rank_offsets, ns_c2_rank_word_offsets, ns_c1_rank_word_offsets, ns_c1_group_offsets, ns_c2_qweight,
        ns_c2_qzeros, ns_c2_scales, ns_c1_qweight, ns_c1_qzeros, ns_c1_scales, max_ns_rank, group_size,
        decode_phase=True)


def _ns_c1_struct(ns: dict, device):
    for k in ("ns_rank_per_expert", "ns_c1_rank_word_offsets", "ns_c1_group_offsets"):
        _check_cuda(k, ns[k], torch.int32, 1, device)
    for k in ("ns_c1_qweight", "ns_c1_qzeros"):
        _check_cuda(k, ns[k], torch.int32, 2, device)
    _check_cuda("ns_c1_scales", ns["ns_c1_scales"], torch.float16, 2, device)
    E = int(ns["ns_rank_per_expert"].numel())
    if any(int(ns[k].numel()) != E for k in ("ns_c1_rank_word_offsets", "ns_c1_group_offsets")):
        raise RuntimeError("grouped NS C1 offset tensor length mismatch")
    out_f = int(ns["ns_c1_qweight"].size(1))
    if int(ns["ns_c1_scales"].size(1)) != out_f or int(ns["ns_c1_qzeros"].size(1)) != (out_f + 7) // 8:
        raise RuntimeError("ns_c1 payload shapes do not match")
    # the C2 fields stay NULL / 0: the C1-only entry does not read them
    return _lib.TrisNsPayload(
        ns_rank_per_expert=_ptr(ns["ns_rank_per_expert"]), ns_c1_rank_word_offsets=_ptr(ns["ns_c1_rank_word_offsets"]),
        ns_c1_group_offsets=_ptr(ns["ns_c1_group_offsets"]), ns_c1_qweight=_ptr(ns["ns_c1_qweight"]),
        ns_c1_qzeros=_ptr(ns["ns_c1_qzeros"]), ns_c1_scales=_ptr(ns["ns_c1_scales"]), num_experts=E,
        outfeatures=out_f, max_ns_rank=int(ns["max_ns_rank"]), group_size=int(ns["group_size"]))


def grouped_ns_c1_forward(hidden, expert_ids, segment_offsets, problem_offsets, total_problem_tiles,
                          ns_rank_per_expert, ns_c1_rank_word_offsets, ns_c1_group_offsets, ns_c1_qweight,
                          ns_c1_qzeros, ns_c1_scales, max_ns_rank: int, group_size: int,
                          decode_phase: bool = False) -> torch.Tensor:
    """The extension's grouped_ns_c1_forward (TriSMoE_cuda.cpp:423-455, kernel.cu:8526-8674): fp16
    [batch, out] = C1_e . hidden[r][0:rank_e] per routed row, for a hidden [batch, max_ns_rank] computed
    elsewhere (a C2 projection shared by every expert, qlinear_cuda.py:1952-2025).  Rows outside every
    segment are zero, as the reference's torch::zeros output."""
    _check_cuda("hidden", hidden, torch.float16, 2)
    dev = hidden.device
    _check_cuda("expert_ids", expert_ids, torch.int32, 1, dev)
    _check_cuda("segment_offsets", segment_offsets, torch.int32, 1, dev)
    if int(hidden.size(1)) != int(max_ns_rank):
        raise RuntimeError("hidden rank mismatch for grouped NS C1 forward")
    if int(segment_offsets.numel()) != int(expert_ids.numel()) + 1:
        raise RuntimeError("segment_offsets length mismatch")
    ns = {"ns_rank_per_expert": ns_rank_per_expert, "ns_c1_rank_word_offsets": ns_c1_rank_word_offsets,
          "ns_c1_group_offsets": ns_c1_group_offsets, "ns_c1_qweight": ns_c1_qweight, "ns_c1_qzeros": ns_c1_qzeros,
          "ns_c1_scales": ns_c1_scales, "max_ns_rank": int(max_ns_rank), "group_size": int(group_size)}
    st = _ns_c1_struct(ns, dev)
    batch = int(hidden.size(0))
    out = torch.zeros((batch, st.outfeatures), dtype=torch.float16, device=dev)
    _lib.check(_lib.load().tris_grouped_ns_c1_forward(
        _ptr(hidden), batch, _ptr(expert_ids), _ptr(segment_offsets), int(expert_ids.numel()), ctypes.byref(st),
        _ptr(out), 0, _stream(hidden)), "tris_grouped_ns_c1_forward")
    return out


# ----------------------------------------------------------------- non-expert compact3 linears
def _is_block_gr(q_gmap_gr_offsets, q_gmap_gr_meta, rank: int, outfeatures: int) -> bool:
    """The reference's format test (kernel.cu:10841-10842): block-GR when the offsets / meta lengths match
    the block grid, else the sparse split-bitmap form."""
    nblk = _num_gr_blocks((rank + 31) // 32, outfeatures)
    return (q_gmap_gr_offsets is not None and int(q_gmap_gr_offsets.numel()) == nblk + 1
            and q_gmap_gr_meta is not None and int(q_gmap_gr_meta.numel()) == nblk)


def _linear_struct(rank, qweight1, qweight2_sparse, qweight2_sparse_prefix, q_gmap_gr_words, q_gmap_gr_offsets,
                   q_gmap_gr_meta, c_map, g_idx, col_pack3, row_pack3, output_scale, has_output_scale, bias, has_bias,
                   device, who):
    """A non-expert module's tensors (2-D / 1-D) as a one-expert payload descriptor: views, no copies."""
    outfeatures = int(qweight1.size(1))
    if not _is_block_gr(q_gmap_gr_offsets, q_gmap_gr_meta, rank, outfeatures):
        raise RuntimeError(f"{who}: sparse split-bitmap payloads are not accepted; convert them to block-GR at load "
                           "(checkpoint.sparse_gmap_to_dense + gr_encode, as GroupedCheckpoint does)")
    one = lambda t: t.unsqueeze(0) if t is not None else None
    g2 = g_idx.reshape(1, -1)
    uniform = bool(torch.equal(g2[:, (torch.arange(rank, device=g2.device) // 64) * 64], g2)) if rank else True
    return make_payload_struct(rank, one(qweight1), one(qweight2_sparse), one(qweight2_sparse_prefix),
                               one(q_gmap_gr_words), one(q_gmap_gr_offsets), one(q_gmap_gr_meta), one(c_map), g2,
                               one(col_pack3), one(row_pack3), one(output_scale) if has_output_scale else output_scale,
                               has_output_scale, one(bias) if has_bias else bias, has_bias, uniform, device, True, who)


def _ns_linear_addend(x16, ns_c1_qweight, ns_c1_qzeros, ns_c1_scales, ns_c1_g_idx, ns_c2_qweight, ns_c2_qzeros,
                      ns_c2_scales, ns_c2_g_idx, outfeatures: int) -> torch.Tensor:
    """fp32 [batch, out] = C1 . (C2 . x) with no rounding between or after, from the exactly dequantised
    packed matrices: the non-expert kernel's null-space term (kernel.cu:2252-2316), which joins the fp32
    accumulator before the output scale."""
    rank = int(x16.size(1))
    ns_rank = int(ns_c2_qweight.size(1))
    c2 = packed4_dequant(Packed4Matrix(ns_c2_qweight, ns_c2_qzeros, ns_c2_scales, ns_c2_g_idx, ns_rank, rank,
                                       uniform_group_size(ns_c2_g_idx)))
    c1 = packed4_dequant(Packed4Matrix(ns_c1_qweight, ns_c1_qzeros, ns_c1_scales, ns_c1_g_idx, outfeatures, ns_rank,
                                       uniform_group_size(ns_c1_g_idx)))
    batch = int(x16.size(0))
    lib = _lib.load()
    hidden = torch.empty((batch, ns_rank), dtype=torch.float32, device=x16.device)
    _lib.check(lib.tris_dense_linear_f32(_ptr(x16), None, batch, rank, _ptr(c2), ns_rank, _ptr(hidden), _stream(x16)),
               "tris_dense_linear_f32")
    addend = torch.empty((batch, outfeatures), dtype=torch.float32, device=x16.device)
    _lib.check(lib.tris_dense_linear_f32(None, _ptr(hidden), batch, ns_rank, _ptr(c1), outfeatures, _ptr(addend),
                                         _stream(x16)), "tris_dense_linear_f32")
    return addend


def compact3_linear_forward(input, qweight1, qweight2_sparse, qweight2_sparse_prefix, q_gmap_sparse,
                            q_gmap_sparse_prefix, q_gmap_gr_words, q_gmap_gr_offsets, q_gmap_gr_meta, c_map, g_idx,
                            col_pack3, row_pack3, input_scale, output_scale, bias, has_input_scale: bool,
                            has_output_scale: bool, has_bias: bool, ns_c1_qweight, ns_c1_qzeros, ns_c1_scales,
                            ns_c1_g_idx, ns_c2_qweight, ns_c2_qzeros, ns_c2_scales, ns_c2_g_idx, has_ns_matrix: bool,
                            split_k_slices: int = 1, request_prefill_tensor_core: bool = False,
                            use_uniform_k64_groups: bool = False) -> torch.Tensor:
    """The extension's compact3_linear_forward (TriSMoE_cuda.cpp:497-563, kernel.cu:10781-11191): fp16
    [batch, out] = fp16((x' . W^T + ns) * output_scale + bias) for one non-expert compact3 matrix, x' the
    input times input_scale per column (fp16), ns the matrix-mode null-space term in fp32.  Block-GR payloads;
    split_k_slices, request_prefill_tensor_core and use_uniform_k64_groups are the reference's launch hints
    (one exact kernel serves every shape here)."""
    who = "compact3_linear_forward"
    _check_cuda("input", input, torch.float16, 2)
    dev = input.device
    rank = int(input.size(1))
    if int(g_idx.numel()) != rank:
        raise RuntimeError(f"{who}: g_idx rank mismatch")
    outfeatures = int(qweight1.size(1))
    st = _linear_struct(rank, qweight1, qweight2_sparse, qweight2_sparse_prefix, q_gmap_gr_words, q_gmap_gr_offsets,
                        q_gmap_gr_meta, c_map, g_idx, col_pack3, row_pack3, output_scale, has_output_scale, bias,
                        has_bias, dev, who)
    batch = int(input.size(0))
    out = torch.zeros((batch, outfeatures), dtype=torch.float16, device=dev)
    if batch == 0 or rank == 0 or outfeatures == 0:
        return out
    scale = None
    if has_input_scale:
        _check_cuda("input_scale", input_scale, torch.float16, 1, dev)
        if int(input_scale.numel()) != rank:
            raise RuntimeError(f"{who}: input_scale length mismatch")
        scale = input_scale
    addend = None
    if has_ns_matrix:
        addend = _ns_linear_addend(input, ns_c1_qweight, ns_c1_qzeros, ns_c1_scales, ns_c1_g_idx, ns_c2_qweight,
                                   ns_c2_qzeros, ns_c2_scales, ns_c2_g_idx, outfeatures)
    _lib.check(_lib.load().tris_compact3_linear_forward(_ptr(input), batch, ctypes.byref(st), _ptr(scale),
                                                        _ptr(addend), _ptr(out), _stream(input)), who)
    return out


def compact3_dual_linear_forward(input, a_qweight1, a_qweight2_sparse, a_qweight2_sparse_prefix, a_gmap_gr_words,
                                 a_gmap_gr_offsets, a_gmap_gr_meta, a_c_map, a_g_idx, a_col_pack3, a_row_pack3,
                                 b_qweight1, b_qweight2_sparse, b_qweight2_sparse_prefix, b_gmap_gr_words,
                                 b_gmap_gr_offsets, b_gmap_gr_meta, b_c_map, b_g_idx, b_col_pack3, b_row_pack3,
                                 split_k_slices: int = 1, use_uniform_k64_groups: bool = False) -> torch.Tensor:
    """The extension's compact3_dual_linear_forward (TriSMoE_cuda.cpp:641-700, kernel.cu:11192-11456): two
    non-expert matrices of the same shape on one input (a shared expert's gate and up), no scale or bias;
    returns them stacked, fp16 [2, batch, out], from one launch."""
    who = "compact3_dual_linear_forward"
    _check_cuda("input", input, torch.float16, 2)
    dev = input.device
    rank = int(input.size(1))
    outfeatures = int(a_qweight1.size(1))
    if int(b_qweight1.size(1)) != outfeatures:
        raise RuntimeError(f"{who}: the two projections' output widths differ")
    sa = _linear_struct(rank, a_qweight1, a_qweight2_sparse, a_qweight2_sparse_prefix, a_gmap_gr_words,
                        a_gmap_gr_offsets, a_gmap_gr_meta, a_c_map, a_g_idx, a_col_pack3, a_row_pack3, None, False,
                        None, False, dev, who)
    sb = _linear_struct(rank, b_qweight1, b_qweight2_sparse, b_qweight2_sparse_prefix, b_gmap_gr_words,
                        b_gmap_gr_offsets, b_gmap_gr_meta, b_c_map, b_g_idx, b_col_pack3, b_row_pack3, None, False,
                        None, False, dev, who)
    batch = int(input.size(0))
    out = torch.zeros((2, batch, outfeatures), dtype=torch.float16, device=dev)
    if batch == 0 or rank == 0 or outfeatures == 0:
        return out
    _lib.check(_lib.load().tris_compact3_dual_linear_forward(_ptr(input), batch, ctypes.byref(sa), ctypes.byref(sb),
                                                             _ptr(out[0]), _ptr(out[1]), _stream(input)), who)
    return out


def compact3_qkv_linear_forward(input, q_qweight1, q_qweight2_sparse, q_qweight2_sparse_prefix, q_gmap_gr_words,
                                q_gmap_gr_offsets, q_gmap_gr_meta, q_c_map, q_g_idx, q_col_pack3, q_row_pack3, q_bias,
                                k_qweight1, k_qweight2_sparse, k_qweight2_sparse_prefix, k_gmap_gr_words,
                                k_gmap_gr_offsets, k_gmap_gr_meta, k_c_map, k_g_idx, k_col_pack3, k_row_pack3, k_bias,
                                v_qweight1, v_qweight2_sparse, v_qweight2_sparse_prefix, v_gmap_gr_words,
                                v_gmap_gr_offsets, v_gmap_gr_meta, v_c_map, v_g_idx, v_col_pack3, v_row_pack3, v_bias,
                                split_k_slices: int = 1, use_uniform_k64_groups: bool = False) -> torch.Tensor:
    """The extension's compact3_qkv_linear_forward (TriSMoE_cuda.cpp:564-640, kernel.cu:11457-11740): the
    attention Q / K / V projections of one input, each fp16((x . W^T) + bias), stacked fp16 [3, batch, out]
    (equal output widths).  Q and K share one launch, V takes a second."""
    who = "compact3_qkv_linear_forward"
    _check_cuda("input", input, torch.float16, 2)
    dev = input.device
    rank = int(input.size(1))
    outfeatures = int(q_qweight1.size(1))
    if int(k_qweight1.size(1)) != outfeatures or int(v_qweight1.size(1)) != outfeatures:
        raise RuntimeError(f"{who}: Q, K and V must have the same output width")
    structs = []
    for (qw1, qw2, qw2p, grw, gro, grm, cmap, gidx, colp, rowp, b) in (
            (q_qweight1, q_qweight2_sparse, q_qweight2_sparse_prefix, q_gmap_gr_words, q_gmap_gr_offsets,
             q_gmap_gr_meta, q_c_map, q_g_idx, q_col_pack3, q_row_pack3, q_bias),
            (k_qweight1, k_qweight2_sparse, k_qweight2_sparse_prefix, k_gmap_gr_words, k_gmap_gr_offsets,
             k_gmap_gr_meta, k_c_map, k_g_idx, k_col_pack3, k_row_pack3, k_bias),
            (v_qweight1, v_qweight2_sparse, v_qweight2_sparse_prefix, v_gmap_gr_words, v_gmap_gr_offsets,
             v_gmap_gr_meta, v_c_map, v_g_idx, v_col_pack3, v_row_pack3, v_bias)):
        has_bias = b is not None and b.numel() > 0
        structs.append(_linear_struct(rank, qw1, qw2, qw2p, grw, gro, grm, cmap, gidx, colp, rowp, None, False, b,
                                      has_bias, dev, who))
    batch = int(input.size(0))
    out = torch.zeros((3, batch, outfeatures), dtype=torch.float16, device=dev)
    if batch == 0 or rank == 0 or outfeatures == 0:
        return out
    lib = _lib.load()
    _lib.check(lib.tris_compact3_dual_linear_forward(_ptr(input), batch, ctypes.byref(structs[0]),
                                                     ctypes.byref(structs[1]), _ptr(out[0]), _ptr(out[1]),
                                                     _stream(input)), who)
    _lib.check(lib.tris_compact3_linear_forward(_ptr(input), batch, ctypes.byref(structs[2]), None, None, _ptr(out[2]),
                                                _stream(input)), who)
    return out


def router_linear_ok(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """True when router_linear can run: x [T, H] and weight [E, H] CUDA tensors of one dtype (bf16 or fp16) on
    one device, contiguous, H a multiple of 8, 16-byte aligned."""
    if not (isinstance(x, torch.Tensor) and isinstance(weight, torch.Tensor)):
        return False
    if x.device.type != "cuda" or weight.device != x.device or x.dtype != weight.dtype:
        return False
    if x.dtype not in (torch.bfloat16, torch.float16) or x.dim() != 2 or weight.dim() != 2:
        return False
    if int(x.size(1)) != int(weight.size(1)) or int(x.size(1)) % 8 or int(x.size(0)) > 16 * 65535:
        return False
    return (x.is_contiguous() and weight.is_contiguous() and x.data_ptr() % 16 == 0
            and weight.data_ptr() % 16 == 0)


def router_linear(x: torch.Tensor, weight: torch.Tensor):
    """The block's router Linear and the expert kernels' input cast in one launch (tris_router_linear):
    returns (router_logits in x's dtype, the same logits as fp32, x16), router_logits = F.linear(x, weight)
    rounded once from the fp32 sum of exact products (modeling_mixtral.py:546), x16 = x.to(float16) (x itself
    when x is fp16)."""
    if not router_linear_ok(x, weight):
        raise RuntimeError("router_linear: x [T, H] and weight [E, H] must be contiguous bf16/fp16 CUDA tensors of "
                           "one dtype, H a multiple of 8, 16-byte aligned")
    tokens, hidden, experts = int(x.size(0)), int(x.size(1)), int(weight.size(0))
    bf16 = x.dtype == torch.bfloat16
    logits = torch.empty((tokens, experts), dtype=x.dtype, device=x.device)
    logits32 = torch.empty((tokens, experts), dtype=torch.float32, device=x.device)
    x16 = torch.empty((tokens, hidden), dtype=torch.float16, device=x.device) if bf16 else x
    _lib.check(_lib.load().tris_router_linear(_ptr(x), _ptr(weight), tokens, hidden, experts, int(bf16), _ptr(logits),
                                              _ptr(logits32), _ptr(x16) if bf16 else None, _stream(x)),
               "tris_router_linear")
    return logits, logits32, x16


def moe_combine(expert_out: torch.Tensor, inverse_perm: torch.Tensor, weights: torch.Tensor,
                shared: torch.Tensor | None = None, expert_comp: torch.Tensor | None = None,
                shared_gate_input: torch.Tensor | None = None, shared_gate_weight: torch.Tensor | None = None,
                out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """out_dtype [T, H] = sum_s fp16(expert_out[inverse_perm[t, s]] * weights[t, s]) (+ shared), fp32-accumulated
    and rounded once (out_dtype bf16 or fp16).  With expert_comp (fp16, the shape of expert_out), each expert row
    is fp16(expert_out + expert_comp) first: the down projection's null-space compensation
    (qlinear_cuda.py:2322-2334) folded into the combine.

    With shared_gate_weight ([H] or [1, H], the one-output gate Linear of the Qwen blocks) the shared expert is
    gated as modeling_qwen2_moe.py:815-818 / modeling_qwen3_5_moe.py:186-188 do it, every step in out_dtype:
    out = dt(dt(routed) + dt(dt(sigmoid(dt(shared_gate_input . w))) * dt(shared))).  shared_gate_input [T, H]
    and the weight are in out_dtype (the block's model dtype)."""
    _check_cuda("expert_out", expert_out, torch.float16, 2)
    dev = expert_out.device
    if out_dtype not in (torch.bfloat16, torch.float16):
        raise RuntimeError("moe_combine: out_dtype must be bfloat16 or float16")
    if expert_comp is not None:
        _check_cuda("expert_comp", expert_comp, torch.float16, 2, dev)
        if expert_comp.shape != expert_out.shape:
            raise RuntimeError("expert_comp must have the shape of expert_out")
    _check_cuda("weights", weights, torch.float16, 2, dev)
    _check_cuda("inverse_perm", inverse_perm, torch.int32, 1, dev)
    tokens, top_k = int(weights.size(0)), int(weights.size(1))
    hidden = int(expert_out.size(1))
    if inverse_perm.numel() != tokens * top_k:
        raise RuntimeError("inverse_perm must hold tokens * top_k entries")
    if shared is not None:
        _check_cuda("shared", shared, torch.float16, 2, dev)
        if tuple(shared.shape) != (tokens, hidden):
            raise RuntimeError("shared must be [tokens, hidden]")
    if shared_gate_weight is not None:
        if shared is None or shared_gate_input is None:
            raise RuntimeError("a shared-expert gate needs the shared output and the gate input")
        _check_cuda("shared_gate_input", shared_gate_input, out_dtype, 2, dev)
        if tuple(shared_gate_input.shape) != (tokens, hidden):
            raise RuntimeError("shared_gate_input must be [tokens, hidden]")
        if shared_gate_weight.numel() != hidden:
            raise RuntimeError("shared_gate_weight must hold hidden values (Linear(hidden, 1))")
        shared_gate_weight = shared_gate_weight.reshape(hidden)
        _check_cuda("shared_gate_weight", shared_gate_weight, out_dtype, 1, dev)
        if hidden % 8 == 0:
            shared_gate_input = _aligned16(shared_gate_input)
            shared_gate_weight = _aligned16(shared_gate_weight)
    out = torch.empty((tokens, hidden), dtype=out_dtype, device=dev)
    if shared_gate_weight is None and out_dtype == torch.bfloat16:
        if expert_comp is None:
            _lib.check(_lib.load().tris_moe_combine(_ptr(expert_out), _ptr(inverse_perm), _ptr(weights), _ptr(shared),
                                                    tokens, top_k, hidden, _ptr(out), _stream(expert_out)),
                       "tris_moe_combine")
        else:
            _lib.check(_lib.load().tris_moe_combine_compensated(
                _ptr(expert_out), _ptr(expert_comp), _ptr(inverse_perm), _ptr(weights), _ptr(shared), tokens, top_k,
                hidden, _ptr(out), _stream(expert_out)), "tris_moe_combine_compensated")
        return out
    _lib.check(_lib.load().tris_moe_combine_gated(
        _ptr(expert_out), _ptr(expert_comp), _ptr(inverse_perm), _ptr(weights), _ptr(shared), _ptr(shared_gate_input),
        _ptr(shared_gate_weight), tokens, top_k, hidden, int(out_dtype == torch.bfloat16), _ptr(out),
        _stream(expert_out)), "tris_moe_combine_gated")
    return out


def swiglu_mul(gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor | None = None,
               comp_gate: torch.Tensor | None = None, comp_up: torch.Tensor | None = None) -> torch.Tensor:
    """fp16 act_fn(gate) * up (modeling_mixtral.py:496): SiLU in fp32 rounded to fp16, then the fp16 product.
    With comp_gate / comp_up, each operand first takes its null-space compensation, fp16(gate + comp_gate)
    (out.add_(compensation), qlinear_cuda.py:2322-2334)."""
    _check_cuda("gate", gate, torch.float16, None)
    _check_cuda("up", up, torch.float16, None, gate.device)
    if gate.shape != up.shape:
        raise RuntimeError("gate and up must have the same shape")
    for name, c in (("comp_gate", comp_gate), ("comp_up", comp_up)):
        if c is not None:
            _check_cuda(name, c, torch.float16, None, gate.device)
            if c.shape != gate.shape:
                raise RuntimeError(f"{name} must have the shape of gate")
    if out is None:
        out = torch.empty_like(gate)
    _check_cuda("out", out, torch.float16, None, gate.device)
    if out.shape != gate.shape:
        raise RuntimeError("out must have the shape of gate")
    if comp_gate is None and comp_up is None:
        _lib.check(_lib.load().tris_swiglu_mul(_ptr(gate), _ptr(up), gate.numel(), _ptr(out), _stream(gate)),
                   "tris_swiglu_mul")
    else:
        _lib.check(_lib.load().tris_swiglu_mul_compensated(_ptr(gate), _ptr(up), _ptr(comp_gate), _ptr(comp_up),
                                                           gate.numel(), _ptr(out), _stream(gate)),
                   "tris_swiglu_mul_compensated")
    return out


def gr_encode(packed, k_min: int = 0, k_max: int = 7, force_raw: bool = False):
    """Host block-GR encoder: int32 [packed_rows, N] (numpy or CPU tensor) -> (words, offsets, meta) int32 numpy."""
    import numpy as np

    arr = np.ascontiguousarray(packed.cpu().numpy() if isinstance(packed, torch.Tensor) else packed, dtype=np.int32)
    rows, n = arr.shape
    nblk = _num_gr_blocks(rows, n)
    words = np.zeros(max(nblk * BLOCK_GR_WORDS_PER_BLOCK, 1), dtype=np.int32)
    offsets = np.zeros(nblk + 1, dtype=np.int32)
    meta = np.zeros(nblk, dtype=np.int32)
    lib = _lib.load()
    total = lib.tris_gr_encode(arr.ctypes.data_as(ctypes.c_void_p), rows, n, k_min, k_max, int(force_raw),
                               words.ctypes.data_as(ctypes.c_void_p), words.size,
                               offsets.ctypes.data_as(ctypes.c_void_p), meta.ctypes.data_as(ctypes.c_void_p))
    _lib.check(int(total), "tris_gr_encode")
    return words[:total].copy(), offsets, meta
