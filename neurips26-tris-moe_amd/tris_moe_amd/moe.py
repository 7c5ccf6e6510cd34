"""Sparse MoE block on the grouped expert path (``modeling_mixtral.py:406-608``).

``TrisSparseMoeBlock.forward(hidden_states) -> (out, router_logits)`` keeps the
reference block's signature and dataflow: router softmax (fp32) -> top-k ->
optional renormalisation (Mixtral/Qwen always, OLMoE when ``norm_topk_prob``,
``modeling_olmoe.py:1053-1058``) -> bf16 -> fp16 cast of the kernel input
(``:83-90``) -> grouped route -> shared backbones -> grouped gate/up pair ->
SiLU * up -> down backbone -> grouped down -> routing-weighted scatter-add in
the output dtype.  An optional always-on fp16 shared expert (A3B-class
layers) runs on a stream of its own beside the routed path and joins in the
combine, through its sigmoid gate when the layer has one, as the Qwen blocks
add it (``modeling_qwen2_moe.py:815-818``, ``modeling_qwen3_5_moe.py:186-188``).

``grouped_moe_forward`` is the same computation with every size fixed by the
input shape (route metadata padded to num_experts segments, launch bounds
from the routed-row count), so it runs without host synchronisation and can
be captured in a HIP graph; ``TrisSparseMoeBlock`` uses it too.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ext
from .qlinear import GROUPED_SEGMENT_M_TILE, shared_projection, shared_projection_pair


def route_topk(router_logits: torch.Tensor, top_k: int, renormalize: bool):
    """modeling_mixtral.py:548-551."""
    weights = F.softmax(router_logits, dim=1, dtype=torch.float)
    weights, selected = torch.topk(weights, top_k, dim=-1)
    if renormalize:
        weights = weights / weights.sum(dim=-1, keepdim=True)
    return weights, selected


def grouped_moe_forward(x16: torch.Tensor, routing_weights: torch.Tensor, selected_experts: torch.Tensor,
                        payloads: dict, backbones: dict, num_experts: int, output_dtype=torch.bfloat16,
                        shared_expert=None, expert_path: str = "auto", x_model: torch.Tensor | None = None
                        ) -> torch.Tensor:
    """The grouped MoE layer on the HIP kernels with no host synchronisation.

    x16 fp16 [T, H]; routing_weights [T, k] (cast to fp16 as in modeling_mixtral.py:555);
    selected_experts int64 [T, k]; payloads {gate, up, down} device payload dicts;
    backbones {gate, up, down}: fp16 SV [rank, in] or qlinear.PackedQuantMatrix4bit, and optionally
    {gate,up,down}_in_scale: the fp16 [in] expert_input_scale of experts[0]'s projection when its ns_mode is 1
    (compute_shared_hidden multiplies the backbone input by it, qlinear_cuda.py:4477-4480; the grouped
    forward projects every expert through experts[0], modeling_mixtral.py:469-470, 497).  payloads may also hold
    matrix-mode null-space payloads under gate_ns / up_ns / down_ns (``qlinear.build_grouped_ns_payload``
    format on the device).  Returns [T, H] in output_dtype.

    shared_expert: None, (w_gate [Is, H], w_up [Is, H], w_down [H, Is]) fp16 added ungated, or those plus the
    shared-expert gate's weight ([1, H] or [H], the model dtype) as a fourth element: the Qwen blocks' gated
    shared expert.  x_model: the block's input in the model dtype (the gate's input, as h in
    modeling_qwen2_moe.py:817); x16 in the gate weight's dtype when None.

    expert_path: "predecoded" decodes the split bitmaps once per projection and runs the MFMA
    grouped GEMMs (needs uniform 64-column groups and no output scale or bias); "fused" decodes
    inside the grouped GEMMs (the in-kernel-decode MFMA kernels when every payload suits them,
    ext.decode_payload_ok); "auto" takes "predecoded" whenever the payloads allow it."""
    T, H = int(x16.size(0)), int(x16.size(1))
    k = int(selected_experts.size(1))
    if T * k == 0:
        return torch.zeros((T, H), dtype=output_dtype, device=x16.device)
    shared = _shared_expert_begin(x16, shared_expert, x_model, output_dtype)
    route = ext.build_grouped_route_device(selected_experts, num_experts, GROUPED_SEGMENT_M_TILE)
    w16 = routing_weights.to(torch.float16).contiguous()
    return _forward_with_route(x16, w16, route, k, payloads, backbones, num_experts, output_dtype, shared,
                               expert_path)


def grouped_moe_forward_from_logits(x16: torch.Tensor, router_logits: torch.Tensor, top_k: int, renormalize: bool,
                                    payloads: dict, backbones: dict, num_experts: int,
                                    output_dtype=torch.bfloat16, shared_expert=None,
                                    expert_path: str = "auto", x_model: torch.Tensor | None = None,
                                    shared_stack: "SharedExpertStack | None" = None) -> torch.Tensor:
    """The layer from router logits: softmax / top-k / renormalisation / route in one kernel when the
    batch is decode-sized (tris_route_topk_grouped), else the token-parallel tris_route_topk (torch's
    route_topk for logits it does not take) + the two-kernel route.  On the
    predecoded path with fp16 gate/up backbones and at most ext.ROUTE_BACKBONE_MAX_TOKENS tokens, the
    gate/up backbones of the tokens run in the router's launch (tris_route_topk_backbone), their split-K
    reduction in the predecode's, and the grouped GEMMs gather their rows through the route's token
    indices (the backbone values equal those of the gathered rows up to the split-K summation order: the
    slice count follows the row count).  shared_expert and x_model: as grouped_moe_forward.  shared_stack: the
    shared expert's weights stacked under the routed backbones (SharedExpertStack); when the batch fits its
    launches, the shared expert runs as their extra columns (_SharedFold) instead of four launches of its own."""
    T, H = int(x16.size(0)), int(x16.size(1))
    if T * top_k == 0:
        return torch.zeros((T, H), dtype=output_dtype, device=x16.device)
    one_launch_router = (router_logits.dtype == torch.float32 and T * top_k <= ext.ROUTE_TOPK_MAX_ROWS
                         and num_experts <= ext.ROUTE_TOPK_MAX_EXPERTS and top_k <= ext.ROUTE_TOPK_MAX_K)
    sc = _in_scales(backbones)
    router_backbone = (one_launch_router and expert_path != "fused" and _predecodable(payloads)
                       and ext.mfma_payload_ok(payloads["gate"]) and ext.mfma_payload_ok(payloads["up"])
                       and ext.route_topk_backbone_ok(x16, backbones["gate"], backbones["up"], sc["gate"], sc["up"]))
    fold = None
    if router_backbone and shared_stack is not None and shared_expert is not None:
        fold = _SharedFold.make(shared_stack, shared_expert, x16, x_model, output_dtype, T * top_k, payloads,
                                backbones)
    if fold is not None:
        route, pending = ext.route_topk_backbone_pair(router_logits, top_k, renormalize, GROUPED_SEGMENT_M_TILE, x16,
                                                      shared_stack.gate, shared_stack.up, split=shared_stack.split_gu,
                                                      out_a_hi=fold.g_s, out_b_hi=fold.u_s)
        return _forward_with_route(x16, route["routing_weights_f16"], route, top_k, payloads, backbones, num_experts,
                                   output_dtype, None, expert_path, backbone_pending=pending, shared_fold=fold)
    shared = _shared_expert_begin(x16, shared_expert, x_model, output_dtype)
    if one_launch_router:
        if router_backbone:
            route, pending = ext.route_topk_backbone_pair(router_logits, top_k, renormalize, GROUPED_SEGMENT_M_TILE,
                                                          x16, backbones["gate"], backbones["up"],
                                                          in_scale_a=sc["gate"], in_scale_b=sc["up"])
            return _forward_with_route(x16, route["routing_weights_f16"], route, top_k, payloads, backbones,
                                       num_experts, output_dtype, shared, expert_path,
                                       backbone_pending=pending)
        route = ext.route_topk_grouped(router_logits, top_k, renormalize, GROUPED_SEGMENT_M_TILE)
        return _forward_with_route(x16, route["routing_weights_f16"], route, top_k, payloads, backbones,
                                   num_experts, output_dtype, shared, expert_path)
    if ext.route_topk_ok(router_logits, top_k):
        # past the one-launch router: the token-parallel softmax / top-k, then the two-kernel route
        _, selected, weights = ext.route_topk(router_logits, top_k, renormalize)
    else:
        weights, selected = route_topk(router_logits, top_k, renormalize)
    route = ext.build_grouped_route_device(selected, num_experts, GROUPED_SEGMENT_M_TILE)
    w16 = weights.to(torch.float16).contiguous()
    return _forward_with_route(x16, w16, route, top_k, payloads, backbones, num_experts, output_dtype, shared,
                               expert_path)


def _sparse(p: dict) -> bool:
    """The payload's split bitmaps are in the sparse form (compact3_use_block_gr false)."""
    return "q_gmap_sparse" in p and not bool(p.get("compact3_use_block_gr", False))


def _predecodable(payloads: dict) -> bool:
    """Every projection has block-GR split bitmaps, uniform 64-column groups and no output scale or bias (the
    predecoded path)."""
    pg, pu, pd = payloads["gate"], payloads["up"], payloads["down"]
    return all(bool(p.get("_compact3_k64_groups_uniform", False)) and not _sparse(p) for p in (pg, pu, pd)) and not any(
        bool(p["has_output_scale"]) or bool(p["has_bias"]) for p in (pg, pu, pd))


def _grouped_projection(p: dict, hidden, expert_ids, seg, prob, tile_bound):
    """One projection's grouped GEMM on the exact kernel: the sparse-form entry (output scale always applied, as
    the reference's sparse kernels do) or the block-GR one."""
    empty = hidden.new_empty((0, 0))
    bias = p["bias"] if p["has_bias"] else empty
    if _sparse(p):
        return ext.compact3_tris_precomputed_grouped_forward(
            hidden, expert_ids, seg, prob, tile_bound, p["qweight1"], p["qweight2_sparse"],
            p["qweight2_sparse_prefix"], p["q_gmap_sparse"], p["q_gmap_sparse_prefix"], p["c_map"], p["g_idx"],
            p["col_pack3"], p["row_pack3"], p["output_scale"], bias, bool(p["has_bias"]))
    return ext.compact3_tris_precomputed_grouped_forward_block_gr(
        hidden, expert_ids, seg, prob, tile_bound, p["qweight1"], p["qweight2_sparse"], p["qweight2_sparse_prefix"],
        p["q_gmap_gr_words"], p["q_gmap_gr_offsets"], p["q_gmap_gr_meta"], p["c_map"], p["g_idx"], p["col_pack3"],
        p["row_pack3"], p["output_scale"], bool(p["has_output_scale"]), bias, bool(p["has_bias"]),
        bool(p.get("_compact3_k64_groups_uniform", False)))


def _forward_with_route(x16, w16, route, k, payloads, backbones, num_experts, output_dtype, shared_expert,
                        expert_path, backbone_pending=None, shared_fold=None):
    if expert_path not in ("auto", "fused", "predecoded"):
        raise ValueError(f"unknown expert_path {expert_path!r}")
    T = int(x16.size(0))
    R = T * k
    gti = route["grouped_token_indices"]
    expert_ids = route["expert_ids"]
    seg = route["segment_offsets"]
    prob = route["problem_offsets"]
    # Launch bound only: every padded segment past the active ones is empty.
    tile_bound = R // GROUPED_SEGMENT_M_TILE + min(num_experts, R) + 1
    pg, pu, pd = payloads["gate"], payloads["up"], payloads["down"]
    ns = _ns_payloads(payloads)
    uniform = bool(pg.get("_compact3_k64_groups_uniform", False) and pu.get("_compact3_k64_groups_uniform", False))
    predecodable = _predecodable(payloads)
    if expert_path == "predecoded" and not predecodable:
        raise RuntimeError("the predecoded expert path needs uniform 64-column groups and no output scale or bias")
    if predecodable and expert_path != "fused":
        return _predecoded_moe_forward(x16, w16, route, payloads, backbones, num_experts, R, output_dtype,
                                       shared_expert, backbone_pending=backbone_pending, shared_fold=shared_fold)
    if backbone_pending is not None or shared_fold is not None:
        raise RuntimeError("a backbone launched beside the router needs the predecoded expert path")
    if not any(_sparse(p) for p in (pg, pu, pd)) and all(ext.decode_payload_ok(p) for p in (pg, pu, pd)):
        return _decode_fused_moe_forward(x16, w16, route, payloads, backbones, num_experts, R, output_dtype,
                                         shared_expert)
    sc = _in_scales(backbones)
    hid_g, hid_u = shared_projection_pair(x16, backbones["gate"], backbones["up"], row_index=gti,
                                          in_scale_a=sc["gate"], in_scale_b=sc["up"])
    empty = x16.new_empty((0, 0))
    if _sparse(pg) or _sparse(pu):
        g_out = _grouped_projection(pg, hid_g, expert_ids, seg, prob, tile_bound)
        u_out = _grouped_projection(pu, hid_u, expert_ids, seg, prob, tile_bound)
    else:
        g_out, u_out = ext.compact3_tris_precomputed_grouped_dual_forward_block_gr(
            hid_g, hid_u, expert_ids, seg, prob, tile_bound,
            pg["qweight1"], pg["qweight2_sparse"], pg["qweight2_sparse_prefix"], pg["q_gmap_gr_words"],
            pg["q_gmap_gr_offsets"], pg["q_gmap_gr_meta"], pg["c_map"], pg["g_idx"], pg["col_pack3"], pg["row_pack3"],
            pg["output_scale"], bool(pg["has_output_scale"]), pg["bias"] if pg["has_bias"] else empty,
            pu["qweight1"], pu["qweight2_sparse"], pu["qweight2_sparse_prefix"], pu["q_gmap_gr_words"],
            pu["q_gmap_gr_offsets"], pu["q_gmap_gr_meta"], pu["c_map"], pu["g_idx"], pu["col_pack3"], pu["row_pack3"],
            pu["output_scale"], bool(pu["has_output_scale"]), pu["bias"] if pu["has_bias"] else empty, uniform)
    if ns["gate"] is not None or ns["up"] is not None:
        ext.ns_compensation_pair_apply_(g_out, u_out, x16, expert_ids, seg, ns["gate"], ns["up"], row_index=gti)
    mlp = F.silu(g_out) * u_out
    hid_d = shared_projection(mlp, backbones["down"], in_scale=sc["down"])
    d_out = _grouped_projection(pd, hid_d, expert_ids, seg, prob, tile_bound)
    if ns["down"] is not None:
        ext.ns_compensation_apply_(d_out, mlp, expert_ids, seg, ns["down"])
    return _combine(x16, d_out, route, w16, output_dtype, shared_expert)


def _in_scales(backbones: dict) -> dict:
    """The backbone input scales of the layer (None where absent)."""
    return {key: backbones.get(f"{key}_in_scale") for key in ("gate", "up", "down")}


def _ns_payloads(payloads: dict) -> dict:
    """The layer's matrix-mode null-space payloads (keys gate_ns, up_ns, down_ns, as the reference's
    _forward_grouped fetches them, modeling_mixtral.py:437-450, 503-509), None where absent or rank 0."""
    out = {}
    for key in ("gate", "up", "down"):
        ns = payloads.get(f"{key}_ns")
        out[key] = ns if isinstance(ns, dict) and int(ns.get("max_ns_rank", 0)) > 0 else None
    return out


class _SharedPending:
    """The shared expert's fp16 output [T, H], computed on a side stream beside the routed path (the buffer
    belongs to the caller's stream, which waits for the side stream before the combine reads it), and its gate
    (the weight and its input, both in the combine's dtype) or None."""

    __slots__ = ("out", "stream", "gate_weight", "gate_input")

    def __init__(self, out, stream, gate_weight, gate_input):
        self.out, self.stream, self.gate_weight, self.gate_input = out, stream, gate_weight, gate_input


class SharedExpertStack:
    """The always-on shared expert's fp16 weights stacked under the routed backbones, so its projections run as
    extra columns of the routed path's launches: gate / up [rank + Is, H] (the routed gate or up backbone SV, then
    the shared expert's weight) and down [rank_d + H, Is] (the routed down backbone, then the shared down weight).
    Needs fp16 backbones without input scales and a shared intermediate size equal to the routed one (the shared
    rows then stack under the routed rows of the down backbone's input)."""

    __slots__ = ("gate", "up", "down", "split_gu", "split_d")

    def __init__(self, backbones: dict, shared_expert):
        wg, wu, wd = shared_expert[:3]
        self.gate = torch.cat([backbones["gate"], wg]).contiguous()
        self.up = torch.cat([backbones["up"], wu]).contiguous()
        self.down = torch.cat([backbones["down"], wd]).contiguous()
        self.split_gu = int(backbones["gate"].size(0))
        self.split_d = int(backbones["down"].size(0))

    @staticmethod
    def ok(backbones: dict, shared_expert) -> bool:
        if shared_expert is None or len(shared_expert) not in (3, 4):
            return False
        wg, wu, wd = shared_expert[:3]
        svs = [backbones.get(k) for k in ("gate", "up", "down")]
        if any(backbones.get(f"{k}_in_scale") is not None for k in ("gate", "up", "down")):
            return False
        ts = svs + [wg, wu, wd]
        if not all(isinstance(t, torch.Tensor) and t.dtype == torch.float16 and t.dim() == 2 for t in ts):
            return False
        if len({t.device for t in ts}) != 1:
            return False
        sv_g, sv_u, sv_d = svs
        # gate / up: one input width; down: the shared and routed intermediates agree
        return (sv_g.shape == sv_u.shape and wg.shape == wu.shape and int(wg.size(1)) == int(sv_g.size(1))
                and int(wd.size(1)) == int(wg.size(0)) == int(sv_d.size(1)))


class _SharedFold:
    """One step's shared expert as extra columns of the routed launches.  Its gate and up always ride in the gate/up
    backbone launched beside the router (the stack's split projection).  With split_down, its rows stack under the
    routed rows in g_all / u_all (the dual GEMM fills the first R rows, the backbone the last T) and one launch of
    the stacked down weights projects both; otherwise (routed and shared rows together past the SwiGLU backbone's
    128 rows, or a shared intermediate other than the routed one) its gate and up land in g_s / u_s and its down
    projection runs apart, after the routed gate/up GEMM.
    gate_weight / gate_input: the combine's gate operands (None without a gate)."""

    __slots__ = ("stack", "split_down", "g_all", "u_all", "g_s", "u_s", "wd", "gate_weight", "gate_input")

    @classmethod
    def make(cls, stack, shared_expert, x16, x_model, output_dtype, R, payloads, backbones):
        """The fold of this step, or None when the batch is outside the launches it rides in."""
        T = int(x16.size(0))
        n_mlp = int(payloads["gate"]["qweight1"].size(2))
        inter = int(shared_expert[0].size(0))
        if R <= FUSED_SWIGLU_MAX_ROWS or any(v is not None for v in _ns_payloads(payloads).values()):
            return None
        f = cls()
        f.stack = stack
        f.wd = shared_expert[2]
        f.split_down = R + T <= FOLD_SPLIT_DOWN_MAX_ROWS and inter == n_mlp
        dev = x16.device
        if f.split_down:
            f.g_all = torch.empty((R + T, n_mlp), dtype=torch.float16, device=dev)
            f.u_all = torch.empty((R + T, n_mlp), dtype=torch.float16, device=dev)
            f.g_s, f.u_s = f.g_all[R:], f.u_all[R:]
        else:
            f.g_all = f.u_all = None
            f.g_s = torch.empty((T, inter), dtype=torch.float16, device=dev)
            f.u_s = torch.empty((T, inter), dtype=torch.float16, device=dev)
        f.gate_weight, f.gate_input = _shared_gate_operands(shared_expert, x16, x_model, output_dtype)
        return f

    def down_apart(self, main) -> "_SharedPending":
        """The shared expert's down projection of act_fn(g) * u on its own rows (the fold without split_down), on
        the caller's stream, as _shared_expert_begin runs it."""
        out = torch.empty((int(self.g_s.size(0)), int(self.wd.size(0))), dtype=torch.float16, device=self.g_s.device)
        if ext.backbone_swiglu_ok(self.g_s, self.wd):
            ext.backbone_swiglu_linear(self.g_s, self.u_s, self.wd, out=out)
        else:
            ext.backbone_linear(ext.swiglu_mul(self.g_s, self.u_s), self.wd, out=out)
        return _SharedPending(out, main, self.gate_weight, self.gate_input)


def _shared_gate_operands(shared_expert, x16, x_model, output_dtype):
    """The shared expert's gate weight and its input in the combine's dtype (None, None without a gate)."""
    if len(shared_expert) != 4 or shared_expert[3] is None:
        return None, None
    gate_w = shared_expert[3]
    cd = gate_w.dtype if gate_w.dtype in (torch.bfloat16, torch.float16) else torch.bfloat16
    if output_dtype is not None:
        cd = _combine_dtype(output_dtype)
    src = x_model if x_model is not None else x16
    return gate_w.reshape(-1).to(cd).contiguous(), src.to(cd).contiguous()


def _combine_dtype(output_dtype) -> torch.dtype:
    """The dtype the combine writes: the output dtype when bf16 or fp16, else bf16 (then cast)."""
    return output_dtype if output_dtype in (torch.bfloat16, torch.float16) else torch.bfloat16


def _shared_expert_begin(x16, shared_expert, x_model=None, output_dtype=None):
    """Start the always-on shared expert down(act_fn(gate x) * up x) on side stream 2 (on the caller's stream
    below SHARED_EXPERT_SIDE_STREAM_MIN_TOKENS tokens): gate and up in one
    backbone launch, then the down projection with act_fn(g) * u formed in its operand staging (or SiLU and
    the product in fp16 as F.silu(g) * u, then the down projection), the reference's fp16 MLP.  Returns a
    _SharedPending or None."""
    if shared_expert is None:
        return None
    if isinstance(shared_expert, _SharedPending):
        return shared_expert
    if len(shared_expert) not in (3, 4):
        raise RuntimeError("shared_expert must be (w_gate, w_up, w_down) or (w_gate, w_up, w_down, gate_weight)")
    wg, wu, wd = shared_expert[:3]
    T, H = int(x16.size(0)), int(x16.size(1))
    dev = x16.device
    gate_w, gate_in = _shared_gate_operands(shared_expert, x16, x_model, output_dtype)
    main = torch.cuda.current_stream(dev)
    out = torch.empty((T, H), dtype=torch.float16, device=dev)
    side = _side_stream(dev, 2) if T >= SHARED_EXPERT_SIDE_STREAM_MIN_TOKENS else main
    if side is not main:
        side.wait_stream(main)
    with torch.cuda.stream(side):
        g, u = ext.backbone_linear_pair(x16, wg, wu)
        if ext.backbone_swiglu_ok(g, wd):
            ext.backbone_swiglu_linear(g, u, wd, out=out)
        else:
            ext.backbone_linear(ext.swiglu_mul(g, u), wd, out=out)
    return _SharedPending(out, side, gate_w, gate_in)


def _combine(x16, d_out, route, w16, output_dtype, shared, d_comp=None):
    """The routed combine in the output dtype, with the shared expert's output (a _SharedPending, or shared
    weights run here) joined ungated or through its gate."""
    shared = _shared_expert_begin(x16, shared, output_dtype=output_dtype)
    cd = _combine_dtype(output_dtype)
    kw = {}
    if shared is not None:
        main = torch.cuda.current_stream(x16.device)
        if shared.stream != main:
            main.wait_stream(shared.stream)
        kw["shared"] = shared.out
        if shared.gate_weight is not None:
            kw["shared_gate_weight"] = shared.gate_weight.to(cd)
            kw["shared_gate_input"] = shared.gate_input.to(cd)
    out = ext.moe_combine(d_out, route["inverse_perm"], w16, expert_comp=d_comp, out_dtype=cd, **kw)
    return out if output_dtype == cd else out.to(output_dtype)


def _predecode_buffer(p, slots, device):
    packed_rows, n = int(p["qweight1"].size(1)), int(p["qweight1"].size(2))
    nblk = ((packed_rows + 1) // 2) * ((n + 63) // 64)
    return torch.empty((slots, nblk, 128), dtype=torch.int32, device=device)


_SIDE_STREAMS: dict = {}


def _side_stream(device: torch.device, which: int = 0) -> torch.cuda.Stream:
    """Extra streams per device (default priority) for work that overlaps the main chain: 0 for the
    bitmap decodes and the down compensation, 1 for the gate/up compensation, 2 for the shared expert."""
    key = (device.index if device.index is not None else torch.cuda.current_device(), which)
    if key not in _SIDE_STREAMS:
        _SIDE_STREAMS[key] = torch.cuda.Stream(device=device)
    return _SIDE_STREAMS[key]


# Up to this many routed rows the gate/up GEMM applies act_fn(g) * u in its epilogue; above it the
# separate gate and up workgroups plus tris_swiglu_mul are faster (measured on MI355X at the Mixtral
# decode shape: 17.6 vs 18.9 us at 2 rows, 49.7 vs 42.3 us at 32 rows).
FUSED_SWIGLU_MAX_ROWS = 4

# From this mean of routed rows per segment the grouped GEMMs run weight-stationary, which stages
# materialised rows faster than it gathers them through token indices (C2 prefill: 0.68 against 0.92 ms), so the
# backbones project the routed rows there; below it the GEMMs gather (A3B T = 1024: 353 -> 339 us).
WS_GATHER_MIN_ROWS_PER_SEGMENT = 64

# The down projection's null-space compensation runs on the side stream beside the down backbone and GEMM
# (True) or on the caller's stream after the GEMM (False).
NS_DOWN_BESIDE_GEMM = True

# The gate/up null-space compensation runs on a side stream beside the decodes and backbones (True) or on the
# caller's stream before them (False; measured on MI355X at the Mixtral decode shape, T = 16: 133.2 us beside,
# 136.7 us before).
NS_GATE_UP_BESIDE = True

# The block runs its shared expert as extra columns of the routed launches when the batch fits them
# (SharedExpertStack, _SharedFold; measured on MI355X at the A3B shape: T = 1 60.6 -> 48.9 us, T = 32 140.2 ->
# 133.4 us); False keeps its four launches of its own.
FOLD_SHARED_EXPERT = True

# After the fused gate/up GEMM the down backbone's split-K partial sums go straight to the down GEMM, whose
# staging adds them (ext.backbone_linear_deferred, ext.grouped_forward_block_gr_predecoded_partials): the same
# bits without the reduction's launch.
DOWN_PARTIALS_IN_GEMM = True
# Stacked rows (routed + shared) up to which the folded shared expert's down projection runs as extra columns of the
# routed down backbone's launch (tris_backbone_swiglu_linear_split); above, in launches of its own.  The decode
# kernel's row groups would take up to 512, but the stacked product's unused quadrants (routed rows x the shared
# columns) cost more than the two launches: measured on MI355X at the A3B shape, T = 32 134.5 against 133.8 us,
# T = 48 156.1 against 152.5 us.
FOLD_SPLIT_DOWN_MAX_ROWS = 128

# One token on two experts (Mixtral at T = 1): the routed combine in the down GEMM's launch
# (ext.grouped_forward_block_gr_predecoded_partials_combine), the combine launch's bits.
COMBINE_IN_DOWN_GEMM = True

# The decode step decodes every expert's split bitmaps (slot e for expert e) when the batch routes at least this
# many rows per expert, so the predecode does not wait for the router's selection (measured on MI355X at the
# Mixtral shape: T = 8, 16 rows over 8 experts, 92.4 -> 89.0 us; T = 4, 8 rows over ~5 experts, 78.8 against
# 78.4 us, where decoding every expert is 1.6 times the blocks; T = 16 routes 32 rows and leaves an expert idle
# about once in 12 steps).
DECODE_ALL_MIN_ROWS_PER_EXPERT = 2

# From this many tokens the shared expert, when it runs in launches of its own, runs on a side stream beside the
# routed experts; below it on the
# caller's stream, since a graph's cross-queue join costs more than the overlap saves there (measured on MI355X at
# the A3B shape: T = 1 64.3 -> 59.0 us inline; T = 32 138 vs 139 us; T = 1024 339 vs 356 us).
SHARED_EXPERT_SIDE_STREAM_MIN_TOKENS = 32


def _predecoded_moe_forward(x16, w16, route, payloads, backbones, num_experts, R, output_dtype, shared_expert,
                            backbone_pending=None, predecoded=None, decoded_by_expert=False, shared_fold=None):
    """Uniform-group payloads without output scale or bias: GR-decode every routed expert's split
    bitmaps once per projection (TriSMoE_cuda.cpp:836-853), then run the predecoded grouped GEMMs
    (TriSMoE_cuda.cpp:855-889, 922-974).  Active experts come first in the padded route, so
    min(num_experts, R) segments cover every routed row and the later segments are empty.  The
    decodes depend only on the route and run in one launch ahead of the gate/up backbones.

    Null-space compensation terms (qlinear_cuda.py:2322-2334) are computed apart from the GEMM outputs and
    joined later, with the same fp16 adds: gate/up's on a stream of their own from the routed inputs
    (read through the route's token indices), beside the decodes and the backbones, and added inside
    act_fn(g) * u; the down projection's on the side stream beside the down backbone and GEMM, and added
    inside the combine.

    backbone_pending: the gate/up backbones of the tokens launched beside the router (ext.BackbonePending);
    their split-K reduction runs in the predecode's launch and the gate/up GEMMs gather their rows through
    the route's token indices.  predecoded: {gate, up, down} buffers already filled for this route (with the
    backbone's reduction) by the launch that built it (ext.route_predecode_multi); decoded_by_expert: they hold
    every expert, slot e for expert e (its decode_all).  shared_fold: the shared expert as extra columns of the
    launches (_SharedFold): the gate/up backbones (launched beside the router) left its gate and up rows in
    shared_fold.g_s / u_s, below the routed rows of g_all / u_all when the down backbone's launch computes its down
    projection too (split_down); else its down projection runs apart after the routed gate/up GEMM."""
    slots = min(num_experts, R)
    eid = route["expert_ids"][:slots]
    seg = route["segment_offsets"][: slots + 1]
    prob = route["problem_offsets"][: slots + 1]
    tile_bound = R // GROUPED_SEGMENT_M_TILE + slots + 1
    pg, pu, pd = payloads["gate"], payloads["up"], payloads["down"]
    ns = _ns_payloads(payloads)
    dev = x16.device
    if predecoded is not None and (backbone_pending is None or any(v is not None for v in ns.values())):
        raise RuntimeError("predecoded buffers come with the router-launched backbones and no null-space payloads")
    if shared_fold is not None and (backbone_pending is None or shared_expert is not None or R <= FUSED_SWIGLU_MAX_ROWS
                                    or any(v is not None for v in ns.values())):
        raise RuntimeError("a folded shared expert comes with the router-launched backbones, above "
                           f"{FUSED_SWIGLU_MAX_ROWS} routed rows and without null-space payloads")
    if decoded_by_expert and (predecoded is None or R <= FUSED_SWIGLU_MAX_ROWS):
        raise RuntimeError("bitmaps decoded for every expert come from route_predecode_multi(decode_all=True), "
                           f"above {FUSED_SWIGLU_MAX_ROWS} routed rows")
    bufs = predecoded if predecoded is not None else {
        name: _predecode_buffer(p, slots, dev) for name, p in (("gate", pg), ("up", pu), ("down", pd))}
    main = torch.cuda.current_stream(dev)
    side = _side_stream(dev)
    n_mlp = int(pg["qweight1"].size(2))
    comp_g = comp_u = None
    ns_side = None
    if ns["gate"] is not None or ns["up"] is not None:
        # the gate/up compensation terms from the routed inputs, beside the decodes and the backbones; the
        # buffers belong to the caller's stream, which waits for this one before reading or freeing them
        comp_g = torch.empty((R, n_mlp), dtype=torch.float16, device=dev) if ns["gate"] is not None else None
        comp_u = torch.empty((R, n_mlp), dtype=torch.float16, device=dev) if ns["up"] is not None else None
        ns_side = _side_stream(dev, 1) if NS_GATE_UP_BESIDE else main
        if ns_side is not main:
            ns_side.wait_stream(main)
        with torch.cuda.stream(ns_side):
            ext.ns_compensation_pair_apply_(comp_g, comp_u, x16, eid, seg, ns["gate"], ns["up"], accumulate=False,
                                            row_index=route["grouped_token_indices"])
        if ns_side is main:
            ns_side = None

    # one launch for the three projections, on the caller's stream: beside the backbones it takes the CUs
    # first and delays them, and the join costs more than the overlap saves (measured on MI355X at the
    # Mixtral decode shape)
    order = (("gate", pg), ("up", pu), ("down", pd))
    pre_jobs = [(bufs[name], p["q_gmap_gr_words"], p["q_gmap_gr_offsets"], p["q_gmap_gr_meta"],
                 int(p["qweight1"].size(1)), int(p["qweight1"].size(2))) for name, p in order]
    decoded = bufs
    sc = _in_scales(backbones)
    if predecoded is not None:
        hid_g, hid_u = backbone_pending.out_a, backbone_pending.out_b
        gather = route["grouped_token_indices"]
    elif backbone_pending is not None:
        ext.grouped_block_gr_predecode_multi(pre_jobs, eid, backbone=backbone_pending)
        hid_g, hid_u = backbone_pending.out_a, backbone_pending.out_b
        gather = route["grouped_token_indices"]
    elif ext.mfma_payload_ok(pg) and ext.mfma_payload_ok(pu) and R < WS_GATHER_MIN_ROWS_PER_SEGMENT * slots:
        ext.grouped_block_gr_predecode_multi(pre_jobs, eid)
        # the tokens' gate/up backbones; the decode-sized MFMA GEMMs read each routed row through its token index,
        # so the projected rows are never gathered (T rows projected instead of T * top_k)
        hid_g, hid_u = shared_projection_pair(x16, backbones["gate"], backbones["up"], in_scale_a=sc["gate"],
                                              in_scale_b=sc["up"])
        gather = route["grouped_token_indices"]
    else:
        ext.grouped_block_gr_predecode_multi(pre_jobs, eid)
        tokens = int(x16.size(0))
        if R % tokens == 0 and ext.backbone_scatter_ok(tokens, backbones["gate"], backbones["up"]):
            # each token projected once and stored to the rows the route sends it to (no gathered copy)
            hid_g, hid_u = ext.backbone_linear_pair_scatter(x16, backbones["gate"], backbones["up"],
                                                            route["inverse_perm"], R // tokens, R,
                                                            in_scale_a=sc["gate"], in_scale_b=sc["up"])
        else:
            hid_g, hid_u = shared_projection_pair(x16, backbones["gate"], backbones["up"],
                                                  row_index=route["grouped_token_indices"], in_scale_a=sc["gate"],
                                                  in_scale_b=sc["up"])
        gather = None
    if ns_side is not None:
        main.wait_stream(ns_side)
    names = ("qweight1", "qweight2_sparse", "qweight2_sparse_prefix", "c_map", "g_idx", "col_pack3", "row_pack3")
    # every routed row lies in a segment, so the outputs need no zero fill
    mlp = None
    hid_d = None
    if R <= FUSED_SWIGLU_MAX_ROWS and comp_g is None and comp_u is None:
        mlp = torch.empty((R, n_mlp), dtype=torch.float16, device=dev)
        # few rows: the gate/up GEMM with act_fn(g) * u in its epilogue (one launch)
        ext.compact3_tris_precomputed_grouped_swiglu_forward_block_gr_predecoded(
            hid_g, hid_u, eid, seg, prob, tile_bound, decoded["gate"], *[pg[k] for k in names], decoded["up"],
            *[pu[k] for k in names], out=mlp, row_index=gather)
    else:
        # more rows: gate and up in separate workgroups (more of them resident per CU), then act_fn(g) * u;
        # the same bits as the fused epilogue
        if shared_fold is not None and shared_fold.split_down:  # the routed rows above the shared expert's
            g, u = shared_fold.g_all[:R], shared_fold.u_all[:R]
        else:
            g = torch.empty((R, n_mlp), dtype=torch.float16, device=dev)
            u = torch.empty((R, n_mlp), dtype=torch.float16, device=dev)
        ext.compact3_tris_precomputed_grouped_dual_forward_block_gr_predecoded(
            hid_g, hid_u, eid, seg, prob, tile_bound, decoded["gate"], *[pg[k] for k in names], decoded["up"],
            *[pu[k] for k in names], True, out_a=g, out_b=u, row_index=gather, decoded_by_expert=decoded_by_expert)
        if shared_fold is not None and not shared_fold.split_down:
            shared_expert = shared_fold.down_apart(main)
        if shared_fold is not None and shared_fold.split_down:
            # one launch of the stacked down weights over the stacked rows: the routed rows' backbone in its first
            # columns, the shared expert's down projection in the rest
            hid_all, sh_all = ext.backbone_swiglu_linear_split(shared_fold.g_all, shared_fold.u_all,
                                                               shared_fold.stack.down, shared_fold.stack.split_d)
            hid_d = hid_all[:R]
            shared_expert = _SharedPending(sh_all[R:], main, shared_fold.gate_weight, shared_fold.gate_input)
        elif (comp_g is None and comp_u is None and ns["down"] is None
                and ext.backbone_swiglu_ok(g, backbones["down"], sc["down"])):
            # act_fn(g) * u formed inside the down backbone (nothing else reads the product)
            hid_d = ext.backbone_swiglu_linear(g, u, backbones["down"], in_scale=sc["down"])
        else:
            # g + comp_g and u + comp_u (fp16 adds) inside act_fn(g) * u
            mlp = torch.empty((R, n_mlp), dtype=torch.float16, device=dev)
            ext.swiglu_mul(g, u, out=mlp, comp_gate=comp_g, comp_up=comp_u)
    n_out = int(pd["qweight1"].size(2))
    comp_d = None
    if ns["down"] is not None and NS_DOWN_BESIDE_GEMM:
        # the down compensation beside the down backbone and GEMM; its buffer belongs to the caller's stream,
        # which waits for the side stream before reading or freeing it
        comp_d = torch.empty((R, n_out), dtype=torch.float16, device=dev)
        side.wait_stream(main)
        with torch.cuda.stream(side):
            ext.ns_compensation_apply_(comp_d, mlp, eid, seg, ns["down"], accumulate=False)
    if hid_d is None:
        if (DOWN_PARTIALS_IN_GEMM and R <= ext.PARTIALS_GEMM_MAX_ROWS and isinstance(backbones["down"], torch.Tensor)
                and ext.partials_gemm_ok(pd)):
            # the down backbone's split-K slices added by the down GEMM's staging (no reduction launch)
            hid_d = ext.backbone_linear_deferred(mlp, backbones["down"], in_scale=sc["down"])
        else:
            hid_d = shared_projection(mlp, backbones["down"], in_scale=sc["down"])
    if (isinstance(hid_d, ext.BackbonePartials) and COMBINE_IN_DOWN_GEMM and int(x16.size(0)) == 1 and R == 2
            and shared_expert is None and ns["down"] is None):
        # one token on two experts: the routed combine in the down GEMM's launch (its two units take the two rows)
        cd = _combine_dtype(output_dtype)
        out = ext.grouped_forward_block_gr_predecoded_partials_combine(
            hid_d, eid, seg, tile_bound, decoded["down"], *[pd[k] for k in names], route["inverse_perm"], w16,
            out_dtype=cd, decoded_by_expert=decoded_by_expert)
        return out if output_dtype == cd else out.to(output_dtype)
    d_out = torch.empty((R, n_out), dtype=torch.float16, device=dev)
    if isinstance(hid_d, ext.BackbonePartials):
        ext.grouped_forward_block_gr_predecoded_partials(
            hid_d, eid, seg, tile_bound, decoded["down"], *[pd[k] for k in names], True, out=d_out,
            decoded_by_expert=decoded_by_expert)
    else:
        ext.compact3_tris_precomputed_grouped_forward_block_gr_predecoded(
            hid_d, eid, seg, prob, tile_bound, decoded["down"], *[pd[k] for k in names], True, out=d_out,
            decoded_by_expert=decoded_by_expert)
    if comp_d is not None:
        main.wait_stream(side)
    elif ns["down"] is not None:
        ext.ns_compensation_apply_(d_out, mlp, eid, seg, ns["down"])
    return _combine(x16, d_out, route, w16, output_dtype, shared_expert, d_comp=comp_d)


def _decode_fused_moe_forward(x16, w16, route, payloads, backbones, num_experts, R, output_dtype, shared_expert,
                              hidden_pair=None):
    """The GR split bitmaps decoded inside the grouped GEMMs (the reference's fused decode path,
    TriSMoE_cuda_kernel.cu:5382-5586): gate and up in one launch with act_fn(g) * u in its epilogue, read through
    the route's token indices from per-token backbone outputs (every routed row of a token has the same shared
    hidden, modeling_mixtral.py:467-476), then the down GEMM over the routed rows.  Output scale and bias, and
    null-space compensation terms, are applied as in the predecoded path.  hidden_pair: the tokens' gate/up
    backbone outputs already computed (the decode step's router launch), else they are projected here."""
    slots = min(num_experts, R)
    eid = route["expert_ids"][:slots]
    seg = route["segment_offsets"][: slots + 1]
    gti = route["grouped_token_indices"]
    pg, pu, pd = payloads["gate"], payloads["up"], payloads["down"]
    ns = _ns_payloads(payloads)
    sc = _in_scales(backbones)
    if hidden_pair is not None:
        hid_g, hid_u = hidden_pair
    else:
        hid_g, hid_u = shared_projection_pair(x16, backbones["gate"], backbones["up"], in_scale_a=sc["gate"],
                                              in_scale_b=sc["up"])
    dev = x16.device
    n_mlp = int(pg["qweight1"].size(2))
    # every routed row lies in one of the min(E, R) segments, so the outputs need no zero fill
    if ns["gate"] is None and ns["up"] is None:
        mlp = ext.grouped_decode_pair_forward(hid_g, hid_u, pg, pu, eid, seg, R, row_index=gti, swiglu=True,
                                              out_a=torch.empty((R, n_mlp), dtype=torch.float16, device=dev))
    else:
        g, u = ext.grouped_decode_pair_forward(
            hid_g, hid_u, pg, pu, eid, seg, R, row_index=gti,
            out_a=torch.empty((R, n_mlp), dtype=torch.float16, device=dev),
            out_b=torch.empty((R, int(pu["qweight1"].size(2))), dtype=torch.float16, device=dev))
        comp_g = torch.empty((R, n_mlp), dtype=torch.float16, device=dev) if ns["gate"] is not None else None
        comp_u = torch.empty((R, n_mlp), dtype=torch.float16, device=dev) if ns["up"] is not None else None
        ext.ns_compensation_pair_apply_(comp_g, comp_u, x16, eid, seg, ns["gate"], ns["up"], accumulate=False,
                                        row_index=gti)
        mlp = ext.swiglu_mul(g, u, comp_gate=comp_g, comp_up=comp_u)
    hid_d = shared_projection(mlp, backbones["down"], in_scale=sc["down"])
    d_out = ext.grouped_decode_forward(hid_d, pd, eid, seg, R,
                                       out=torch.empty((R, int(pd["qweight1"].size(2))), dtype=torch.float16,
                                                       device=dev))
    if ns["down"] is not None:
        ext.ns_compensation_apply_(d_out, mlp, eid, seg, ns["down"])
    return _combine(x16, d_out, route, w16, output_dtype, shared_expert)


def decode_prologue_ok(x: torch.Tensor, router_weight: torch.Tensor, top_k: int, num_experts: int, payloads: dict,
                       backbones: dict, expert_path: str = "auto") -> bool:
    """The block's decode step can start with ext.router_backbone_pair and route in its predecode's launch
    (ext.route_predecode_multi): bf16 activations and router, the one-wavefront route (tokens * top_k <= 64, at
    most 8 experts), fp16 gate/up backbones, no null-space payloads, and the expert path's payload conditions:
    the predecoded MFMA path ("auto", "predecoded"), or the in-kernel-decode GEMMs ("fused")."""
    if x.dim() != 2:
        return False
    t = int(x.size(0))
    if not (0 < t and t * top_k <= ext.ROUTE_WAVE_MAX_ROWS and num_experts <= ext.ROUTE_WAVE_MAX_EXPERTS):
        return False
    if expert_path == "fused":
        if not all(not _sparse(p) and ext.decode_payload_ok(p) for p in payloads.values()):
            return False
    elif not (_predecodable(payloads) and ext.mfma_payload_ok(payloads["gate"])
              and ext.mfma_payload_ok(payloads["up"])):
        return False
    if any(v is not None for v in _ns_payloads(payloads).values()):
        return False
    sc = _in_scales(backbones)
    return ext.router_backbone_ok(x, router_weight, backbones["gate"], backbones["up"], sc["gate"], sc["up"])


def grouped_moe_decode_step(x: torch.Tensor, router_weight: torch.Tensor, top_k: int, renormalize: bool,
                            payloads: dict, backbones: dict, num_experts: int, output_dtype=torch.bfloat16,
                            shared_expert=None, expert_path: str = "auto"):
    """The whole block at decode from its bf16 input (decode_prologue_ok): the router Linear, the fp16 cast and
    the gate/up backbones in one launch, the route and the predecode (with the backbones' split-K reduction) in
    the next, then the grouped GEMMs and the combine.  expert_path "fused": the route launch only reduces the
    backbones, and the grouped GEMMs decode the split bitmaps themselves.  Returns (out [T, H] in output_dtype,
    router_logits bf16 [T, E]).  The same outputs as TrisSparseMoeBlock's other path, bit for bit."""
    sc = _in_scales(backbones)
    logits, logits32, x16, pending = ext.router_backbone_pair(x, router_weight, backbones["gate"], backbones["up"],
                                                              in_scale_a=sc["gate"], in_scale_b=sc["up"])
    T = int(x.size(0))
    R = T * top_k
    shared = _shared_expert_begin(x16, shared_expert, x, output_dtype)
    if expert_path == "fused":
        # the route and the backbones' reduction in one launch, then the GEMMs that decode the bitmaps themselves
        route = ext.route_predecode_multi(logits32, top_k, renormalize, GROUPED_SEGMENT_M_TILE, [], backbone=pending)
        out = _decode_fused_moe_forward(x16, route["routing_weights_f16"], route, payloads, backbones, num_experts, R,
                                        output_dtype, shared, hidden_pair=(pending.out_a, pending.out_b))
        return out, logits
    # with rows enough to reach nearly every expert, every expert is decoded (slot e for expert e), so the decoders
    # need nothing from the route and start without reading the logits
    decode_all = R >= DECODE_ALL_MIN_ROWS_PER_EXPERT * num_experts and R > FUSED_SWIGLU_MAX_ROWS
    slots = num_experts if decode_all else min(num_experts, R)
    dev = x.device
    order = (("gate", payloads["gate"]), ("up", payloads["up"]), ("down", payloads["down"]))
    bufs = {name: _predecode_buffer(p, slots, dev) for name, p in order}
    jobs = [(bufs[name], p["q_gmap_gr_words"], p["q_gmap_gr_offsets"], p["q_gmap_gr_meta"],
             int(p["qweight1"].size(1)), int(p["qweight1"].size(2))) for name, p in order]
    route = ext.route_predecode_multi(logits32, top_k, renormalize, GROUPED_SEGMENT_M_TILE, jobs, backbone=pending,
                                      decode_all=decode_all)
    out = _predecoded_moe_forward(x16, route["routing_weights_f16"], route, payloads, backbones, num_experts, R,
                                  output_dtype, shared, backbone_pending=pending, predecoded=bufs,
                                  decoded_by_expert=decode_all)
    return out, logits


class TrisSparseMoeBlock(nn.Module):
    """Grouped-expert sparse MoE block (MixtralSparseMoeBlock / OlmoeSparseMoeBlock / Qwen2MoeSparseMoeBlock
    shape).  The router ``gate`` is an nn.Linear in the model dtype (``router_dtype``, bf16 by default), as the
    reference's block keeps it; its logits go through an fp32 softmax (modeling_mixtral.py:546-549).

    shared_expert: None or (w_gate [Is, H], w_up [Is, H], w_down [H, Is]) fp16, the always-on shared expert of
    the Qwen-style blocks.  shared_expert_gate: its gate's weight ([1, H] or [H]); the block then holds
    ``shared_expert_gate = nn.Linear(H, 1, bias=False)`` in the model dtype and adds
    sigmoid(shared_expert_gate(h)) * shared_expert(h) in the output dtype, as modeling_qwen2_moe.py:815-818
    and modeling_qwen3_5_moe.py:186-188 do.  Without it the shared expert is added ungated."""

    def __init__(self, hidden_size: int, num_experts: int, top_k: int, payloads: dict, backbones: dict,
                 router_weight: torch.Tensor | None = None, renormalize: bool = True, shared_expert=None,
                 router_dtype: torch.dtype = torch.bfloat16, shared_expert_gate: torch.Tensor | None = None):
        super().__init__()
        self.hidden_dim = hidden_size
        self.num_experts = num_experts
        self.top_k = top_k
        self.renormalize = renormalize
        self.gate = nn.Linear(hidden_size, num_experts, bias=False, dtype=router_dtype)
        if router_weight is not None:
            self.gate.weight.data = router_weight.to(router_dtype)
        self.payloads = payloads
        self.backbones = backbones
        self.expert_path = "auto"  # grouped_moe_forward's expert_path
        self.shared_expert = tuple(shared_expert) if shared_expert is not None else None
        self.shared_expert_gate = None
        if shared_expert_gate is not None:
            if self.shared_expert is None:
                raise ValueError("shared_expert_gate needs a shared_expert")
            self.shared_expert_gate = nn.Linear(hidden_size, 1, bias=False, dtype=router_dtype,
                                                device=shared_expert_gate.device)
            self.shared_expert_gate.weight.data = shared_expert_gate.reshape(1, hidden_size).to(router_dtype)
        # the shared expert's weights stacked under the routed backbones (its projections then ride in the routed
        # launches at decode batches)
        self.shared_stack = (SharedExpertStack(backbones, self.shared_expert)
                             if SharedExpertStack.ok(backbones, self.shared_expert) else None)

    def _shared(self, model_dtype: torch.dtype):
        if self.shared_expert is None or self.shared_expert_gate is None:
            return self.shared_expert
        return (*self.shared_expert, self.shared_expert_gate.weight.detach().to(model_dtype))

    def forward_routed(self, hidden_states: torch.Tensor, router_logits: torch.Tensor,
                       x16: torch.Tensor | None = None) -> torch.Tensor:
        """The block after the router: [T, H] activations and [T, E] logits -> [T, H].  x16: the activations
        already cast to fp16 (else cast here)."""
        output_dtype = hidden_states.dtype
        if x16 is None:
            x16 = hidden_states.to(torch.float16) if hidden_states.dtype == torch.bfloat16 else hidden_states
        if x16.dtype != torch.float16 or x16.device.type != "cuda":
            raise RuntimeError("grouped expert kernels require CUDA float16/bfloat16 hidden states")
        logits = router_logits if router_logits.dtype == torch.float32 else router_logits.float()
        return grouped_moe_forward_from_logits(x16.contiguous(), logits.contiguous(), self.top_k,
                                               self.renormalize, self.payloads, self.backbones, self.num_experts,
                                               output_dtype, self._shared(output_dtype),
                                               expert_path=self.expert_path, x_model=hidden_states.contiguous(),
                                               shared_stack=self.shared_stack if FOLD_SHARED_EXPERT else None)

    def forward(self, hidden_states: torch.Tensor):
        """modeling_mixtral.py:539-608: hidden_states [B, S, H] (bf16 or fp16) -> (out [B, S, H] in the input
        dtype, router_logits [B*S, E] in the router's dtype).  At decode (decode_prologue_ok) the block runs as
        grouped_moe_decode_step; otherwise, when the activations and the router share the model dtype, the router
        Linear and the fp16 cast run as one launch (ext.router_linear); else the Linear is torch's."""
        batch, seq, hidden = hidden_states.shape
        flat = hidden_states.reshape(-1, hidden)
        weight = self.gate.weight.detach()
        if decode_prologue_ok(flat, weight, self.top_k, self.num_experts, self.payloads, self.backbones,
                              self.expert_path):
            out, router_logits = grouped_moe_decode_step(flat, weight, self.top_k, self.renormalize, self.payloads,
                                                         self.backbones, self.num_experts, flat.dtype,
                                                         self._shared(flat.dtype), expert_path=self.expert_path)
            return out.reshape(batch, seq, hidden), router_logits
        if ext.router_linear_ok(flat, weight):
            router_logits, logits32, x16 = ext.router_linear(flat, weight)
            out = self.forward_routed(flat, logits32, x16=x16)
        else:
            router_logits = self.gate(flat.to(self.gate.weight.dtype))
            out = self.forward_routed(flat, router_logits)
        return out.reshape(batch, seq, hidden), router_logits
