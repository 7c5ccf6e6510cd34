"""CPU-only checks of the product's host side and of the oracle's dequant / route / layer pins.

* the C-ABI library loads and exports every symbol declared in include/tris_moe_hip.h;
* argument-contract errors come back as RuntimeError without touching a GPU;
* the product's host GR encoder is bit-identical to the oracle (known answers + random);
* the product's packing helpers equal the oracle's restatement of pack_utils.py;
* oracle fp16 arithmetic equals single-rounding float64 arithmetic;
* the oracle's weight reconstruction equals the reference CPU formula
  (qlinear_cuda.py:4213-4236, masks and per-term fp16 products in torch CPU half);
* the oracle's route equals a brute-force grouping;
* the oracle MoE layer agrees with a float64 evaluation of the same weights.
"""
import ctypes
import math
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from gr_cases import block_from_positions, case_positions, load_known_answers, random_bitmap, structured_bitmap

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "tris_moe_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tris_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_header_symbols(tris):
    from tris_moe_amd import _lib

    lib = _lib.load()
    names = declared_functions()
    assert "tris_grouped_forward_block_gr" in names and len(names) >= 12
    for name in names:
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert lib.tris_abi_version() == 2


def test_ext_module_passes_reference_abi_probe(tris):
    """qlinear_cuda.py:14-37 requires these callables and ABI attribute."""
    ext = tris["ext"]
    required = ("compact3_linear_forward", "compact3_qkv_linear_forward", "compact3_dual_linear_forward",
                "compact3_tris_precomputed_grouped_forward_block_gr",
                "compact3_tris_precomputed_grouped_dual_forward_block_gr",
                "compact3_tris_precomputed_grouped_block_gr_predecode",
                "compact3_tris_precomputed_grouped_forward_block_gr_predecoded",
                "compact3_tris_precomputed_grouped_dual_forward_block_gr_predecoded",
                "compact3_tris_precomputed_grouped_forward_block_gr_predecoded_hybrid",
                "compact3_tris_precomputed_grouped_dual_forward_block_gr_predecoded_hybrid")
    assert ext.TRIS_COMPACT3_KERNEL_ABI_VERSION == 2
    for name in required:
        assert callable(getattr(ext, name)), name
    import torch

    with pytest.raises(RuntimeError):   # a CPU input is outside the kernel contract, as the reference's CHECK_CUDA
        ext.compact3_linear_forward(*([torch.zeros((2, 2), dtype=torch.float16)] * 28))


def test_c_abi_argument_errors_without_gpu(tris):
    from tris_moe_amd import _lib

    lib = _lib.load()
    rc = lib.tris_build_grouped_route(None, 1, 2, 8, 0, None, None, None, None, None, None, None, None, None, None)
    assert rc == -1 and b"m_tile" in lib.tris_last_error()
    rc = lib.tris_grouped_forward_block_gr(None, 4, None, None, None, 1, 1, None, None, None)
    assert rc == -1 and b"null payload" in lib.tris_last_error()
    assert lib.tris_backbone_workspace_bytes(1, 4096, 512) > 0    # split-K partial sums at decode
    assert lib.tris_backbone_pair_workspace_bytes(1, 4096, 512) > 0
    assert lib.tris_backbone_workspace_bytes(4096, 64, 512) == 0  # one slice: no scratch
    rc = lib.tris_backbone_linear(None, 2, 4096, None, None, 512, None, ctypes.c_void_p(16), None, 0, None)
    assert rc == -1 and b"null input" in lib.tris_last_error()
    rc = lib.tris_backbone_linear_pair(None, 2, 4096, None, ctypes.c_void_p(16), None, 512, None, None,
                                       ctypes.c_void_p(16), ctypes.c_void_p(16), None, 0, None)
    assert rc == -1 and b"null sv_b" in lib.tris_last_error()


def test_ext_rejects_cpu_tensors(tris):
    ext = tris["ext"]
    with pytest.raises(RuntimeError, match="CUDA"):
        ext.build_grouped_route(torch.zeros((2, 2), dtype=torch.long), 4, 4)
    with pytest.raises(RuntimeError, match="CUDA"):
        ext.backbone_linear(torch.zeros((2, 8), dtype=torch.float16), torch.zeros((4, 8), dtype=torch.float16))


@pytest.mark.parametrize("case", load_known_answers()["single_block"], ids=lambda c: c["name"])
def test_product_encoder_known_answers(tris, oracle_mod, case):
    dense = block_from_positions(case_positions(case))
    got = tris["ext"].gr_encode(dense)
    want = oracle_mod.gr_encode(dense)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)
    assert got[2].tolist() == [case["meta"]]


@pytest.mark.parametrize("p", [0.0, 0.05, 0.15, 0.3, 0.9])
@pytest.mark.parametrize("kmin,kmax", [(0, 7), (2, 4), (5, 5)])
def test_product_encoder_matches_oracle(tris, oracle_mod, p, kmin, kmax):
    rng = np.random.default_rng(int(p * 100) + kmin * 10 + kmax)
    dense = random_bitmap(rng, 16, 200, p)
    got = tris["ext"].gr_encode(dense, kmin, kmax)
    want = oracle_mod.gr_encode(dense, kmin, kmax)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)


@pytest.mark.parametrize("kind", ["full", "corners", "stripes", "sparse_long_runs"])
def test_product_encoder_structured(tris, oracle_mod, kind):
    dense = structured_bitmap(kind, 7, 65, np.random.default_rng(1))
    for force_raw in (False, True):
        got = tris["ext"].gr_encode(dense, force_raw=force_raw)
        want = oracle_mod.gr_encode(dense, force_raw=force_raw)
        for g, w in zip(got, want):
            np.testing.assert_array_equal(g, w)


def test_product_encoder_rejects_bad_k_bounds(tris):
    with pytest.raises(RuntimeError, match="k bounds"):
        tris["ext"].gr_encode(np.zeros((2, 64), dtype=np.int32), 3, 9)


def test_product_packing_matches_oracle(oracle_mod):
    from tris_moe_amd import packing

    rng = np.random.default_rng(2)
    for n, k in ((5, 7), (64, 512), (33, 100)):
        m = rng.random((n, k)) < 0.4
        np.testing.assert_array_equal(packing.pack_bool_matrix(m), oracle_mod.pack_bool_matrix(m))
        v = rng.random(k) < 0.3
        np.testing.assert_array_equal(packing.pack_bool_vector(v), oracle_mod.pack_bool_vector(v))
        np.testing.assert_array_equal(packing.sparse_prefix(v), oracle_mod.sparse_prefix(v))
        np.testing.assert_array_equal(packing.pack_sparse_bool_matrix(m, v), oracle_mod.pack_sparse_bool_matrix(m, v))
        h = rng.standard_normal((4, k)).astype(np.float16)
        np.testing.assert_array_equal(packing.pack_half4(*h), oracle_mod.pack_half4(*h))
        np.testing.assert_array_equal(oracle_mod.unpack_bool_matrix(oracle_mod.pack_bool_matrix(m), k), m)


def test_fp16_arithmetic_single_rounding(oracle_mod):
    """Products/sums computed via fp32 then rounded equal one rounding of the exact (float64) result."""
    rng = np.random.default_rng(4)
    bits = rng.integers(0, 0x7C00, size=(2, 200000), dtype=np.uint16)  # finite non-negative halves
    sign = rng.integers(0, 2, size=(2, 200000), dtype=np.uint16) << 15
    a, b = (bits | sign).view(np.float16)
    exact_mul = (a.astype(np.float64) * b.astype(np.float64)).astype(np.float16)
    exact_add = (a.astype(np.float64) + b.astype(np.float64)).astype(np.float16)
    np.testing.assert_array_equal(oracle_mod.f16_mul(a, b).view(np.uint16), exact_mul.view(np.uint16))
    np.testing.assert_array_equal(oracle_mod.f16_add(a, b).view(np.uint16), exact_add.view(np.uint16))


def _reference_cpu_dequant(oracle_mod, ex, gmap_dense, n, k):
    """qlinear_cuda.py:4213-4236 restated with torch CPU half ops (masks and per-term products)."""
    half = torch.float16
    b1 = torch.from_numpy(oracle_mod.unpack_bool_matrix(ex["qweight1"], k)).to(half) * 2 - 1
    sal = torch.from_numpy(oracle_mod.unpack_bool_vector(ex["c_map"], k))
    nonsal = ~sal
    q2 = ex["qweight2_sparse"]
    b2 = torch.zeros((n, k), dtype=torch.bool)
    if int(sal.sum()) > 0 and q2.shape[0] > 0:
        b2[:, sal] = torch.from_numpy(oracle_mod.unpack_bool_matrix(q2, int(sal.sum())))
    b2 = b2.to(half) * 2 - 1
    g = torch.from_numpy(oracle_mod.unpack_bool_matrix(gmap_dense, k))
    cols = [torch.from_numpy(c.astype(np.float16)) for c in oracle_mod.unpack_half4(ex["col_pack3"])]
    rows = [torch.from_numpy(r.astype(np.float16))[:, torch.from_numpy(ex["g_idx"].astype(np.int64))]
            for r in oracle_mod.unpack_half4(ex["row_pack3"])]
    smask = sal.unsqueeze(0).expand(n, -1).to(half)
    dmask = (nonsal.unsqueeze(0) & g).to(half)
    nmask = (nonsal.unsqueeze(0) & ~g).to(half)
    w = torch.zeros((n, k), dtype=half)
    w += b1 * (rows[0] * cols[0].unsqueeze(0)) * smask
    w += b2 * (rows[1] * cols[1].unsqueeze(0)) * smask
    w += b1 * (rows[2] * cols[2].unsqueeze(0)) * dmask
    w += b1 * (rows[3] * cols[3].unsqueeze(0)) * nmask
    return w.numpy()


@pytest.mark.parametrize("n,k,p", [(64, 128, 0.15), (100, 256, 0.3), (70, 96, 0.05)])
def test_oracle_dequant_matches_reference_cpu_formula(oracle_mod, n, k, p):
    from tris_moe_amd import synthetic

    rng = synthetic.rng_for(n * k)
    sal = synthetic.salient_columns(rng, rng.random(k) + 0.5, math.ceil(0.05 * k))
    ex = synthetic.make_expert(rng, n, k, p, sal)
    ours = oracle_mod.dequant_compact3(ex["qweight1"], ex["qweight2_sparse"], ex["qweight2_sparse_prefix"],
                                       ex["gmap_dense"], ex["c_map"], ex["g_idx"], ex["col_pack3"], ex["row_pack3"], k)
    ref = _reference_cpu_dequant(oracle_mod, ex, ex["gmap_dense"], n, k)
    np.testing.assert_array_equal(ours.astype(np.float32), ref.astype(np.float32))  # +0 == -0
    assert np.isfinite(ours.astype(np.float32)).all()


def test_oracle_dequant_group_selection(oracle_mod):
    """Non-uniform g_idx uses g_idx[k] per column; the uniform fast path uses the 64-column tile's
    first group; an out-of-range group gives zero weights (kernel.cu:830-853)."""
    from tris_moe_amd import synthetic

    rng = synthetic.rng_for(77)
    n, k = 64, 128
    sal = synthetic.salient_columns(rng, rng.random(k), 7)
    ex = synthetic.make_expert(rng, n, k, 0.2, sal)
    args = (ex["qweight1"], ex["qweight2_sparse"], ex["qweight2_sparse_prefix"], ex["gmap_dense"], ex["c_map"])
    g_perm = (np.arange(k) * 7 % 2).astype(np.int32)          # alternating groups 0/1 within tiles
    per_k = oracle_mod.dequant_compact3(*args, g_perm, ex["col_pack3"], ex["row_pack3"], k, False)
    tile = oracle_mod.dequant_compact3(*args, g_perm, ex["col_pack3"], ex["row_pack3"], k, True)
    only0 = oracle_mod.dequant_compact3(*args, np.zeros(k, np.int32), ex["col_pack3"], ex["row_pack3"], k)
    only1 = oracle_mod.dequant_compact3(*args, np.ones(k, np.int32), ex["col_pack3"], ex["row_pack3"], k)
    sel = g_perm.astype(bool)
    np.testing.assert_array_equal(per_k[:, sel], only1[:, sel])
    np.testing.assert_array_equal(per_k[:, ~sel], only0[:, ~sel])
    np.testing.assert_array_equal(tile, only0)               # both tiles start with group 0
    bad = g_perm.copy()
    bad[5] = 9
    w_bad = oracle_mod.dequant_compact3(*args, bad, ex["col_pack3"], ex["row_pack3"], k)
    assert np.all(w_bad[:, 5].astype(np.float32) == 0)


@pytest.mark.parametrize("t,k,e", [(1, 2, 8), (7, 3, 5), (16, 8, 64), (0, 2, 4)])
def test_oracle_route_brute_force(oracle_mod, t, k, e):
    rng = np.random.default_rng(t * 100 + k * 10 + e)
    sel = np.stack([rng.choice(e, size=k, replace=False) for _ in range(t)]) if t else np.zeros((0, k), np.int64)
    route = oracle_mod.build_route(sel, e, 4)
    flat = sel.reshape(-1)
    active = sorted(set(flat.tolist()))
    assert route["expert_ids"].tolist() == active
    seg = route["segment_offsets"]
    for s, ex in enumerate(active):
        rows = route["perm"][seg[s]:seg[s + 1]]
        assert sorted(rows.tolist()) == [i for i in range(flat.size) if flat[i] == ex]
        assert list(rows) == sorted(rows)                      # stable within a segment
    assert route["problem_offsets"].tolist() == [0] + list(np.cumsum([(int(np.sum(flat == ex)) + 3) // 4 for ex in active]))
    np.testing.assert_array_equal(route["grouped_token_indices"] * k + route["grouped_slots"], route["perm"])


@pytest.mark.parametrize("t,k,e,renorm", [(5, 2, 8, True), (9, 8, 64, True), (4, 3, 16, False), (3, 1, 4, True)])
def test_oracle_route_topk_against_float64(oracle_mod, t, k, e, renorm):
    """softmax -> top-k -> renormalisation (modeling_mixtral.py:548-551): selection equals a brute-force
    descending order of the float64 softmax with ties to the lower expert id; weights equal the float64
    values to fp32 precision."""
    rng = np.random.default_rng(t * 1000 + k * 10 + e)
    logits = rng.standard_normal((t, e)).astype(np.float32)
    logits[0, : min(e, 3)] = 1.5                      # exact ties at the top
    w, sel = oracle_mod.route_topk(logits, k, renorm)
    p64 = np.exp(logits.astype(np.float64) - logits.max(axis=1, keepdims=True))
    p64 /= p64.sum(axis=1, keepdims=True)
    for i in range(t):
        order = sorted(range(e), key=lambda j: (-p64[i, j], j))[:k]
        assert sel[i].tolist() == order
        want = p64[i, order] / (p64[i, order].sum() if renorm else 1.0)
        np.testing.assert_allclose(w[i], want, rtol=3e-6)


def test_oracle_layer_against_float64(oracle_mod, tris):
    """The oracle layer (fp16 between stages, fp32 accumulation) stays within the layer tolerance of a
    float64 evaluation of the same exact weights."""
    from tris_moe_amd.configs import MoELayerSpec

    spec = MoELayerSpec("tiny", hidden=256, num_experts=4, intermediate=384, top_k=2, rank=128, tokens=(5,))
    syn = tris["synthetic"]
    layer = syn.make_layer(spec, 5, oracle_mod.gr_encode)
    inp = syn.make_inputs(spec, 5, 6, layer["outlier_idx"])
    w, sel = oracle_mod.route_topk(inp["router_logits"], spec.top_k, spec.renormalize)
    x16 = inp["x"].astype(np.float16)
    out = oracle_mod.moe_layer(x16, w, sel, {p: layer[p] for p in ("gate", "up", "down")}, layer["backbones"],
                               spec.num_experts)
    # float64 reference: same fp16 weights and inputs, no intermediate rounding
    sv = {p: layer["backbones"][p].astype(np.float64) for p in ("gate", "up", "down")}
    ref = np.zeros((5, spec.hidden))
    w16 = w.astype(np.float16).astype(np.float64)
    for t in range(5):
        for s in range(spec.top_k):
            e = int(sel[t, s])
            Wg = oracle_mod.dequant_grouped_expert(layer["gate"], e).astype(np.float64)
            Wu = oracle_mod.dequant_grouped_expert(layer["up"], e).astype(np.float64)
            Wd = oracle_mod.dequant_grouped_expert(layer["down"], e).astype(np.float64)
            xv = x16[t].astype(np.float64)
            g = Wg @ (sv["gate"] @ xv)
            u = Wu @ (sv["up"] @ xv)
            m = g / (1 + np.exp(-g)) * u
            ref[t] += w16[t, s] * (Wd @ (sv["down"] @ m))
    err = out - ref
    assert np.abs(err).max() < 2e-2
    assert np.linalg.norm(err) / np.linalg.norm(ref) < 1e-3


def _float64_layer(oracle_mod, layer, x16, w, sel, spec):
    """The layer in float64 from the same exact fp16 weights, with no intermediate rounding."""
    sv = {p: layer["backbones"][p].astype(np.float64) for p in ("gate", "up", "down")}
    t_count = x16.shape[0]
    ref = np.zeros((t_count, spec.hidden))
    w16 = w.astype(np.float16).astype(np.float64)
    for t in range(t_count):
        for s in range(spec.top_k):
            e = int(sel[t, s])
            Wg = oracle_mod.dequant_grouped_expert(layer["gate"], e).astype(np.float64)
            Wu = oracle_mod.dequant_grouped_expert(layer["up"], e).astype(np.float64)
            Wd = oracle_mod.dequant_grouped_expert(layer["down"], e).astype(np.float64)
            xv = x16[t].astype(np.float64)
            g = Wg @ (sv["gate"] @ xv)
            u = Wu @ (sv["up"] @ xv)
            m = g / (1 + np.exp(-g)) * u
            ref[t] += w16[t, s] * (Wd @ (sv["down"] @ m))
    return ref


def _float64_shared(x, shared_expert):
    """down(silu(gate x) * up x) in float64 from the fp16 weights."""
    wg, wu, wd = (np.asarray(m, dtype=np.float64) for m in shared_expert)
    g = x @ wg.T
    u = x @ wu.T
    return ((g / (1 + np.exp(-g))) * u) @ wd.T


def _within_layer_tolerance(out, ref, rel_l2=1e-3) -> bool:
    err = out - ref
    return bool(np.abs(err).max() < 2e-2 and np.linalg.norm(err) / np.linalg.norm(ref) < rel_l2)


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_oracle_layer_shared_expert_against_float64(oracle_mod, tris, dtype):
    """The oracle's shared-expert branch (the Qwen blocks' shared expert, modeling_qwen2_moe.py:815-818 and
    modeling_qwen3_5_moe.py:186-188) against a float64 evaluation: y = routed + sigmoid(h . w_g) * down(silu(gate
    h) * up h), with no intermediate rounding, and ungated y = routed + shared.  The gated branch rounds every
    tensor to the model dtype as the reference does, so the bound is the dtype's: rel-L2 1e-3 for fp16, 5e-3 for
    bf16 (bf16's own rounding of a value is ~1.6e-3 rel-L2).  Planted slips fail the same check by two orders
    of magnitude: the shared expert's gate and up swapped, the gate dropped (ungated), the gate applied to the
    routed part instead, and the gate's sigmoid left out.  The rounding order itself is pinned bit for bit by
    the reference's expression run by torch (test_oracle_shared_expert_combination_is_the_reference_expression)."""
    from tris_moe_amd.configs import MoELayerSpec

    spec = MoELayerSpec("tiny", hidden=256, num_experts=4, intermediate=384, top_k=2, rank=128, tokens=(5,),
                        shared_expert_intermediate=192)
    syn = tris["synthetic"]
    layer = syn.make_layer(spec, 21, oracle_mod.gr_encode)
    assert layer["shared_expert_gate"].shape == (spec.hidden,)
    inp = syn.make_inputs(spec, 5, 22, layer["outlier_idx"])
    w, sel = oracle_mod.route_topk(inp["router_logits"], spec.top_k, spec.renormalize)
    x16 = inp["x"].astype(np.float16)
    pl = {p: layer[p] for p in ("gate", "up", "down")}
    shared = layer["shared_expert"]
    wgate = layer["shared_expert_gate"]
    xm = inp["x"] if dtype == "bf16" else x16.astype(np.float32)   # the block input in the model dtype
    routed = _float64_layer(oracle_mod, layer, x16, w, sel, spec)
    s64 = _float64_shared(x16.astype(np.float64), shared)
    g64 = 1.0 / (1.0 + np.exp(-(xm.astype(np.float64) @ wgate.astype(np.float64))))[:, None]
    assert 0.05 < g64.min() and g64.max() < 0.95            # the gate matters on this data
    assert np.linalg.norm(s64) > 0.3 * np.linalg.norm(routed)  # and so does the shared expert
    tol = 5e-3 if dtype == "bf16" else 1e-3

    def layer_out(sh, gate):
        return oracle_mod.moe_layer(x16, w, sel, pl, layer["backbones"], spec.num_experts, sh, shared_gate=gate,
                                    x_model=xm, out_dtype=dtype)

    gated_ref = routed + g64 * s64
    assert _within_layer_tolerance(layer_out(shared, wgate), gated_ref, tol)
    assert _within_layer_tolerance(layer_out(shared, None), routed + s64)
    # planted slips
    assert not _within_layer_tolerance(layer_out((shared[1], shared[0], shared[2]), wgate), gated_ref, tol)
    assert not _within_layer_tolerance(layer_out(shared, None), gated_ref, tol)
    assert not _within_layer_tolerance(g64 * routed + s64, gated_ref, tol)
    logit_only = routed + (xm.astype(np.float64) @ wgate.astype(np.float64))[:, None] * s64
    assert not _within_layer_tolerance(logit_only, gated_ref, tol)
    # the shared MLP reads the fp16 cast of the input, its own gate/up/down in that order
    assert np.array_equal(oracle_mod.shared_expert_mlp(x16, shared), oracle_mod.linear_f16(
        (oracle_mod.silu_f16(oracle_mod.linear_f16(x16, shared[0])).astype(np.float32)
         * oracle_mod.linear_f16(x16, shared[1]).astype(np.float32)).astype(np.float16), shared[2]))


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_oracle_shared_expert_combination_is_the_reference_expression(oracle_mod, tris, dtype):
    """The gated join's rounding order: the reference's own lines (modeling_qwen2_moe.py:816-818)
        shared_expert_output = shared_expert(h).to(dt); final = final + gate.to(dt) * shared_expert_output
    executed by torch on the CPU in the model dtype, from the oracle's routed sum (rounded to dt as the
    reference's index_add result is held), its fp16 shared output and its gate, give the oracle's output bits
    after the caller's rounding."""
    from tris_moe_amd.configs import MoELayerSpec

    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    spec = MoELayerSpec("tiny", hidden=256, num_experts=4, intermediate=384, top_k=2, rank=128, tokens=(7,),
                        shared_expert_intermediate=192)
    syn = tris["synthetic"]
    layer = syn.make_layer(spec, 31, oracle_mod.gr_encode)
    inp = syn.make_inputs(spec, 7, 32, layer["outlier_idx"])
    w, sel = oracle_mod.route_topk(inp["router_logits"], spec.top_k, spec.renormalize)
    x16 = inp["x"].astype(np.float16)
    xm = inp["x"] if dtype == "bf16" else x16.astype(np.float32)
    pl = {p: layer[p] for p in ("gate", "up", "down")}
    routed = oracle_mod.moe_layer(x16, w, sel, pl, layer["backbones"], spec.num_experts)
    got = oracle_mod.round_dtype(oracle_mod.moe_layer(
        x16, w, sel, pl, layer["backbones"], spec.num_experts, layer["shared_expert"],
        shared_gate=layer["shared_expert_gate"], x_model=xm, out_dtype=dtype), dtype)
    final = torch.from_numpy(routed).to(tdt)
    shared_expert_output = torch.from_numpy(oracle_mod.shared_expert_mlp(x16, layer["shared_expert"])).to(tdt)
    gate = torch.from_numpy(oracle_mod.shared_expert_gate(xm, layer["shared_expert_gate"], dtype)).to(tdt)
    want = (final + gate * shared_expert_output).float().numpy()
    np.testing.assert_array_equal(got, want)
    # a slip in the order (the product kept in fp32, one rounding at the end) changes bits on this data
    slip = (final.float() + gate.float() * shared_expert_output.float()).to(tdt).float().numpy()
    assert not np.array_equal(slip, want)


def test_oracle_shared_expert_gate_rounding(oracle_mod):
    """shared_expert_gate's roundings against torch's CPU bf16/fp16 evaluation of the same module
    (sigmoid(F.linear(h, w)).to(dt)): one rounding of the exact dot product, then the sigmoid rounded to dt."""
    import torch.nn.functional as F

    rng = np.random.default_rng(5)
    for dt, tdt in (("bf16", torch.bfloat16), ("fp16", torch.float16)):
        h = rng.standard_normal((64, 96)).astype(np.float32)
        w = (rng.standard_normal(96) * 0.2).astype(np.float32)
        ht = torch.from_numpy(h).to(tdt)
        wt = torch.from_numpy(w).to(tdt)
        h_v, w_v = ht.float().numpy(), wt.float().numpy()
        got = oracle_mod.shared_expert_gate(h_v, w_v, dt)
        # torch's CPU linear over bf16/fp16 sums in fp32 (an order that can differ from the exact sum by an
        # fp32 ulp): compare through the same exact-sum rounding, then check the sigmoid stage on its output
        logit = F.linear(ht.double(), wt.double().reshape(1, -1)).to(tdt)
        want = torch.sigmoid(logit.float()).to(tdt).float().numpy()
        np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_oracle_router_logits_against_torch_linear(oracle_mod, dtype):
    """oracle.router_logits against torch's own CPU nn.Linear in the model dtype (self.gate(hidden_states),
    modeling_mixtral.py:546), which sums in fp32 and rounds once: equal except where an fp32 summation order
    decides a rounding tie (at most 0.2 % of the logits, each then one ulp apart); a plausible slip (the
    weight's rows misread as columns of a transposed layout, i.e. x . w for the wrong expert) is far off."""
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    rng = np.random.default_rng(11)
    x = torch.from_numpy(rng.standard_normal((64, 512)).astype(np.float32)).to(tdt)
    w = torch.from_numpy((rng.standard_normal((16, 512)) * 0.05).astype(np.float32)).to(tdt)
    got = oracle_mod.router_logits(x.float().numpy(), w.float().numpy(), dtype)
    lin = torch.nn.Linear(512, 16, bias=False, dtype=tdt)
    lin.weight.data = w
    with torch.no_grad():
        want = lin(x).float().numpy()
    eq = got == want
    assert eq.mean() > 0.998
    rel_ulp = 2.0 ** (-7 if dtype == "bf16" else -10)  # one ulp is at most the larger |v| * 2^-(mantissa bits)
    assert np.all(np.abs(got - want) <= np.maximum(np.abs(got), np.abs(want)) * rel_ulp)
    assert got.dtype == np.float32 and np.array_equal(oracle_mod.round_dtype(got, dtype), got)
    slip = oracle_mod.router_logits(x.float().numpy(), np.roll(w.float().numpy(), 1, axis=0), dtype)
    assert np.abs(slip - want).max() > 0.1


def test_oracle_grouped_forward_epilogue_is_the_composition(oracle_mod, tris):
    """oracle.grouped_forward's output scale and bias epilogue (TriSMoE_cuda_kernel.cu:4662-4680; the sparse
    form's kernels scale unconditionally, :4051-4064) against torch on the CPU: per segment,
    fp16(F.linear(hidden, W_e) * scale_e + bias_e) in fp32, zeros for a negative expert slot.  Experts carry
    distinct scales and biases over three segments; three plausible slips give other bits on this data: the
    bias added before the scale, one expert's scale used for every segment, and the bias left out."""
    import torch.nn.functional as F

    rng = np.random.default_rng(7)
    ext = tris["ext"]
    E, n, k = 3, 96, 128
    col_norm = rng.random(k).astype(np.float32) + 0.5
    proj = dict(tris["synthetic"].make_projection(rng, E, n, k, 0.15, col_norm, ext.gr_encode, keep_dense_gmap=True))
    proj["output_scale"] = (rng.random((E, n)) * 2 + 0.25).astype(np.float16)
    proj["bias"] = rng.standard_normal((E, n)).astype(np.float16)
    proj["has_output_scale"] = True
    proj["has_bias"] = True
    hidden = (rng.standard_normal((11, k)) * 2).astype(np.float16)
    eids = np.asarray([2, 0, -1, 1], dtype=np.int32)
    seg = np.asarray([0, 4, 7, 8, 11], dtype=np.int32)
    got = oracle_mod.grouped_forward(proj, hidden, eids, seg)

    def composition(bias_first=False, one_scale=False, no_bias=False):
        out = torch.zeros((11, n), dtype=torch.float16)
        for s, e in enumerate(eids.tolist()):
            lo, hi = int(seg[s]), int(seg[s + 1])
            if e < 0:
                continue
            wt = torch.from_numpy(oracle_mod.dequant_grouped_expert(proj, e)).double()
            acc = F.linear(torch.from_numpy(hidden[lo:hi]).double(), wt).float()
            sc = torch.from_numpy(proj["output_scale"][0 if one_scale else e]).float()
            bi = torch.from_numpy(proj["bias"][e]).float()
            if no_bias:
                acc = acc * sc
            elif bias_first:
                acc = (acc + bi) * sc
            else:
                acc = acc * sc + bi
            out[lo:hi] = acc.half()
        return out.numpy()

    want = composition()
    np.testing.assert_array_equal(got, want)
    assert not np.any(got[7:8])                                   # the negative slot's rows are zero
    for slip in (dict(bias_first=True), dict(one_scale=True), dict(no_bias=True)):
        assert not np.array_equal(composition(**slip), want), slip
    # scale only, and bias only
    only_scale = dict(proj, has_bias=False)
    ws = oracle_mod.grouped_forward(only_scale, hidden, eids, seg)
    np.testing.assert_array_equal(ws, composition(no_bias=True))
    wb = oracle_mod.grouped_forward(dict(proj, has_output_scale=False), hidden, eids, seg)
    plain = oracle_mod.grouped_forward(dict(proj, has_output_scale=False, has_bias=False), hidden, eids, seg)
    for s, e in enumerate(eids.tolist()):
        lo, hi = int(seg[s]), int(seg[s + 1])
        if e < 0:
            continue
        acc = F.linear(torch.from_numpy(hidden[lo:hi]).double(),
                       torch.from_numpy(oracle_mod.dequant_grouped_expert(proj, e)).double()).float()
        np.testing.assert_array_equal(wb[lo:hi], (acc + torch.from_numpy(proj["bias"][e]).float()).half().numpy())
        np.testing.assert_array_equal(plain[lo:hi], acc.half().numpy())
    # the sparse form scales unconditionally (TriSMoE_cuda_kernel.cu:4051-4064): a sparse payload without the
    # has_output_scale flag still applies the scale
    from gr_cases import to_sparse

    sparse = to_sparse(oracle_mod, proj, k)
    sparse["has_output_scale"] = False
    sparse["has_bias"] = False
    np.testing.assert_array_equal(oracle_mod.grouped_forward(sparse, hidden, eids, seg), composition(no_bias=True))


def test_oracle_layer_input_scales(oracle_mod, tris):
    """The oracle's ns_mode == 1 backbone input scales (qlinear_cuda.py:4477-4480): unit scales change nothing;
    power-of-two scales (exact fp16 products) give the bits of the layer whose backbone columns carry the same
    factors, so the scale sits on the input columns of the named projection; a scale on up instead of gate
    changes the output."""
    from tris_moe_amd.configs import MoELayerSpec

    spec = MoELayerSpec("tiny", hidden=256, num_experts=4, intermediate=384, top_k=2, rank=128, tokens=(5,))
    syn = tris["synthetic"]
    layer = syn.make_layer(spec, 9, oracle_mod.gr_encode)
    inp = syn.make_inputs(spec, 5, 10, layer["outlier_idx"])
    w, sel = oracle_mod.route_topk(inp["router_logits"], spec.top_k, spec.renormalize)
    x16 = inp["x"].astype(np.float16)
    pl = {p: layer[p] for p in ("gate", "up", "down")}
    bb = layer["backbones"]
    plain = oracle_mod.moe_layer(x16, w, sel, pl, bb, spec.num_experts)
    ones = {"gate": np.ones(spec.hidden, np.float16), "down": np.ones(spec.intermediate, np.float16)}
    assert np.array_equal(oracle_mod.moe_layer(x16, w, sel, pl, bb, spec.num_experts, input_scales=ones), plain)
    rng = np.random.default_rng(3)
    p2 = {"gate": np.exp2(rng.integers(-2, 3, spec.hidden)).astype(np.float16),
          "down": np.exp2(rng.integers(-2, 3, spec.intermediate)).astype(np.float16)}
    scaled = oracle_mod.moe_layer(x16, w, sel, pl, bb, spec.num_experts, input_scales=p2)
    bb2 = dict(bb, gate=(bb["gate"] * p2["gate"][None, :]).astype(np.float16),
               down=(bb["down"] * p2["down"][None, :]).astype(np.float16))
    assert np.array_equal(scaled, oracle_mod.moe_layer(x16, w, sel, pl, bb2, spec.num_experts))
    assert not np.array_equal(scaled, plain)
    on_up = oracle_mod.moe_layer(x16, w, sel, pl, bb, spec.num_experts, input_scales={"up": p2["gate"]})
    assert not np.array_equal(on_up, oracle_mod.moe_layer(x16, w, sel, pl, bb, spec.num_experts,
                                                           input_scales={"gate": p2["gate"]}))


def test_shared_expert_stack_conditions_and_layout():
    """SharedExpertStack (the A3B shared expert's weights under the routed backbones, run as extra columns of the
    routed launches): built for fp16 backbones without input scales whose down input width is the shared
    intermediate; the stacks hold the routed rows first, then the shared expert's, unchanged."""
    import torch

    from tris_moe_amd import moe

    H, rank, rank_d, inter = 64, 32, 16, 48
    g = torch.Generator().manual_seed(5)
    mk = lambda *s: torch.randn(*s, generator=g).to(torch.float16)
    backbones = {"gate": mk(rank, H), "up": mk(rank, H), "down": mk(rank_d, inter)}
    shared = (mk(inter, H), mk(inter, H), mk(H, inter))
    assert moe.SharedExpertStack.ok(backbones, shared)
    assert moe.SharedExpertStack.ok(backbones, shared + (mk(1, H).to(torch.bfloat16),))
    st = moe.SharedExpertStack(backbones, shared)
    assert (st.split_gu, st.split_d) == (rank, rank_d)
    assert torch.equal(st.gate[:rank], backbones["gate"]) and torch.equal(st.gate[rank:], shared[0])
    assert torch.equal(st.up[:rank], backbones["up"]) and torch.equal(st.up[rank:], shared[1])
    assert torch.equal(st.down[:rank_d], backbones["down"]) and torch.equal(st.down[rank_d:], shared[2])
    assert tuple(st.down.shape) == (rank_d + H, inter)
    # a shared intermediate other than the routed one (the down input widths differ), input scales, other dtypes
    assert not moe.SharedExpertStack.ok({**backbones, "down": mk(rank_d, inter + 16)}, shared)
    assert not moe.SharedExpertStack.ok({**backbones, "gate_in_scale": mk(H)}, shared)
    assert not moe.SharedExpertStack.ok(backbones, (shared[0].float(), shared[1], shared[2]))
    assert not moe.SharedExpertStack.ok(backbones, None)
