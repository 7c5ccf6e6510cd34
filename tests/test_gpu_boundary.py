"""The reference's Python boundary on the GPU against the oracle: QuantLinear.forward / compute_shared_hidden /
forward_from_precomputed_hidden (qlinear_cuda.py:4451-4566), build_grouped_precomputed_payload over expert
modules (:1512-1636), run_grouped_structured_expert[_pair]_forward (:2131-2634) and
TrisSparseMoeBlock.forward on bf16 activations (modeling_mixtral.py:539-608)."""
import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

from tris_moe_amd.configs import MoELayerSpec

TINY = MoELayerSpec("tiny", hidden=256, num_experts=4, intermediate=384, top_k=2, rank=128, tokens=(6,))
EXPERT_KEYS = ("qweight1", "qweight2_sparse", "qweight2_sparse_prefix", "c_map", "g_idx", "col_pack3", "row_pack3")


def note(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def assert_close(got, want, what):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    err = got - want
    max_abs = float(np.abs(err).max())
    rel = float(np.linalg.norm(err) / np.linalg.norm(want))
    assert max_abs <= 2e-2 and rel <= 1e-3, f"{what}: max_abs={max_abs:.3g} rel_l2={rel:.3g}"


def expert_tensors(payload, e):
    """One expert's packed tensors from a stacked host payload (its own qweight2_sparse rows and GR words)."""
    t = {k: np.ascontiguousarray(payload[k][e]) for k in EXPERT_KEYS}
    nsal = int(payload["qweight2_sparse_prefix"][e][-1])
    t["qweight2_sparse"] = np.ascontiguousarray(payload["qweight2_sparse"][e][: (nsal + 31) // 32])
    offs = payload["q_gmap_gr_offsets"][e]
    t["q_gmap_gr_words"] = np.ascontiguousarray(payload["q_gmap_gr_words"][e][: int(offs[-1])])
    t["q_gmap_gr_offsets"] = np.ascontiguousarray(offs)
    t["q_gmap_gr_meta"] = np.ascontiguousarray(payload["q_gmap_gr_meta"][e])
    return t


def modules_of(tris, payload, sv, infeatures, cuda, input_scale=None):
    ql = tris["qlinear"]
    shared = ql.ExpertSharedMatrix(torch.from_numpy(sv).to(cuda))
    n, rank = int(payload["qweight1"].shape[2]), int(payload["g_idx"].shape[1])
    scale = None if input_scale is None else torch.from_numpy(input_scale).to(cuda)
    mods = []
    for e in range(int(payload["qweight1"].shape[0])):
        m = ql.QuantLinear(infeatures, n, rank, shared, expert_input_scale=scale)
        m.load_expert_payload(expert_tensors(payload, e))
        mods.append(m.to(cuda))
    return mods


@pytest.fixture(scope="module")
def tiny_layer(tris):
    return tris["synthetic"].make_layer(TINY, 1234, tris["ext"].gr_encode)


@pytest.mark.parametrize("scaled", [False, True])
def test_quantlinear_forward_matches_oracle(tris, oracle_mod, cuda, tiny_layer, scaled):
    """QuantLinear.forward(x) = forward_from_precomputed_hidden(compute_shared_hidden(x), x): the shared fp16
    backbone (with the ns_mode 1 input scale when set) then the expert's compact3 matrix, for every expert."""
    note(f"QuantLinear.forward scaled={scaled}")
    rng = np.random.default_rng(21)
    pg, sv = tiny_layer["gate"], tiny_layer["backbones"]["gate"]
    scale = rng.uniform(0.5, 1.5, TINY.hidden).astype(np.float16) if scaled else None
    mods = modules_of(tris, pg, sv, TINY.hidden, cuda, scale)
    x = rng.standard_normal((2, 5, TINY.hidden)).astype(np.float16)
    xt = torch.from_numpy(x).to(cuda)
    x2 = x.reshape(-1, TINY.hidden)
    hid_want = oracle_mod.linear_f16(oracle_mod.f16_mul(x2, scale[None, :]) if scaled else x2, sv)
    for e, m in enumerate(mods):
        assert m.can_precompute_shared()
        hid = m.compute_shared_hidden(xt)
        assert tuple(hid.shape) == (2, 5, TINY.rank)
        assert_close(hid.reshape(-1, TINY.rank).cpu().numpy(), hid_want, f"shared hidden e={e}")
        out = m.forward(xt)
        assert tuple(out.shape) == (2, 5, TINY.intermediate)
        # the oracle on the module's own fp16 hidden (the GEMM alone), and end to end from x
        want = oracle_mod.grouped_forward(pg, hid.reshape(-1, TINY.rank).cpu().numpy(), [e], [0, 10])
        assert_close(out.reshape(-1, TINY.intermediate).cpu().numpy(), want, f"forward e={e}")
        want_x = oracle_mod.grouped_forward(pg, hid_want, [e], [0, 10])
        assert_close(out.reshape(-1, TINY.intermediate).cpu().numpy(), want_x, f"forward from x e={e}")
        again = m.forward_from_precomputed_hidden(hid, xt)
        assert torch.equal(again, out)


def test_payload_from_modules_stacks_the_reference_layout(tris, oracle_mod, cuda, tiny_layer):
    """build_grouped_precomputed_payload(modules) reproduces the stacked payload (ragged qweight2_sparse and GR
    words zero-padded) bit for bit, and the grouped runner on the module list matches the oracle."""
    note("payload from modules")
    ql = tris["qlinear"]
    pd = tiny_layer["down"]
    mods = modules_of(tris, pd, tiny_layer["backbones"]["down"], TINY.intermediate, cuda)
    pay = ql.build_grouped_precomputed_payload(mods, cuda, torch.float16)
    for k in EXPERT_KEYS + ("q_gmap_gr_offsets", "q_gmap_gr_meta"):
        np.testing.assert_array_equal(pay[k].cpu().numpy(), pd[k], err_msg=k)
    width = max(int(o[-1]) for o in pd["q_gmap_gr_offsets"])
    assert int(pay["q_gmap_gr_words"].shape[1]) == width
    np.testing.assert_array_equal(pay["q_gmap_gr_words"].cpu().numpy(), pd["q_gmap_gr_words"][:, :width])
    assert pay["has_output_scale"] is False and pay["has_bias"] is False
    rng = np.random.default_rng(22)
    lengths = [3, 0, 5, 2]
    R = sum(lengths)
    hid = rng.standard_normal((R, TINY.rank)).astype(np.float16)
    x = rng.standard_normal((R, TINY.intermediate)).astype(np.float16)
    out = ql.run_grouped_structured_expert_forward(mods, torch.from_numpy(hid).to(cuda), torch.from_numpy(x).to(cuda),
                                                   lengths)
    ids = [e for e in range(4) if lengths[e] > 0]
    seg = np.concatenate([[0], np.cumsum([lengths[e] for e in ids])])
    want = oracle_mod.grouped_forward(pd, hid, ids, seg)
    assert_close(out.cpu().numpy(), want, "module-list grouped forward")


@pytest.mark.parametrize("rows_per_expert,source", [(2, "dict"), (40, "dict"), (3, "modules")])
def test_pair_forward_matches_oracle(tris, oracle_mod, cuda, tiny_layer, rows_per_expert, source):
    """run_grouped_structured_expert_pair_forward: gate and up over one route (the in-kernel-decode pair at
    decode sizes, predecode + MFMA pair for long segments), from payload dicts or module lists."""
    note(f"pair forward rows={rows_per_expert} source={source}")
    ql = tris["qlinear"]
    pg, pu = tiny_layer["gate"], tiny_layer["up"]
    if source == "dict":
        a = ql.payload_to_device(pg, cuda)
        b = ql.payload_to_device(pu, cuda)
    else:
        a = modules_of(tris, pg, tiny_layer["backbones"]["gate"], TINY.hidden, cuda)
        b = modules_of(tris, pu, tiny_layer["backbones"]["up"], TINY.hidden, cuda)
    rng = np.random.default_rng(23 + rows_per_expert)
    T = rows_per_expert * TINY.num_experts // TINY.top_k
    sel = np.stack([rng.choice(TINY.num_experts, TINY.top_k, replace=False) for _ in range(T)]).astype(np.int64)
    route = ql.build_grouped_route(torch.from_numpy(sel).to(cuda), TINY.num_experts)
    R = T * TINY.top_k
    ha = rng.standard_normal((R, TINY.rank)).astype(np.float16)
    hb = rng.standard_normal((R, TINY.rank)).astype(np.float16)
    x = rng.standard_normal((R, TINY.hidden)).astype(np.float16)
    oa, ob = ql.run_grouped_structured_expert_pair_forward(
        a, b, torch.from_numpy(ha).to(cuda), torch.from_numpy(hb).to(cuda), torch.from_numpy(x).to(cuda), route)
    assert oa is not None and ob is not None
    ids = route["expert_ids"].cpu().numpy()
    seg = route["segment_offsets"].cpu().numpy()
    assert_close(oa.cpu().numpy(), oracle_mod.grouped_forward(pg, ha, ids, seg), "pair gate")
    assert_close(ob.cpu().numpy(), oracle_mod.grouped_forward(pu, hb, ids, seg), "pair up")


@pytest.mark.parametrize("batch,seq", [(1, 1), (2, 4)])
def test_sparse_moe_block_forward_bf16(tris, oracle_mod, cuda, batch, seq):
    """TrisSparseMoeBlock.forward on bf16 [B, S, H] hidden states with a bf16 router (the reference block's
    dtypes): the output keeps the input shape and dtype, the router logits are the bf16 linear's (the fused
    router launch: the oracle's rounding of the exact sum, and torch's Linear, up to rare one-ulp ties), and the
    output matches the oracle layer fed those logits (single-token calls: four of them, scored together)."""
    from tris_moe_amd.configs import C1_MIXTRAL_DECODE as SPEC

    note(f"TrisSparseMoeBlock.forward bf16 B={batch} S={seq}")
    syn, ql = tris["synthetic"], tris["qlinear"]
    layer = syn.make_layer(SPEC, 5100, tris["ext"].gr_encode)
    payloads = {p: ql.payload_to_device(layer[p], cuda) for p in ("gate", "up", "down")}
    backbones = {p: torch.from_numpy(layer["backbones"][p]).to(cuda) for p in ("gate", "up", "down")}
    rng = np.random.default_rng(24)
    router = torch.from_numpy((rng.standard_normal((SPEC.num_experts, SPEC.hidden)) * 0.02).astype(np.float32))
    block = tris["moe"].TrisSparseMoeBlock(SPEC.hidden, SPEC.num_experts, SPEC.top_k, payloads, backbones,
                                           router_weight=router.to(cuda)).to(cuda)
    caches = {"gate": {}, "up": {}, "down": {}}
    gots, wants = [], []
    for call in range(4 if batch * seq == 1 else 1):
        inp = syn.make_inputs(SPEC, batch * seq, 25 + call, layer["outlier_idx"])
        h = torch.from_numpy(inp["x"]).to(cuda).to(torch.bfloat16).reshape(batch, seq, SPEC.hidden)
        with torch.no_grad():
            out, logits = block(h)
            want_logits = torch.nn.functional.linear(h.reshape(-1, SPEC.hidden), block.gate.weight)
        assert out.dtype == torch.bfloat16 and tuple(out.shape) == (batch, seq, SPEC.hidden)
        assert logits.dtype == torch.bfloat16 and tuple(logits.shape) == (batch * seq, SPEC.num_experts)
        lg, wl = logits.float().cpu().numpy(), want_logits.float().cpu().numpy()
        exact = oracle_mod.router_logits(h.reshape(-1, SPEC.hidden).float().cpu().numpy(),
                                         block.gate.weight.detach().float().cpu().numpy(), "bf16")
        for ref in (exact, wl):
            assert np.all(np.abs(lg - ref) <= np.maximum(np.abs(lg), np.abs(ref)) * 2.0 ** -7), "beyond one ulp"
        assert (lg == exact).mean() >= 0.99
        x16 = h.reshape(-1, SPEC.hidden).float().cpu().numpy().astype(np.float16)
        w, sel = oracle_mod.route_topk(logits.float().cpu().numpy(), SPEC.top_k, SPEC.renormalize)
        wants.append(oracle_mod.bf16_round(oracle_mod.moe_layer(
            x16, w, sel, {p: layer[p] for p in ("gate", "up", "down")}, layer["backbones"], SPEC.num_experts,
            weight_caches=caches)))
        gots.append(out.reshape(-1, SPEC.hidden).float().cpu().numpy())
    assert_close(np.concatenate(gots), np.concatenate(wants), "block forward")
