"""The sparse split-bitmap grouped entry (compact3_tris_precomputed_grouped_forward, TriSMoE_cuda.cpp:795-832)
against the oracle: ragged sparse rows, rows of salient columns only, a partial last packed row, output scale
and bias, dropped experts, multi-tile segments; exact weights through one-hot activations; the runner and the
pair runner on sparse payload dicts, and a layer whose payloads are all sparse."""
import sys

import numpy as np
import pytest
import torch

from gr_cases import to_sparse

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
REL_L2 = 1e-3


def note(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def assert_close(got, want, what):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    assert np.isfinite(got).all(), what
    err = got - want
    max_abs = float(np.abs(err).max()) if err.size else 0.0
    denom = float(np.linalg.norm(want))
    rel = float(np.linalg.norm(err)) / denom if denom > 0 else float(np.linalg.norm(err))
    assert max_abs <= MAX_ABS and rel <= REL_L2, f"{what}: max_abs={max_abs:.3g} rel_l2={rel:.3g}"


def make_projection(tris, seed, E, n, k, p=0.15, salient_counts=None, scale=False, bias=False):
    syn = tris["synthetic"]
    rng = syn.rng_for(seed)
    os_ = rng.uniform(0.5, 1.5, (E, n)).astype(np.float16) if scale else None
    bs = (rng.standard_normal((E, n)) * 0.1).astype(np.float16) if bias else None
    return syn.make_projection(rng, E, n, k, p, rng.random(k) + 0.5, tris["ext"].gr_encode,
                               salient_counts=salient_counts, output_scale=os_, bias=bs, keep_dense_gmap=True)


def segments(lengths, drop=None):
    off = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    ids = np.arange(len(lengths), dtype=np.int32)
    if drop is not None:
        ids[drop] = -1
    prob = np.concatenate([[0], np.cumsum([-(-x // 4) for x in lengths])]).astype(np.int32)
    return ids, off, prob


def run_sparse(tris, pl, hidden, ids, off, prob, dev):
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    has_bias = bool(pl["has_bias"])
    bias = pl["bias"] if has_bias else hidden.new_empty((0, 0))
    return tris["ext"].compact3_tris_precomputed_grouped_forward(
        hidden, t(ids), t(off), t(prob), torch.tensor([int(prob[-1])], dtype=torch.int64), pl["qweight1"],
        pl["qweight2_sparse"], pl["qweight2_sparse_prefix"], pl["q_gmap_sparse"], pl["q_gmap_sparse_prefix"],
        pl["c_map"], pl["g_idx"], pl["col_pack3"], pl["row_pack3"], pl["output_scale"], bias, has_bias)


CASES = [
    dict(E=3, n=128, k=256, seg=[5, 0, 3]),
    dict(E=2, n=100, k=96, seg=[17, 2]),                                     # partial output tile, K = 3 rows
    dict(E=4, n=64, k=200, seg=[1, 40, 3, 2], salient_counts=[0, 1, 40, 70]),  # partial last row, ragged sparse rows
    dict(E=3, n=192, k=512, seg=[4, 9, 33], scale=True, bias=True),
    dict(E=3, n=64, k=256, seg=[6, 2, 5], drop=1, scale=True),
    dict(E=2, n=64, k=128, seg=[3, 3], p=0.05),
]


def case_id(c):
    return "-".join(f"{a}{b}" for a, b in c.items() if a not in ("salient_counts", "seg"))


@pytest.mark.parametrize("case", CASES, ids=case_id)
def test_sparse_grouped_forward_matches_oracle(tris, oracle_mod, cuda, case):
    note(f"sparse grouped {case_id(case)}")
    E, n, k = case["E"], case["n"], case["k"]
    host = make_projection(tris, 40 + E + n + k, E, n, k, case.get("p", 0.15), case.get("salient_counts"),
                           case.get("scale", False), case.get("bias", False))
    sp = to_sparse(oracle_mod, host, k)
    if not case.get("scale", False):
        # the sparse kernels always apply the output scale: give it non-unit values here too
        sp["output_scale"] = np.random.default_rng(7).uniform(0.5, 1.5, (E, n)).astype(np.float16)
    pl = tris["qlinear"].payload_to_device(sp, cuda)
    ids, off, prob = segments(case["seg"], case.get("drop"))
    rng = np.random.default_rng(n + k)
    hidden = rng.standard_normal((int(off[-1]), k)).astype(np.float16)
    got = run_sparse(tris, pl, torch.from_numpy(hidden).to(cuda), ids, off, prob, cuda).cpu().numpy()
    want = oracle_mod.grouped_forward(sp, hidden, ids, off)
    assert_close(got.astype(np.float32), want.astype(np.float32), "sparse grouped forward")
    if case.get("drop") is not None:
        d = case["drop"]
        assert not got[off[d]:off[d + 1]].any()


def test_sparse_weights_exact_through_one_hot(tris, oracle_mod, cuda):
    """hidden rows that are unit vectors read single weights: with a unit output scale the outputs are the
    oracle's dequantised fp16 weights bit for bit."""
    note("sparse one-hot")
    E, n, k = 2, 64, 96
    host = make_projection(tris, 5, E, n, k, salient_counts=[3, 33])
    sp = to_sparse(oracle_mod, host, k)
    sp["output_scale"] = np.ones((E, n), dtype=np.float16)
    pl = tris["qlinear"].payload_to_device(sp, cuda)
    ids, off, prob = segments([k, k])
    hidden = np.zeros((2 * k, k), dtype=np.float16)
    hidden[np.arange(2 * k), np.arange(2 * k) % k] = 1.0
    got = run_sparse(tris, pl, torch.from_numpy(hidden).to(cuda), ids, off, prob, cuda).cpu().numpy()
    for e in range(E):
        w = oracle_mod.dequant_grouped_expert(sp, e)  # [N, K]
        np.testing.assert_array_equal(got[e * k:(e + 1) * k].view(np.uint16), w.T.view(np.uint16))


def test_sparse_equals_block_gr_entry(tris, oracle_mod, cuda):
    """The same weights through the block-GR entry (with the same output scale) give the same bits."""
    note("sparse vs block-GR")
    E, n, k = 3, 128, 256
    host = make_projection(tris, 9, E, n, k, scale=True)
    sp = to_sparse(oracle_mod, host, k)
    pl_s = tris["qlinear"].payload_to_device(sp, cuda)
    pl_g = tris["qlinear"].payload_to_device({kk: v for kk, v in host.items() if kk != "gmap_dense"}, cuda)
    ids, off, prob = segments([7, 20, 1])
    hidden = torch.from_numpy(np.random.default_rng(2).standard_normal((28, k)).astype(np.float16)).to(cuda)
    got_s = run_sparse(tris, pl_s, hidden, ids, off, prob, cuda)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    got_g = tris["ext"].compact3_tris_precomputed_grouped_forward_block_gr(
        hidden, t(ids), t(off), t(prob), torch.tensor([int(prob[-1])], dtype=torch.int64), pl_g["qweight1"],
        pl_g["qweight2_sparse"], pl_g["qweight2_sparse_prefix"], pl_g["q_gmap_gr_words"], pl_g["q_gmap_gr_offsets"],
        pl_g["q_gmap_gr_meta"], pl_g["c_map"], pl_g["g_idx"], pl_g["col_pack3"], pl_g["row_pack3"],
        pl_g["output_scale"], True, hidden.new_empty((0, 0)), False, False)
    assert torch.equal(got_s, got_g)


def test_sparse_runners_match_oracle(tris, oracle_mod, cuda):
    """run_grouped_structured_expert_forward and the pair runner on sparse payload dicts (the pair takes one
    launch per projection, qlinear_cuda.py:2381-2411)."""
    note("sparse runners")
    q = tris["qlinear"]
    E, n, k = 4, 96, 128
    host_a = make_projection(tris, 13, E, n, k, bias=True)
    host_b = make_projection(tris, 14, E, n, k)
    sa, sb = to_sparse(oracle_mod, host_a, k), to_sparse(oracle_mod, host_b, k)
    pa, pb = q.payload_to_device(sa, cuda), q.payload_to_device(sb, cuda)
    sel = torch.tensor([[0, 2], [3, 2], [1, 0], [2, 3], [0, 1]], dtype=torch.int64, device=cuda)
    route = q.build_grouped_route(sel, E)
    R = sel.numel()
    rng = np.random.default_rng(4)
    ha = rng.standard_normal((R, k)).astype(np.float16)
    hb = rng.standard_normal((R, k)).astype(np.float16)
    x = torch.zeros((R, 8), dtype=torch.float16, device=cuda)
    out = q.run_grouped_structured_expert_forward(pa, torch.from_numpy(ha).to(cuda), x, route)
    assert out is not None
    ids = route["expert_ids"].cpu().numpy()
    off = route["segment_offsets"].cpu().numpy()
    assert_close(out.cpu().numpy().astype(np.float32), oracle_mod.grouped_forward(sa, ha, ids, off).astype(np.float32),
                 "sparse runner")
    oa, ob = q.run_grouped_structured_expert_pair_forward(pa, pb, torch.from_numpy(ha).to(cuda),
                                                          torch.from_numpy(hb).to(cuda), x, route)
    assert oa is not None and ob is not None
    assert_close(oa.cpu().numpy().astype(np.float32), oracle_mod.grouped_forward(sa, ha, ids, off).astype(np.float32),
                 "sparse pair a")
    assert_close(ob.cpu().numpy().astype(np.float32), oracle_mod.grouped_forward(sb, hb, ids, off).astype(np.float32),
                 "sparse pair b")


def test_sparse_layer_matches_oracle(tris, oracle_mod, cuda):
    """A whole MoE layer whose three projections are sparse-form payloads."""
    note("sparse layer")
    from tris_moe_amd.configs import MoELayerSpec

    syn, q, moe = tris["synthetic"], tris["qlinear"], tris["moe"]
    spec = MoELayerSpec("sparse", hidden=512, num_experts=8, intermediate=768, top_k=2, rank=256, tokens=(6,))
    layer = syn.make_layer(spec, 17, tris["ext"].gr_encode, keep_dense_gmap=True)
    sparse = {p: to_sparse(oracle_mod, layer[p], spec.rank) for p in ("gate", "up", "down")}
    payloads = {p: q.payload_to_device(sparse[p], cuda) for p in sparse}
    backbones = {p: torch.from_numpy(layer["backbones"][p]).to(cuda) for p in ("gate", "up", "down")}
    inp = syn.make_inputs(spec, 6, 3, layer["outlier_idx"])
    x16 = torch.from_numpy(inp["x"]).to(cuda).to(torch.bfloat16).to(torch.float16)
    out = moe.grouped_moe_forward_from_logits(x16, torch.from_numpy(inp["router_logits"]).to(cuda), spec.top_k,
                                              spec.renormalize, payloads, backbones, spec.num_experts)
    w, sel = oracle_mod.route_topk(inp["router_logits"], spec.top_k, spec.renormalize)
    ref = oracle_mod.bf16_round(oracle_mod.moe_layer(inp["x"].astype(np.float16), w, sel, sparse,
                                                     layer["backbones"], spec.num_experts))
    assert_close(out.float().cpu().numpy(), ref, "sparse layer")
