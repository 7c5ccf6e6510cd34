"""Matrix-mode null-space compensation (grouped C1_e . (C2_e . x) per routed row, qlinear_cuda.py:1734-2336):
the payload layout on the host against the oracle's slicing, and on the GPU the kernels and a Mixtral layer
with gate/up/down compensation against the oracle."""
import numpy as np
import pytest
import torch

from tris_moe_amd import qlinear, synthetic
from tris_moe_amd.packing import pack_4bit


def _blocks(rng, ranks, infeatures, outfeatures, gs):
    c2 = [None if r == 0 else pack_4bit(rng.standard_normal((r, infeatures)).astype(np.float32) * 0.05, gs)
          for r in ranks]
    c1 = [None if r == 0 else pack_4bit(rng.standard_normal((outfeatures, r)).astype(np.float32) * 0.05, min(r, gs))
          for r in ranks]
    return c2, c1


@pytest.mark.parametrize("ranks,gs", [([8, 0, 24, 16], 64), ([40, 3, 0], 16), ([0, 0], 32)])
def test_payload_layout_round_trip(oracle_mod, ranks, gs):
    """build_grouped_ns_payload concatenates per-expert blocks so that the oracle's per-expert slices
    (offsets, word offsets, C1 groups of min(rank, group_size)) dequantise to each expert's own matrices."""
    rng = np.random.default_rng(len(ranks) + gs)
    infeatures, outfeatures = 200, 72
    c2, c1 = _blocks(rng, ranks, infeatures, outfeatures, gs)
    ns = qlinear.build_grouped_ns_payload(c2, c1, infeatures, outfeatures, gs)
    assert ns["max_ns_rank"] == max(ranks) and ns["ns_rank_per_expert"].tolist() == ranks
    for e, r in enumerate(ranks):
        m = oracle_mod.ns_expert_matrices(ns, e)
        if r == 0:
            assert m is None
            continue
        w2 = oracle_mod.packed4_dequant(c2[e]["qweight"], c2[e]["qzeros"], c2[e]["scales"], c2[e]["g_idx"], r,
                                        infeatures)
        w1 = oracle_mod.packed4_dequant(c1[e]["qweight"], c1[e]["qzeros"], c1[e]["scales"], c1[e]["g_idx"],
                                        outfeatures, r)
        np.testing.assert_array_equal(m[0], w2)
        np.testing.assert_array_equal(m[1], w1)


def test_shared_c2_blocks(oracle_mod):
    """Experts with one C2 key share its block (one copy, equal offsets), each with its own C1."""
    rng = np.random.default_rng(2)
    ns = synthetic.make_ns_payload(rng, 4, 128, 64, [16, 16, 8, 16], group_size=32, share_c2=True)
    off = ns["ns_c2_rank_offsets"].tolist()
    assert off[0] == off[1] == off[3] != off[2]
    assert ns["ns_c2_qweight"].shape[1] == 16 + 8
    m0, m1 = oracle_mod.ns_expert_matrices(ns, 0), oracle_mod.ns_expert_matrices(ns, 1)
    np.testing.assert_array_equal(m0[0], m1[0])
    assert not np.array_equal(m0[1], m1[1])


def test_oracle_is_the_reference_fallback(oracle_mod):
    """oracle.ns_compensation against the reference's own fallback, F.linear(F.linear(x_seg, c2), c1) on fp16
    tensors (qlinear_cuda.py:1943-1946), run by torch on the CPU per segment: bit-identical, including
    a segment with no expert and a rank-0 expert.  The same data without the fp16 rounding of the hidden
    row (a plausible slip) does not match, so the check sees that rounding."""
    import torch.nn.functional as F

    rng = np.random.default_rng(3)
    ns = synthetic.make_ns_payload(rng, 4, 96, 40, [8, 0, 24, 5], group_size=32, magnitude=0.05)
    ids = np.asarray([2, 0, 3, -1, 1], np.int32)
    offs = np.concatenate([[0], np.cumsum([6, 3, 4, 2, 3])]).astype(np.int32)
    x = (rng.standard_normal((18, 96)) * 1.5).astype(np.float16)
    got = oracle_mod.ns_compensation(x, ns, ids, offs)
    want = np.zeros_like(got)
    unrounded = np.zeros_like(got)
    for s, e in enumerate(ids):
        lo, hi = int(offs[s]), int(offs[s + 1])
        m = oracle_mod.ns_expert_matrices(ns, int(e)) if 0 <= e < 4 else None
        if m is None:
            continue
        c2, c1 = (torch.from_numpy(a) for a in m)
        want[lo:hi] = F.linear(F.linear(torch.from_numpy(x[lo:hi]), c2), c1).numpy()
        h32 = F.linear(torch.from_numpy(x[lo:hi]).float(), c2.float())
        unrounded[lo:hi] = F.linear(h32, c1.float()).half().numpy()
    np.testing.assert_array_equal(got, want)
    assert not np.array_equal(unrounded, want)


def test_oracle_c1_is_the_second_half(oracle_mod):
    """oracle.ns_c1 on the hidden fp16(C2_e . x) of each row gives ns_compensation(x) bit for bit, whatever the
    hidden holds past each expert's rank (large values there: reading them would show)."""
    rng = np.random.default_rng(9)
    ns = synthetic.make_ns_payload(rng, 4, 64, 48, [8, 0, 24, 5], group_size=16, magnitude=0.05)
    ids = np.asarray([3, 1, 0, -1, 2], np.int32)
    offs = np.concatenate([[0], np.cumsum([2, 3, 6, 1, 4])]).astype(np.int32)
    x = (rng.standard_normal((16, 64)) * 1.5).astype(np.float16)
    hidden = np.full((16, int(ns["max_ns_rank"])), 300.0, np.float16)
    for s, e in enumerate(ids):
        lo, hi = int(offs[s]), int(offs[s + 1])
        m = oracle_mod.ns_expert_matrices(ns, int(e)) if 0 <= e < 4 else None
        if m is not None:
            hidden[lo:hi, :m[0].shape[0]] = oracle_mod.linear_f16(x[lo:hi], m[0])
    np.testing.assert_array_equal(oracle_mod.ns_c1(hidden, ns, ids, offs), oracle_mod.ns_compensation(x, ns, ids, offs))


def test_out_of_range_slices_are_rejected():
    rng = np.random.default_rng(4)
    ns = synthetic.make_ns_payload(rng, 3, 64, 32, [8, 16, 8], group_size=32)
    qlinear.validate_ns_payload(ns)
    bad = dict(ns, ns_c2_rank_offsets=ns["ns_c2_rank_offsets"] + np.asarray([0, 0, 20], np.int32))
    with pytest.raises(ValueError, match="expert 2"):
        qlinear.validate_ns_payload(bad)
    bad = dict(ns, ns_c1_group_offsets=ns["ns_c1_group_offsets"] + np.asarray([0, 9, 0], np.int32))
    with pytest.raises(ValueError, match="expert 1"):
        qlinear.validate_ns_payload(bad)


def test_chain_mismatch_is_rejected():
    rng = np.random.default_rng(3)
    c2, c1 = _blocks(rng, [8], 64, 32, 32)
    c1[0] = pack_4bit(np.zeros((32, 16), np.float32), 16)
    with pytest.raises(ValueError, match="do not chain"):
        qlinear.build_grouped_ns_payload(c2, c1, 64, 32, 32)


# ------------------------------------------------------------------------------------------------ GPU
def _dev_ns(ns, dev):
    return qlinear.ns_payload_to_device(ns, dev)


@pytest.mark.gpu
@pytest.mark.parametrize("accumulate,infeatures,outfeatures,group_size", [
    (False, 512, 320, 128), (True, 512, 320, 128), (True, 1000, 200, 128), (False, 14336, 264, 128),
    (True, 512, 320, 20)])
def test_compensation_kernel_matches_oracle(tris, oracle_mod, cuda, accumulate, infeatures, outfeatures, group_size):
    """Ragged segments, an empty segment, a segment routed to no expert, a rank-0 expert and a rank above
    one C2 workgroup (64): comp (or out + comp) within tolerance of the oracle, untouched rows exact.  The
    input widths split C2 into 2 slices of 256 columns, 4 slices (the last 232 columns: a partial chunk) and 14
    slices of 1024 columns (4 passes each, the next one's loads issued before the current one's
    products).  Group size 20 puts group boundaries inside packed words of C2 and
    (ranks 24 and 72) of C1: the scale and zero point are taken per element there."""
    from test_gpu_parity import assert_close, note

    note(f"ns compensation accumulate={accumulate} in={infeatures} out={outfeatures} gs={group_size}")
    ext = tris["ext"]
    rng = np.random.default_rng(7)
    E = 5
    ns = synthetic.make_ns_payload(rng, E, infeatures, outfeatures, [16, 0, 72, 8, 24], group_size=group_size,
                                   magnitude=0.05)
    ids = np.asarray([2, 0, 1, -1, 4, 3], np.int32)
    lens = [37, 5, 9, 4, 0, 17]
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    R = int(offs[-1])
    x = (rng.standard_normal((R, infeatures)) * 1.5).astype(np.float16)
    base = (rng.standard_normal((R, outfeatures))).astype(np.float16)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    dns = _dev_ns(ns, cuda)
    out = t(base).clone()
    ext.ns_compensation_apply_(out, t(x), t(ids), t(offs), dns, accumulate=accumulate)
    comp = oracle_mod.ns_compensation(x, ns, ids, offs)
    want = oracle_mod.f16_add(base, comp) if accumulate else comp
    got = out.cpu().numpy()
    assert_close(got, want, "ns compensation")
    untouched = np.r_[offs[3]:offs[4]]   # the segment with no expert: comp = 0
    if accumulate:
        np.testing.assert_array_equal(got[untouched], base[untouched])
    else:
        assert not got[untouched].any()
    api = ext.grouped_ns_compensation_forward(
        t(x), t(ids), t(offs), t(offs), 0, *[dns[k] for k in ext.NS_PAYLOAD_TENSORS], dns["max_ns_rank"],
        dns["group_size"])
    assert_close(api.cpu().numpy(), comp, "grouped_ns_compensation_forward")


@pytest.mark.gpu
@pytest.mark.parametrize("accumulate", [False, True])
def test_compensation_pair_matches_single_calls(tris, oracle_mod, cuda, accumulate):
    """The gate/up pair launch: payloads of different ranks and output widths (one of them with a rank-0
    expert routed) give the bits of two single calls, within tolerance of the oracle; reading the rows
    through a token index gives the bits of reading a gathered copy."""
    from test_gpu_parity import assert_close, note

    note(f"ns compensation pair accumulate={accumulate}")
    ext = tris["ext"]
    rng = np.random.default_rng(11)
    E, infeatures = 4, 768
    ns_a = synthetic.make_ns_payload(rng, E, infeatures, 384, [8, 40, 0, 16], group_size=128, magnitude=0.05)
    ns_b = synthetic.make_ns_payload(rng, E, infeatures, 640, [96, 8, 24, 0], group_size=128, magnitude=0.05)
    ids = np.asarray([1, 3, 0, 2], np.int32)
    offs = np.concatenate([[0], np.cumsum([3, 21, 1, 6])]).astype(np.int32)
    R = int(offs[-1])
    x = (rng.standard_normal((R, infeatures)) * 1.5).astype(np.float16)
    base_a = rng.standard_normal((R, 384)).astype(np.float16)
    base_b = rng.standard_normal((R, 640)).astype(np.float16)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    da, db = _dev_ns(ns_a, cuda), _dev_ns(ns_b, cuda)
    pa, pb = t(base_a).clone(), t(base_b).clone()
    ext.ns_compensation_pair_apply_(pa, pb, t(x), t(ids), t(offs), da, db, accumulate=accumulate)
    sa, sb = t(base_a).clone(), t(base_b).clone()
    ext.ns_compensation_apply_(sa, t(x), t(ids), t(offs), da, accumulate=accumulate)
    ext.ns_compensation_apply_(sb, t(x), t(ids), t(offs), db, accumulate=accumulate)
    np.testing.assert_array_equal(pa.cpu().numpy(), sa.cpu().numpy())
    np.testing.assert_array_equal(pb.cpu().numpy(), sb.cpu().numpy())
    # the rows read through a token index (the route's grouped_token_indices) instead of a gathered copy
    tok = rng.permutation(np.arange(R) % 11).astype(np.int64)
    xt = (rng.standard_normal((11, infeatures)) * 1.5).astype(np.float16)
    ia, ib = t(base_a).clone(), t(base_b).clone()
    ext.ns_compensation_pair_apply_(ia, ib, t(xt), t(ids), t(offs), da, db, accumulate=accumulate, row_index=t(tok))
    ga, gb = t(base_a).clone(), t(base_b).clone()
    ext.ns_compensation_pair_apply_(ga, gb, t(xt[tok]), t(ids), t(offs), da, db, accumulate=accumulate)
    np.testing.assert_array_equal(ia.cpu().numpy(), ga.cpu().numpy())
    np.testing.assert_array_equal(ib.cpu().numpy(), gb.cpu().numpy())
    for got, ns, base in ((pa, ns_a, base_a), (pb, ns_b, base_b)):
        comp = oracle_mod.ns_compensation(x, ns, ids, offs)
        assert_close(got.cpu().numpy(), oracle_mod.f16_add(base, comp) if accumulate else comp, "ns pair")


@pytest.mark.gpu
@pytest.mark.parametrize("tokens", [2, 16, 160])
def test_layer_with_ns_compensation(tris, oracle_mod, cuda, tokens):
    """A Mixtral-shaped layer (smaller intermediate) with gate/up/down null-space payloads: the fused-SwiGLU
    size (2 tokens), the dual path (16) and multi-tile segments (160) against the oracle layer."""
    from test_gpu_parity import assert_close, note
    from tris_moe_amd.configs import MoELayerSpec

    note(f"layer with ns T={tokens}")
    spec = MoELayerSpec("ns", hidden=1024, num_experts=8, intermediate=1536, top_k=2, rank=256, tokens=(tokens,))
    syn, ql = tris["synthetic"], tris["qlinear"]
    layer = syn.make_layer(spec, 8100 + tokens, tris["ext"].gr_encode)
    inp = syn.make_inputs(spec, tokens, 8101 + tokens, layer["outlier_idx"])
    rng = np.random.default_rng(tokens)
    ranks = rng.integers(0, 48, spec.num_experts)
    ns_host = {"gate": syn.make_ns_payload(rng, 8, spec.hidden, spec.intermediate, ranks, 128, magnitude=0.03),
               "up": syn.make_ns_payload(rng, 8, spec.hidden, spec.intermediate, ranks, 128, magnitude=0.03),
               "down": syn.make_ns_payload(rng, 8, spec.intermediate, spec.hidden, ranks, 128, magnitude=0.03)}
    payloads = {p: ql.payload_to_device(layer[p], cuda) for p in ("gate", "up", "down")}
    for p in ("gate", "up", "down"):
        payloads[f"{p}_ns"] = ql.ns_payload_to_device(ns_host[p], cuda)
    backbones = {p: torch.from_numpy(layer["backbones"][p]).to(cuda) for p in ("gate", "up", "down")}
    block = tris["moe"].TrisSparseMoeBlock(spec.hidden, spec.num_experts, spec.top_k, payloads, backbones,
                                           renormalize=spec.renormalize)
    x = torch.from_numpy(inp["x"]).to(cuda).to(torch.bfloat16)
    out = block.forward_routed(x, torch.from_numpy(inp["router_logits"]).to(cuda)).float().cpu().numpy()
    w, sel = oracle_mod.route_topk(inp["router_logits"], spec.top_k, spec.renormalize)
    want = oracle_mod.moe_layer(inp["x"].astype(np.float16), w, sel, {p: layer[p] for p in ("gate", "up", "down")},
                                layer["backbones"], spec.num_experts, ns_payloads=ns_host)
    without = oracle_mod.moe_layer(inp["x"].astype(np.float16), w, sel, {p: layer[p] for p in ("gate", "up", "down")},
                                   layer["backbones"], spec.num_experts)
    # the compensation moves the output beyond the tolerance, so leaving it out could not pass (larger
    # magnitudes make C1 . C2 dominate the layer and its bf16 rounding)
    assert np.abs(want - without).max() > 0.02
    assert_close(out, oracle_mod.bf16_round(want), f"layer with ns T={tokens}")
    # the exact (in-kernel decode) expert path applies the terms in place instead: same result
    logits = torch.from_numpy(inp["router_logits"]).to(cuda)
    fused = tris["moe"].grouped_moe_forward_from_logits(
        x.to(torch.float16), logits, spec.top_k, spec.renormalize, payloads, backbones, spec.num_experts,
        torch.bfloat16, expert_path="fused").float().cpu().numpy()
    assert_close(fused, oracle_mod.bf16_round(want), f"layer with ns T={tokens} (fused path)")


@pytest.mark.gpu
def test_c1_only_and_runner_mirrors(tris, oracle_mod, cuda):
    """grouped_ns_c1_forward on a given hidden (values past each expert's rank set large: never read), the
    fused-decode binding, and the reference's runner functions run_grouped_ns_compensation_forward /
    run_grouped_ns_c1_forward, against the oracle (rows outside every segment stay zero)."""
    from test_gpu_parity import assert_close, note

    note("ns c1-only and runner mirrors")
    ext, ql = tris["ext"], tris["qlinear"]
    rng = np.random.default_rng(12)
    E, infeatures, outfeatures = 4, 384, 200
    ns = synthetic.make_ns_payload(rng, E, infeatures, outfeatures, [8, 40, 0, 16], group_size=32, magnitude=0.05)
    ids = np.asarray([1, 3, 0, 2], np.int32)
    offs = np.concatenate([[0], np.cumsum([5, 0, 19, 3])]).astype(np.int32)
    R = int(offs[-1])
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    dns = _dev_ns(ns, cuda)
    hidden = (rng.standard_normal((R, int(ns["max_ns_rank"]))) * 2).astype(np.float16)
    for s, e in enumerate(ids):
        hidden[offs[s]:offs[s + 1], int(ns["ns_rank_per_expert"][e]):] = 1000.0
    got = ext.grouped_ns_c1_forward(t(hidden), t(ids), t(offs), t(offs), 0, dns["ns_rank_per_expert"],
                                    dns["ns_c1_rank_word_offsets"], dns["ns_c1_group_offsets"], dns["ns_c1_qweight"],
                                    dns["ns_c1_qzeros"], dns["ns_c1_scales"], dns["max_ns_rank"], dns["group_size"])
    assert_close(got.cpu().numpy(), oracle_mod.ns_c1(hidden, ns, ids, offs), "grouped_ns_c1_forward")
    x = (rng.standard_normal((R, infeatures)) * 1.5).astype(np.float16)
    comp = oracle_mod.ns_compensation(x, ns, ids, offs)
    args = [dns[k] for k in ext.NS_PAYLOAD_TENSORS] + [dns["max_ns_rank"], dns["group_size"]]
    plain = ext.grouped_ns_compensation_forward(t(x), t(ids), t(offs), t(offs), 0, *args)
    fused = ext.grouped_ns_compensation_fused_decode_forward(t(x), t(ids), t(offs), t(offs), 0, *args)
    assert torch.equal(plain, fused)
    sel =torch.from_numpy(np.repeat(ids, np.diff(offs)).astype(np.int64)).reshape(-1, 1).to(cuda)
    route = ql.build_grouped_route(sel, E)
    order = route["expert_ids"].cpu().numpy()
    # the route lists experts ascending: the same rows regrouped, so compare per expert
    xr = np.concatenate([x[offs[list(ids).index(e)]:offs[list(ids).index(e) + 1]] for e in order])
    hr = np.concatenate([hidden[offs[list(ids).index(e)]:offs[list(ids).index(e) + 1]] for e in order])
    seg = route["segment_offsets"].cpu().numpy()
    comp_r = ql.run_grouped_ns_compensation_forward(dns, t(xr), route)
    assert_close(comp_r.cpu().numpy(), oracle_mod.ns_compensation(xr, ns, order, seg), "run_grouped_ns_compensation_forward")
    c1_r = ql.run_grouped_ns_c1_forward(dns, t(hr), route)
    assert_close(c1_r.cpu().numpy(), oracle_mod.ns_c1(hr, ns, order, seg), "run_grouped_ns_c1_forward")
    assert ql.run_grouped_ns_compensation_forward(dns, t(xr).float(), route) is None   # outside the contract


@pytest.mark.gpu
def test_swiglu_and_combine_take_the_compensation(tris, cuda):
    """The compensated act_fn(g) * u and combine give the bits of the plain kernels on fp16(out + comp),
    the reference's out.add_(compensation) (qlinear_cuda.py:2322-2334) done first; ragged element counts
    and a missing term too."""
    from test_gpu_parity import note

    note("compensated swiglu / combine")
    ext = tris["ext"]
    gen = torch.Generator(device="cpu").manual_seed(5)
    rnd = lambda *s: (torch.randn(*s, generator=gen) * 3).half().to(cuda)
    add = lambda a, b: (a.float() + b.float()).half()
    for shape in ((37, 1536), (5, 1003)):
        g, u, cg, cu = rnd(*shape), rnd(*shape), rnd(*shape), rnd(*shape)
        got = ext.swiglu_mul(g, u, comp_gate=cg, comp_up=cu)
        assert torch.equal(got, ext.swiglu_mul(add(g, cg), add(u, cu)))
        got = ext.swiglu_mul(g, u, comp_gate=None, comp_up=cu)
        assert torch.equal(got, ext.swiglu_mul(g, add(u, cu)))
    tokens, k = 9, 2
    for hidden in (1024, 1001):
        d, c = rnd(tokens * k, hidden), rnd(tokens * k, hidden)
        perm = torch.randperm(tokens * k, generator=gen).to(torch.int32).to(cuda)
        w = torch.rand(tokens, k, generator=gen).half().to(cuda)
        got = ext.moe_combine(d, perm, w, expert_comp=c)
        assert torch.equal(got, ext.moe_combine(add(d, c), perm, w))
