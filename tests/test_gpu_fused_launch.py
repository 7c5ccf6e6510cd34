"""Launches that carry independent work of the decode step together, against the separate calls they
replace: the router with the gate/up backbones of the same tokens (tris_route_topk_backbone), the backbone's
split-K slice reduction inside the predecode launch (tris_grouped_block_gr_predecode_multi_reduce), and the
predecoded dual / SwiGLU GEMMs gathering their activation rows through a row index (the *_rows entries, on
the decode kernel and on the weight-stationary prefill kernel).  Each gives the bits of the calls it
replaces; the gathered GEMMs are also checked against the oracle."""
import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
REL_L2 = 1e-3
ROUTE_KEYS = ("perm", "grouped_token_indices", "grouped_slots", "grouped_expert_ids", "expert_ids", "segment_offsets",
              "problem_offsets", "counts", "inverse_perm", "routing_weights_f16", "routing_weights",
              "selected_experts")
NAMES = ("qweight1", "qweight2_sparse", "qweight2_sparse_prefix", "c_map", "g_idx", "col_pack3", "row_pack3")


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


def t_i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(dev)


def make_projection(tris, seed, E, n, k, p=0.15):
    syn = tris["synthetic"]
    rng = syn.rng_for(seed)
    return syn.make_projection(rng, E, n, k, p, rng.random(k) + 0.5, tris["ext"].gr_encode)


def backbone_inputs(seed, tokens, in_f, rank, scales, dev):
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.standard_normal((tokens, in_f)).astype(np.float16)).to(dev)
    sv_a = torch.from_numpy((rng.standard_normal((rank, in_f)) * 0.05).astype(np.float16)).to(dev)
    sv_b = torch.from_numpy((rng.standard_normal((rank, in_f)) * 0.05).astype(np.float16)).to(dev)
    sa = sb = None
    if scales:
        sa = torch.from_numpy(rng.uniform(0.5, 1.5, in_f).astype(np.float16)).to(dev)
        sb = torch.from_numpy(rng.uniform(0.5, 1.5, in_f).astype(np.float16)).to(dev)
    return x, sv_a, sv_b, sa, sb


ROUTE_BB_CASES = [
    # tokens, experts, top_k, renormalize, in_features, rank, input scales
    (1, 8, 2, True, 4096, 512, False),     # Mixtral decode: one-wavefront router, 8 slices
    (16, 8, 2, True, 4096, 512, True),     # with ns_mode 1 input scales
    (16, 64, 8, False, 2048, 256, False),  # workgroup router, one expert a lane
    (20, 60, 4, True, 1024, 128, False),   # two token tiles per backbone workgroup
    (40, 256, 8, True, 520, 64, True),     # three token tiles, four experts a lane
    (64, 128, 8, True, 4096, 512, False),  # four token tiles: the merged launch's token limit
    (7, 16, 3, True, 100, 64, False),      # columns not a multiple of 8 (element loads)
    (5, 8, 2, True, 128, 128, False),      # one slice: the outputs are written in the launch itself
]


@pytest.mark.parametrize("case", ROUTE_BB_CASES, ids=lambda c: "T{}E{}k{}in{}r{}".format(c[0], c[1], c[2], c[4], c[5]))
def test_route_topk_backbone_matches_separate_launches(tris, cuda, case):
    t, e, k, renorm, in_f, rank, scales = case
    note(f"route+backbone T={t} E={e} k={k} in={in_f} rank={rank}")
    ext = tris["ext"]
    rng = np.random.default_rng(t * 7 + e)
    logits = torch.from_numpy(rng.standard_normal((t, e)).astype(np.float32)).to(cuda)
    x, sv_a, sv_b, sa, sb = backbone_inputs(t + in_f, t, in_f, rank, scales, cuda)
    want_route = ext.route_topk_grouped(logits, k, renorm, 4)
    want_a, want_b = ext.backbone_linear_pair(x, sv_a, sv_b, in_scale_a=sa, in_scale_b=sb)
    assert ext.route_topk_backbone_ok(x, sv_a, sv_b, sa, sb)
    route, pending = ext.route_topk_backbone_pair(logits, k, renorm, 4, x, sv_a, sv_b, in_scale_a=sa, in_scale_b=sb)
    got_a, got_b = ext.finish_backbone(pending)
    for key in ROUTE_KEYS:
        assert torch.equal(route[key], want_route[key]), key
    assert torch.equal(got_a, want_a) and torch.equal(got_b, want_b)


def test_route_topk_backbone_rejects_what_it_cannot_run(tris, cuda):
    note("route+backbone limits")
    ext = tris["ext"]
    x, sv_a, sv_b, _, _ = backbone_inputs(3, 65, 256, 64, False, cuda)
    assert not ext.route_topk_backbone_ok(x, sv_a, sv_b)  # more tokens than the merged launch takes
    logits = torch.zeros((65, 8), dtype=torch.float32, device=cuda)
    with pytest.raises(RuntimeError):
        ext.route_topk_backbone_pair(logits, 2, True, 4, x, sv_a, sv_b)
    x2, sa2, sb2, _, _ = backbone_inputs(4, 4, 256, 64, False, cuda)
    assert not ext.route_topk_backbone_ok(x2, sa2, sb2[:, :128])  # shapes differ


@pytest.mark.parametrize("tokens", [1, 16])
def test_predecode_with_backbone_reduction(tris, oracle_mod, cuda, tokens):
    """The predecode launch that also reduces a deferred backbone: the decoded bitmaps are the plain
    predecode's and the backbone outputs tris_backbone_linear_pair's."""
    note(f"predecode + backbone reduction T={tokens}")
    ext = tris["ext"]
    E, n, k = 4, 320, 256
    payloads = [make_projection(tris, 71 + i, E, n, k) for i in range(2)]
    dev_p = [tris["qlinear"].payload_to_device(p, cuda) for p in payloads]
    eid = t_i32(np.asarray([2, 0, -1], dtype=np.int32), cuda)  # a padded (inactive) slot
    nblk = tris["synthetic"].packing.num_gr_blocks(k, n)

    def jobs():
        out = []
        for d in dev_p:
            buf = torch.full((3, nblk, 128), -7, dtype=torch.int32, device=cuda)
            out.append((buf, d["q_gmap_gr_words"], d["q_gmap_gr_offsets"], d["q_gmap_gr_meta"], k // 32, n))
        return out

    want_dec = ext.grouped_block_gr_predecode_multi(jobs(), eid)
    rng = np.random.default_rng(tokens)
    logits = torch.from_numpy(rng.standard_normal((tokens, 8)).astype(np.float32)).to(cuda)
    x, sv_a, sv_b, sa, sb = backbone_inputs(tokens, tokens, 4096, 512, True, cuda)
    want_a, want_b = ext.backbone_linear_pair(x, sv_a, sv_b, in_scale_a=sa, in_scale_b=sb)
    _, pending = ext.route_topk_backbone_pair(logits, 2, True, 4, x, sv_a, sv_b, in_scale_a=sa, in_scale_b=sb)
    got_dec = ext.grouped_block_gr_predecode_multi(jobs(), eid, backbone=pending)
    for g, w in zip(got_dec, want_dec):
        assert torch.equal(g[:2], w[:2])
    assert torch.equal(pending.out_a, want_a) and torch.equal(pending.out_b, want_b)
    # the decoded bitmaps are the oracle's
    p0 = payloads[0]
    want0 = oracle_mod.gr_predecode(p0["q_gmap_gr_words"], p0["q_gmap_gr_offsets"], p0["q_gmap_gr_meta"],
                                    np.asarray([2, 0], dtype=np.int32), nblk)
    np.testing.assert_array_equal(got_dec[0][:2].cpu().numpy(), want0)


def gathered_inputs(rng, tokens, rows, k, dev):
    ha = (rng.standard_normal((tokens, k)) * 1.5).astype(np.float16)
    hb = (rng.standard_normal((tokens, k)) * 1.5).astype(np.float16)
    ridx = rng.integers(0, tokens, rows).astype(np.int64)
    ridx[min(3, rows - 1)] = -1      # indices outside [0, tokens) read zero rows
    ridx[rows // 2] = tokens
    valid = (ridx >= 0) & (ridx < tokens)
    ga = np.where(valid[:, None], ha[np.clip(ridx, 0, tokens - 1)], np.float16(0))
    gb = np.where(valid[:, None], hb[np.clip(ridx, 0, tokens - 1)], np.float16(0))
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    return to(ha), to(hb), to(ridx), to(ga), to(gb), ga, gb


@pytest.mark.parametrize("lengths", [[2, 37, 0, 5], [300, 0, 200, 90]], ids=["decode", "prefill-ws"])
def test_gathered_predecoded_gemms_match_materialised_rows(tris, oracle_mod, cuda, lengths):
    """Grouped row r reads hidden[row_index[r]]: the dual and SwiGLU outputs equal the calls on the
    materialised rows bit for bit (on the decode kernel, and on the weight-stationary kernel for long
    segments), and the oracle's within tolerance."""
    note(f"gathered dual/swiglu segments={lengths}")
    ext = tris["ext"]
    E, n, k = 4, 320, 256
    pa, pb = make_projection(tris, 81, E, n, k), make_projection(tris, 82, E, n, k)
    da, db = (tris["qlinear"].payload_to_device(p, cuda) for p in (pa, pb))
    ids = np.asarray([e for e in range(E) if lengths[e] > 0], dtype=np.int32)
    offs = np.concatenate([[0], np.cumsum([lengths[e] for e in ids])]).astype(np.int32)
    prob = np.concatenate([[0], np.cumsum((np.diff(offs) + 3) // 4)]).astype(np.int32)
    rows = int(offs[-1])
    rng = np.random.default_rng(rows)
    ha, hb, ridx, ga, gb, ga_np, gb_np = gathered_inputs(rng, max(8, rows // 3), rows, k, cuda)
    args = (t_i32(ids, cuda), t_i32(offs, cuda), t_i32(prob, cuda), torch.tensor([int(prob[-1])]))
    nblk = tris["synthetic"].packing.num_gr_blocks(k, n)
    dec = []
    for d in (da, db):
        buf = torch.empty((ids.size, nblk, 128), dtype=torch.int32, device=cuda)
        dec.append(ext.compact3_tris_precomputed_grouped_block_gr_predecode(
            buf, t_i32(ids, cuda), d["q_gmap_gr_words"], d["q_gmap_gr_offsets"], d["q_gmap_gr_meta"], k // 32, n))
    pa_args = [da[x] for x in NAMES]
    pb_args = [db[x] for x in NAMES]
    want = ext.compact3_tris_precomputed_grouped_dual_forward_block_gr_predecoded(
        ga, gb, *args, dec[0], *pa_args, dec[1], *pb_args, True)
    got = ext.compact3_tris_precomputed_grouped_dual_forward_block_gr_predecoded(
        ha, hb, *args, dec[0], *pa_args, dec[1], *pb_args, True, row_index=ridx)
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
    assert_close(got[0].cpu().numpy(), oracle_mod.grouped_forward(pa, ga_np, ids, offs, True), "gathered gate")
    sw_want = ext.compact3_tris_precomputed_grouped_swiglu_forward_block_gr_predecoded(
        ga, gb, *args, dec[0], *pa_args, dec[1], *pb_args)
    sw_got = ext.compact3_tris_precomputed_grouped_swiglu_forward_block_gr_predecoded(
        ha, hb, *args, dec[0], *pa_args, dec[1], *pb_args, row_index=ridx)
    assert torch.equal(sw_got, sw_want)


@pytest.mark.parametrize("tokens", [1, 16, 64])
def test_layer_with_router_backbone_launch_matches_oracle(tris, oracle_mod, cuda, tokens, monkeypatch):
    """The Mixtral-shaped layer from router logits takes the merged launches (router + gate/up backbones,
    predecode + backbone reduction, gathered GEMMs) up to 64 tokens: its output is the oracle's within the
    layer tolerance."""
    from tris_moe_amd.configs import C1_MIXTRAL_DECODE as spec

    note(f"layer router+backbone T={tokens}")
    ext, moe, syn, ql = tris["ext"], tris["moe"], tris["synthetic"], tris["qlinear"]
    calls = []
    merged = ext.route_topk_backbone_pair

    def counting(*a, **kw):
        calls.append(1)
        return merged(*a, **kw)

    monkeypatch.setattr(ext, "route_topk_backbone_pair", counting)
    layer = syn.make_layer(spec, 5000 + tokens, ext.gr_encode)
    payloads = {p: ql.payload_to_device(layer[p], cuda) for p in ("gate", "up", "down")}
    backbones = {p: torch.from_numpy(layer["backbones"][p]).to(cuda) for p in ("gate", "up", "down")}
    caches = {"gate": {}, "up": {}, "down": {}}
    outs, wants = [], []
    for i in range(4 if tokens == 1 else 1):
        inp = syn.make_inputs(spec, tokens, 5001 + tokens + i, layer["outlier_idx"])
        x16 = torch.from_numpy(inp["x"].astype(np.float16)).to(cuda)
        logits = torch.from_numpy(inp["router_logits"]).to(cuda)
        out = moe.grouped_moe_forward_from_logits(x16, logits, spec.top_k, spec.renormalize, payloads, backbones,
                                                  spec.num_experts, torch.bfloat16)
        w, sel = oracle_mod.route_topk(inp["router_logits"], spec.top_k, spec.renormalize)
        want = oracle_mod.moe_layer(inp["x"].astype(np.float16), w, sel, {p: layer[p] for p in ("gate", "up", "down")},
                                    layer["backbones"], spec.num_experts, None, weight_caches=caches)
        outs.append(out.float().cpu().numpy())
        wants.append(oracle_mod.bf16_round(want))
    assert calls, "the layer did not take the router + backbone launch"
    assert_close(np.concatenate(outs), np.concatenate(wants), f"layer T={tokens}")


@pytest.mark.parametrize("rows,scaled", [(1, False), (16, True), (33, False), (64, True), (100, True), (128, False),
                                         (300, True), (600, False)])
def test_backbone_swiglu_product_is_exact(tris, cuda, rows, scaled):
    """With SV the identity, the fused down backbone returns its operand: the product fp16(silu(g) * u)
    (times the input scale) must be swiglu_mul's bits (one product per output, nothing rounds twice).  At 300 rows
    (rank 256) the decode kernel's three row groups form it, at 600 rows the tiled GEMM in its operand staging."""
    note(f"backbone swiglu identity rows={rows} scaled={scaled}")
    ext = tris["ext"]
    n = 256
    rng = np.random.default_rng(rows)
    g = torch.from_numpy((rng.standard_normal((rows, n)) * 3).astype(np.float16)).to(cuda)
    u = torch.from_numpy((rng.standard_normal((rows, n)) * 3).astype(np.float16)).to(cuda)
    sc = torch.from_numpy(rng.uniform(0.5, 1.5, n).astype(np.float16)).to(cuda) if scaled else None
    eye = torch.eye(n, dtype=torch.float16, device=cuda)
    got = ext.backbone_swiglu_linear(g, u, eye, in_scale=sc)
    want = ext.swiglu_mul(g, u)
    if sc is not None:
        want = want * sc  # fp16 product, as the kernel's
    assert torch.equal(got, want)


@pytest.mark.parametrize("rows,in_f,rank", [(32, 14336, 512), (16, 1024, 256), (64, 512, 128), (7, 4096, 64),
                                             (128, 1024, 256), (257, 512, 256), (300, 2048, 256), (512, 512, 192),
                                             (600, 14336, 512), (1000, 1056, 128)])
def test_backbone_swiglu_matches_unfused(tris, cuda, rows, in_f, rank, monkeypatch):
    """The fused down backbone against swiglu_mul followed by backbone_linear (below 512 rows the split over K
    differs, so the fp32 sums agree within rounding; from 512 rows both run the tiled GEMM with the same slices
    and give the same bits) and against an fp32 reference."""
    note(f"backbone swiglu rows={rows} in={in_f} rank={rank}")
    ext = tris["ext"]
    monkeypatch.setattr(ext, "BACKBONE_GEMM_MIN_WORKGROUPS", 1)  # every eligible shape to the tiled GEMMs
    rng = np.random.default_rng(in_f + rows)
    g = torch.from_numpy(rng.standard_normal((rows, in_f)).astype(np.float16)).to(cuda)
    u = torch.from_numpy(rng.standard_normal((rows, in_f)).astype(np.float16)).to(cuda)
    sv = torch.from_numpy((rng.standard_normal((rank, in_f)) * 0.02).astype(np.float16)).to(cuda)
    sc = torch.from_numpy(rng.uniform(0.5, 1.5, in_f).astype(np.float16)).to(cuda)
    # the layer's policy takes the fused form up to 128 rows, up to 512 rows for ranks that are not 512s (the decode
    # kernel's row groups) and, from 512 rows, for ranks of 512s (full-rank GEMM tiles); the C entry takes any rank
    # of 128s above
    assert ext.backbone_swiglu_ok(g, sv, sc) == (rows <= 128 or (rows <= 512 and rank % 512 != 0)
                                                 or (rows >= 512 and rank % 512 == 0))
    got = ext.backbone_swiglu_linear(g, u, sv, in_scale=sc)
    mlp = ext.swiglu_mul(g, u)
    unfused = ext.backbone_linear(mlp, sv, in_scale=sc)
    ref = ((mlp * sc).float() @ sv.float().t()).cpu().numpy()
    assert_close(got.float().cpu().numpy(), ref, "fused vs fp32")
    assert_close(got.float().cpu().numpy(), unfused.float().cpu().numpy(), "fused vs unfused")
    if rows >= ext.BACKBONE_GEMM_MIN_ROWS and (rank % 512 == 0 or rows > ext.SWIGLU_BACKBONE_GROUPED_MAX_ROWS):
        assert torch.equal(got, unfused)  # both on the tiled GEMM
    again = ext.backbone_swiglu_linear(g, u, sv, in_scale=sc)
    assert torch.equal(got, again)  # slices added in fixed order


@pytest.mark.parametrize("tokens,in_f,rank,top_k", [(512, 4096, 512, 2), (1024, 2048, 256, 8), (700, 1056, 128, 3)])
def test_backbone_pair_scatter_matches_token_projection(tris, cuda, tokens, in_f, rank, top_k, monkeypatch):
    """The gate/up backbones written to routed rows: row inverse_perm[t, j] holds the pair's projection of token t
    (the same tiled GEMM over the tokens, so the same bits), slots of -1 write nothing, and the rows equal the
    fp32 product of the gathered rows within rounding."""
    note(f"backbone pair scatter T={tokens} in={in_f} rank={rank} k={top_k}")
    ext = tris["ext"]
    monkeypatch.setattr(ext, "BACKBONE_GEMM_MIN_WORKGROUPS", 1)
    rng = np.random.default_rng(tokens + in_f)
    x = torch.from_numpy(rng.standard_normal((tokens, in_f)).astype(np.float16)).to(cuda)
    sv_a = torch.from_numpy((rng.standard_normal((rank, in_f)) * 0.02).astype(np.float16)).to(cuda)
    sv_b = torch.from_numpy((rng.standard_normal((rank, in_f)) * 0.02).astype(np.float16)).to(cuda)
    sc = torch.from_numpy(rng.uniform(0.5, 1.5, in_f).astype(np.float16)).to(cuda)
    R = tokens * top_k
    inv = rng.permutation(R).astype(np.int32)
    inv[rng.choice(R, 5, replace=False)] = -1  # slots routed nowhere
    assert ext.backbone_scatter_ok(tokens, sv_a, sv_b)
    out_a, out_b = ext.backbone_linear_pair_scatter(x, sv_a, sv_b, torch.from_numpy(inv).to(cuda), top_k, R,
                                                    in_scale_b=sc)
    ta, tb = ext.backbone_linear_pair(x, sv_a, sv_b, in_scale_b=sc)
    slot_token = np.repeat(np.arange(tokens), top_k)
    ok = inv >= 0
    rows = torch.from_numpy(inv[ok].astype(np.int64)).to(cuda)
    toks = torch.from_numpy(slot_token[ok]).to(cuda)
    assert torch.equal(out_a.index_select(0, rows), ta.index_select(0, toks))
    assert torch.equal(out_b.index_select(0, rows), tb.index_select(0, toks))
    ref = ((x * sc).float() @ sv_b.float().t()).index_select(0, toks).cpu().numpy()
    assert_close(out_b.index_select(0, rows).float().cpu().numpy(), ref, "scatter vs fp32")


PROLOGUE_CASES = [
    # tokens, experts, top_k, renormalize, hidden, rank, input scales
    (1, 8, 2, True, 4096, 512, False),     # Mixtral decode
    (16, 8, 2, True, 4096, 512, True),     # with ns_mode 1 input scales
    (32, 8, 2, True, 2048, 256, False),    # 64 routed rows: the one-wavefront route's limit
    (5, 6, 3, False, 1024, 128, False),    # fewer experts, three picks, no renormalisation
    (3, 8, 2, True, 512, 128, False),      # one slice: the backbone writes its outputs in the first launch
]


@pytest.mark.parametrize("case", PROLOGUE_CASES, ids=lambda c: "T{}E{}k{}h{}r{}".format(c[0], c[1], c[2], c[4], c[5]))
def test_router_backbone_and_route_predecode_match_separate_launches(tris, cuda, case):
    """tris_router_backbone (the router Linear, the fp16 cast and the gate/up backbones in one launch) and
    tris_route_predecode_multi_reduce (the route beside the predecode and the backbones' slice reduction) give
    the bits of the launches they replace: tris_router_linear, tris_backbone_linear_pair on x16,
    tris_route_topk_grouped and tris_grouped_block_gr_predecode_multi for its expert ids."""
    t, e, k, renorm, hidden, rank, scales = case
    note(f"router+backbone, route+predecode T={t} E={e} k={k} h={hidden} r={rank}")
    ext = tris["ext"]
    rng = np.random.default_rng(t * 11 + e)
    x = torch.from_numpy(rng.standard_normal((t, hidden)).astype(np.float32)).to(torch.bfloat16).to(cuda)
    w = torch.from_numpy((rng.standard_normal((e, hidden)) / np.sqrt(hidden)).astype(np.float32))
    w = w.to(torch.bfloat16).to(cuda)
    _, sv_a, sv_b, sa, sb = backbone_inputs(t + 100, t, hidden, rank, scales, cuda)
    logits, logits32, x16, pending = ext.router_backbone_pair(x, w, sv_a, sv_b, in_scale_a=sa, in_scale_b=sb)
    want_logits, want32, want_x16 = ext.router_linear(x, w)
    assert torch.equal(logits.view(torch.int16), want_logits.view(torch.int16))
    assert torch.equal(logits32, want32)
    assert torch.equal(x16.view(torch.int16), want_x16.view(torch.int16))
    # two projections (rank x packed rows) with blocks for every expert
    projs = [make_projection(tris, 300 + i, e, n, kk) for i, (n, kk) in enumerate([(256, 128), (192, 256)])]
    pays = [tris["qlinear"].payload_to_device(p, cuda) for p in projs]
    slots = min(e, t * k)
    jobs, bufs = [], []
    for p in pays:
        pr, n = int(p["qweight1"].size(1)), int(p["qweight1"].size(2))
        nblk = ((pr + 1) // 2) * ((n + 63) // 64)
        buf = torch.full((slots, nblk, 128), -7, dtype=torch.int32, device=cuda)
        bufs.append(buf)
        jobs.append((buf, p["q_gmap_gr_words"], p["q_gmap_gr_offsets"], p["q_gmap_gr_meta"], pr, n))
    route = ext.route_predecode_multi(logits32, k, renorm, 4, jobs, backbone=pending)
    want_route = ext.route_topk_grouped(want32, k, renorm, 4)
    for key in ROUTE_KEYS:
        assert torch.equal(route[key], want_route[key]), key
    ref_bufs = [torch.full_like(b, -7) for b in bufs]
    ref_jobs = [(rb,) + j[1:] for rb, j in zip(ref_bufs, jobs)]
    ext.grouped_block_gr_predecode_multi(ref_jobs, want_route["expert_ids"][:slots])
    for b, rb in zip(bufs, ref_bufs):
        assert torch.equal(b, rb)
    want_a, want_b = ext.backbone_linear_pair(want_x16, sv_a, sv_b, in_scale_a=sa, in_scale_b=sb)
    assert torch.equal(pending.out_a.view(torch.int16), want_a.view(torch.int16))
    assert torch.equal(pending.out_b.view(torch.int16), want_b.view(torch.int16))


@pytest.mark.parametrize("path", ["auto", "fused"])
@pytest.mark.parametrize("tokens", [1, 4, 16])
def test_block_decode_step_matches_unfused_block(tris, oracle_mod, cuda, tokens, path):
    """TrisSparseMoeBlock.forward at decode (grouped_moe_decode_step: router Linear + backbones, then route +
    predecode, or with the "fused" expert path route + backbone reduction and the in-kernel-decode GEMMs) against
    the same block with the step's other path (router_linear, then the route, the backbones and the expert path's
    GEMMs): the same output and router logits, bit for bit, on the C1 layer."""
    from tris_moe_amd.configs import C1_MIXTRAL_DECODE as SPEC

    note(f"block decode step T={tokens} path={path}")
    syn, ql, moe = tris["synthetic"], tris["qlinear"], tris["moe"]
    layer = syn.make_layer(SPEC, 6100 + tokens, tris["ext"].gr_encode)
    payloads = {p: ql.payload_to_device(layer[p], cuda) for p in ("gate", "up", "down")}
    backbones = {p: torch.from_numpy(layer["backbones"][p]).to(cuda) for p in ("gate", "up", "down")}
    rng = np.random.default_rng(tokens)
    router = torch.from_numpy((rng.standard_normal((SPEC.num_experts, SPEC.hidden)) * 0.015).astype(np.float32))
    block = moe.TrisSparseMoeBlock(SPEC.hidden, SPEC.num_experts, SPEC.top_k, payloads, backbones,
                                   router_weight=router.to(cuda))
    block.expert_path = path
    inp = syn.make_inputs(SPEC, tokens, 6200 + tokens, layer["outlier_idx"])
    h = torch.from_numpy(inp["x"]).to(cuda).to(torch.bfloat16)
    flat = h.reshape(-1, SPEC.hidden)
    assert moe.decode_prologue_ok(flat, block.gate.weight.detach(), SPEC.top_k, SPEC.num_experts, payloads,
                                  backbones, path)
    with torch.no_grad():
        out, logits = block(h.reshape(1, tokens, SPEC.hidden))
        lg, lg32, x16 = tris["ext"].router_linear(flat, block.gate.weight.detach())
        want = block.forward_routed(flat, lg32, x16=x16)
    assert torch.equal(logits.view(torch.int16), lg.view(torch.int16))
    assert torch.equal(out.reshape(tokens, SPEC.hidden).view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("case", [(16, 8, 2), (3, 8, 2), (5, 6, 3)], ids=lambda c: "T{}E{}k{}".format(*c))
def test_route_predecode_all_experts_matches_separate_launches(tris, cuda, case):
    """tris_route_predecode_all_reduce (decode_all: every expert's bitmaps, slot e for expert e, with the route and
    the backbones' reduction in the same launch) writes tris_route_topk_grouped's route and, in slot e,
    tris_grouped_block_gr_predecode_multi's bitmaps of expert e, also for experts the route leaves idle (T = 3 and
    5 route fewer rows than there are experts)."""
    t, e, k = case
    note(f"route+predecode of every expert T={t} E={e} k={k}")
    ext = tris["ext"]
    rng = np.random.default_rng(t * 13 + e)
    hidden, rank = 512, 256
    x = torch.from_numpy(rng.standard_normal((t, hidden)).astype(np.float32)).to(torch.bfloat16).to(cuda)
    w = torch.from_numpy((rng.standard_normal((e, hidden)) / np.sqrt(hidden)).astype(np.float32))
    w = w.to(torch.bfloat16).to(cuda)
    _, sv_a, sv_b, sa, sb = backbone_inputs(t + 200, t, hidden, rank, False, cuda)
    logits, logits32, x16, pending = ext.router_backbone_pair(x, w, sv_a, sv_b, in_scale_a=sa, in_scale_b=sb)
    projs = [make_projection(tris, 400 + i, e, n, kk) for i, (n, kk) in enumerate([(256, 128), (192, 256)])]
    pays = [tris["qlinear"].payload_to_device(p, cuda) for p in projs]
    jobs, bufs = [], []
    for p in pays:
        pr, n = int(p["qweight1"].size(1)), int(p["qweight1"].size(2))
        nblk = ((pr + 1) // 2) * ((n + 63) // 64)
        buf = torch.full((e, nblk, 128), -7, dtype=torch.int32, device=cuda)
        bufs.append(buf)
        jobs.append((buf, p["q_gmap_gr_words"], p["q_gmap_gr_offsets"], p["q_gmap_gr_meta"], pr, n))
    route = ext.route_predecode_multi(logits32, k, True, 4, jobs, backbone=pending, decode_all=True)
    want_route = ext.route_topk_grouped(logits32, k, True, 4)
    for key in ROUTE_KEYS:
        assert torch.equal(route[key], want_route[key]), key
    ref_bufs = [torch.full_like(b, -7) for b in bufs]
    ext.grouped_block_gr_predecode_multi([(rb,) + j[1:] for rb, j in zip(ref_bufs, jobs)],
                                         torch.arange(e, dtype=torch.int32, device=cuda))
    for b, rb in zip(bufs, ref_bufs):
        assert torch.equal(b, rb)
    want_a, want_b = ext.backbone_linear_pair(x16, sv_a, sv_b, in_scale_a=sa, in_scale_b=sb)
    assert torch.equal(pending.out_a.view(torch.int16), want_a.view(torch.int16))
    assert torch.equal(pending.out_b.view(torch.int16), want_b.view(torch.int16))


@pytest.mark.parametrize("tokens", [4, 16])
def test_block_decode_step_decoding_every_expert_matches_unfused_block(tris, cuda, tokens, monkeypatch):
    """The decode step with every expert's bitmaps decoded (moe.DECODE_ALL_MIN_ROWS_PER_EXPERT lowered to 1, so T = 4
    takes it with 8 routed rows over 8 experts and some experts idle: segment s reads slot expert_ids[s], not s)
    gives the unfused block's output and router logits bit for bit on the C1 layer."""
    from tris_moe_amd.configs import C1_MIXTRAL_DECODE as SPEC

    note(f"block decode step, every expert decoded, T={tokens}")
    syn, ql, moe = tris["synthetic"], tris["qlinear"], tris["moe"]
    monkeypatch.setattr(moe, "DECODE_ALL_MIN_ROWS_PER_EXPERT", 1)
    layer = syn.make_layer(SPEC, 6300 + tokens, tris["ext"].gr_encode)
    payloads = {p: ql.payload_to_device(layer[p], cuda) for p in ("gate", "up", "down")}
    backbones = {p: torch.from_numpy(layer["backbones"][p]).to(cuda) for p in ("gate", "up", "down")}
    rng = np.random.default_rng(tokens + 50)
    router = torch.from_numpy((rng.standard_normal((SPEC.num_experts, SPEC.hidden)) * 0.015).astype(np.float32))
    block = moe.TrisSparseMoeBlock(SPEC.hidden, SPEC.num_experts, SPEC.top_k, payloads, backbones,
                                   router_weight=router.to(cuda))
    inp = syn.make_inputs(SPEC, tokens, 6400 + tokens, layer["outlier_idx"])
    h = torch.from_numpy(inp["x"]).to(cuda).to(torch.bfloat16)
    flat = h.reshape(-1, SPEC.hidden)
    with torch.no_grad():
        lg, lg32, x16 = tris["ext"].router_linear(flat, block.gate.weight.detach())
        # T = 4 routes 8 rows: with this seed some experts are idle, so segments and expert ids differ
        active = torch.unique(torch.topk(lg32, SPEC.top_k, dim=1).indices)
        out, logits = block(h.reshape(1, tokens, SPEC.hidden))
        want = block.forward_routed(flat, lg32, x16=x16)
    if tokens == 4:
        assert int(active.numel()) < SPEC.num_experts, "the case needs an idle expert"
    assert torch.equal(logits.view(torch.int16), lg.view(torch.int16))
    assert torch.equal(out.reshape(tokens, SPEC.hidden).view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("tokens,in_f,rank,split", [(1, 2048, 768, 256), (3, 512, 320, 64), (24, 1024, 272, 144)])
def test_backbone_column_split_matches_whole_projection(tris, cuda, tokens, in_f, rank, split):
    """A gate/up backbone pair with a column split (two stacked projections, as the A3B block runs the routed
    backbones and the shared expert's gate/up) writes the whole projection's columns [0, split) to out and
    [split, rank) to out_hi, bit for bit: launched beside the router and reduced in the predecode launch."""
    note(f"backbone column split T={tokens} in={in_f} rank={rank} split={split}")
    ext = tris["ext"]
    x, sv_a, sv_b, _, _ = backbone_inputs(tokens * 7 + split, tokens, in_f, rank, False, cuda)
    logits = torch.from_numpy(np.random.default_rng(tokens).standard_normal((tokens, 16)).astype(np.float32)).to(cuda)
    hi_a = torch.full((tokens, rank - split), float("nan"), dtype=torch.float16, device=cuda)
    hi_b = torch.full_like(hi_a, float("nan"))
    route, pend = ext.route_topk_backbone_pair(logits, 2, True, 4, x, sv_a, sv_b, split=split, out_a_hi=hi_a,
                                               out_b_hi=hi_b)
    ext.finish_backbone(pend)
    _, whole = ext.route_topk_backbone_pair(logits, 2, True, 4, x, sv_a, sv_b)
    ext.finish_backbone(whole)
    for lo, hi, full in ((pend.out_a, hi_a, whole.out_a), (pend.out_b, hi_b, whole.out_b)):
        assert torch.equal(lo.view(torch.int16), full[:, :split].contiguous().view(torch.int16))
        assert torch.equal(hi.view(torch.int16), full[:, split:].contiguous().view(torch.int16))


@pytest.mark.parametrize("rows,in_f,rank,split", [(9, 512, 2304, 256), (40, 1024, 640, 512), (128, 512, 384, 128),
                                                   (288, 512, 2304, 256)])
def test_backbone_swiglu_column_split_matches_whole_projection(tris, cuda, rows, in_f, rank, split):
    """tris_backbone_swiglu_linear_split (the routed down backbone and the shared expert's down projection as one
    stacked projection) gives tris_backbone_swiglu_linear's columns [0, split) and [split, rank) bit for bit (288
    rows: three row groups of the decode kernel), and rejects a split on the tiled GEMM (513 rows)."""
    note(f"swiglu backbone column split rows={rows} in={in_f} rank={rank} split={split}")
    ext = tris["ext"]
    rng = np.random.default_rng(rows + rank)
    g = torch.from_numpy(rng.standard_normal((rows, in_f)).astype(np.float16)).to(cuda)
    u = torch.from_numpy(rng.standard_normal((rows, in_f)).astype(np.float16)).to(cuda)
    sv = torch.from_numpy((rng.standard_normal((rank, in_f)) * 0.05).astype(np.float16)).to(cuda)
    lo, hi = ext.backbone_swiglu_linear_split(g, u, sv, split)
    whole = ext.backbone_swiglu_linear(g, u, sv)
    assert torch.equal(lo.view(torch.int16), whole[:, :split].contiguous().view(torch.int16))
    assert torch.equal(hi.view(torch.int16), whole[:, split:].contiguous().view(torch.int16))
    big = torch.zeros((ext.SWIGLU_BACKBONE_GROUPED_MAX_ROWS + 1, in_f), dtype=torch.float16, device=cuda)
    with pytest.raises(RuntimeError, match="column split"):
        ext.backbone_swiglu_linear_split(big, big, sv, split)


PARTIAL_CASES = [
    # rows per segment (expert id, rows), in_features, rank, outfeatures, input scale, every expert decoded
    ([(3, 1), (6, 1)], 14336, 512, 256, False, False),   # Mixtral T = 1 down shape: 8 slices, one row a tile
    ([(2, 4)], 4096, 512, 192, True, False),              # four rows in one segment, input scale
    ([(0, 2), (5, 1)], 4096, 128, 128, False, True),      # 32 slices (two load batches), slots by expert id
    ([(1, 2), (4, 1), (7, 1)], 1024, 256, 320, True, True),  # 3 segments, slots by expert id
    ([(5, 1)], 512, 64, 64, False, False),                # 4 slices
]


@pytest.mark.parametrize("case", PARTIAL_CASES,
                         ids=lambda c: "R{}in{}r{}{}".format(sum(n for _, n in c[0]), c[1], c[2], "x" if c[5] else ""))
def test_down_gemm_from_partial_sums_matches_reduced_backbone(tris, cuda, case):
    """tris_backbone_linear_deferred leaves the split-K partial sums and
    tris_grouped_forward_block_gr_predecoded_partials adds them in its staging: the output is the predecoded GEMM's
    over tris_backbone_linear's rows, bit for bit (one and two batches of slices in flight, several rows in one
    segment, slots per segment and per expert)."""
    segs, in_f, rank, n, scaled, by_expert = case
    R = sum(c for _, c in segs)
    E = 8
    note(f"down GEMM from partial sums R={R} in={in_f} rank={rank} N={n} by_expert={by_expert}")
    ext, ql = tris["ext"], tris["qlinear"]
    rng = np.random.default_rng(R * 31 + rank)
    x = torch.from_numpy(rng.standard_normal((R, in_f)).astype(np.float16)).to(cuda)
    sv = torch.from_numpy((rng.standard_normal((rank, in_f)) * 0.02).astype(np.float16)).to(cuda)
    sc = torch.from_numpy(rng.uniform(0.5, 1.5, in_f).astype(np.float16)).to(cuda) if scaled else None
    pay = ql.payload_to_device(make_projection(tris, 900 + rank, E, n, rank), cuda)
    assert ext.partials_gemm_ok(pay)
    eid = t_i32([e for e, _ in segs], cuda)
    offs = np.concatenate([[0], np.cumsum([c for _, c in segs])])
    seg = t_i32(offs, cuda)
    prob = t_i32(np.concatenate([[0], np.cumsum([(c + 15) // 16 for _, c in segs])]), cuda)
    tiles = int(sum((c + 15) // 16 for _, c in segs))
    pr = int(pay["qweight1"].size(1))
    nblk = ((pr + 1) // 2) * ((n + 63) // 64)
    slots = E if by_expert else len(segs)
    dec = torch.full((slots, nblk, 128), -7, dtype=torch.int32, device=cuda)
    ids = torch.arange(E, dtype=torch.int32, device=cuda) if by_expert else eid
    ext.grouped_block_gr_predecode_multi([(dec, pay["q_gmap_gr_words"], pay["q_gmap_gr_offsets"],
                                           pay["q_gmap_gr_meta"], pr, n)], ids)
    pend = ext.backbone_linear_deferred(x, sv, in_scale=sc)
    assert isinstance(pend, ext.BackbonePartials) and pend.slices > 1
    got = torch.full((R, n), float("nan"), dtype=torch.float16, device=cuda)
    ext.grouped_forward_block_gr_predecoded_partials(pend, eid, seg, tiles, dec, *[pay[k] for k in NAMES], True,
                                                     out=got, decoded_by_expert=by_expert)
    hid = ext.backbone_linear(x, sv, in_scale=sc)
    want = torch.full_like(got, float("nan"))
    ext.compact3_tris_precomputed_grouped_forward_block_gr_predecoded(
        hid, eid, seg, prob, tiles, dec, *[pay[k] for k in NAMES], True, out=want, decoded_by_expert=by_expert)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    # the partial sums themselves: their slice-order sum is tris_backbone_linear's output
    acc = torch.zeros((R, rank), dtype=torch.float32, device=cuda)
    for s in range(pend.slices):
        acc = acc + pend.partials[s]
    assert torch.equal(acc.to(torch.float16).view(torch.int16), hid.view(torch.int16))


def test_deferred_backbone_entries_reject_unsupported_shapes(tris, cuda):
    """One slice: backbone_linear_deferred returns the projection itself.  The C entries reject what they cannot
    run with an error: a shape that takes the tiled GEMM (its reduction cannot be deferred) and partial sums for
    a rank past one 512-column chunk."""
    import ctypes

    from tris_moe_amd import _lib as lib

    ext = tris["ext"]
    note("deferred backbone: one slice, rejected shapes")
    rng = np.random.default_rng(5)
    x = torch.from_numpy(rng.standard_normal((2, 128)).astype(np.float16)).to(cuda)
    sv = torch.from_numpy((rng.standard_normal((128, 128)) * 0.05).astype(np.float16)).to(cuda)
    one = ext.backbone_linear_deferred(x, sv)
    assert isinstance(one, torch.Tensor)
    assert torch.equal(one.view(torch.int16), ext.backbone_linear(x, sv).view(torch.int16))
    L = lib.load()
    tokens, in_f, rank = 512, 4096, 512
    xs = torch.zeros((tokens, in_f), dtype=torch.float16, device=cuda)
    svs = torch.zeros((rank, in_f), dtype=torch.float16, device=cuda)
    out = torch.empty((tokens, rank), dtype=torch.float16, device=cuda)
    nbytes = int(L.tris_backbone_workspace_bytes(tokens, in_f, rank))
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=cuda)
    slices = ctypes.c_int32(-1)
    rc = L.tris_backbone_linear_deferred(xs.data_ptr(), tokens, in_f, None, svs.data_ptr(), rank, None,
                                         out.data_ptr(), ws.data_ptr(), int(ws.numel()), ctypes.byref(slices),
                                         torch.cuda.current_stream().cuda_stream)
    assert rc != 0 and b"tiled GEMM" in L.tris_last_error()
    pay = tris["qlinear"].payload_to_device(make_projection(tris, 77, 2, 64, 576), cuda)
    assert not ext.partials_gemm_ok(pay)
    pstruct = ext.make_payload_struct(576, *[pay[k] for k in ("qweight1", "qweight2_sparse", "qweight2_sparse_prefix")],
                                      None, None, None, *[pay[k] for k in ("c_map", "g_idx", "col_pack3", "row_pack3")],
                                      None, False, None, False, True, cuda, need_gr=False)
    part = torch.zeros((2, 1, 576), dtype=torch.float32, device=cuda)
    dec = torch.zeros((1, 9 * 1, 128), dtype=torch.int32, device=cuda)
    o = torch.empty((1, 64), dtype=torch.float16, device=cuda)
    rc = L.tris_grouped_forward_block_gr_predecoded_partials(
        part.data_ptr(), 2, 1, t_i32([0], cuda).data_ptr(), t_i32([0, 1], cuda).data_ptr(), 1, 1, dec.data_ptr(),
        ctypes.byref(pstruct), o.data_ptr(), 0, torch.cuda.current_stream().cuda_stream)
    assert rc != 0 and b"rank <= 512" in L.tris_last_error()


@pytest.mark.parametrize("tokens", [1, 2])
def test_block_down_partials_in_gemm_matches_reduced_backbone(tris, cuda, tokens, monkeypatch):
    """The decode step at fused-SwiGLU batches with the down backbone's partial sums added by the down GEMM
    (moe.DOWN_PARTIALS_IN_GEMM) gives the step with the reduction's own launch bit for bit, on the C1 layer."""
    from tris_moe_amd.configs import C1_MIXTRAL_DECODE as SPEC

    note(f"block decode step, down partial sums in the GEMM, T={tokens}")
    syn, ql, moe = tris["synthetic"], tris["qlinear"], tris["moe"]
    layer = syn.make_layer(SPEC, 6500 + tokens, tris["ext"].gr_encode)
    payloads = {p: ql.payload_to_device(layer[p], cuda) for p in ("gate", "up", "down")}
    backbones = {p: torch.from_numpy(layer["backbones"][p]).to(cuda) for p in ("gate", "up", "down")}
    rng = np.random.default_rng(tokens + 70)
    router = torch.from_numpy((rng.standard_normal((SPEC.num_experts, SPEC.hidden)) * 0.015).astype(np.float32))
    block = moe.TrisSparseMoeBlock(SPEC.hidden, SPEC.num_experts, SPEC.top_k, payloads, backbones,
                                   router_weight=router.to(cuda))
    inp = syn.make_inputs(SPEC, tokens, 6600 + tokens, layer["outlier_idx"])
    h = torch.from_numpy(inp["x"]).to(cuda).to(torch.bfloat16).reshape(1, tokens, SPEC.hidden)
    assert tokens * SPEC.top_k <= moe.FUSED_SWIGLU_MAX_ROWS
    with torch.no_grad():
        monkeypatch.setattr(moe, "DOWN_PARTIALS_IN_GEMM", True)
        got, lg_got = block(h)
        monkeypatch.setattr(moe, "DOWN_PARTIALS_IN_GEMM", False)
        want, lg_want = block(h)
    assert torch.equal(lg_got.view(torch.int16), lg_want.view(torch.int16))
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


COMBINE_CASES = [
    # experts of the two segments, inverse_perm (pick -> row), output dtype, every expert decoded
    ((3, 6), (0, 1), torch.bfloat16, False),
    ((1, 7), (1, 0), torch.bfloat16, True),   # the first pick's expert holds the second row
    ((0, 5), (1, 0), torch.float16, False),
]


@pytest.mark.parametrize("case", COMBINE_CASES, ids=lambda c: "e{}{}inv{}{}{}{}".format(
    c[0][0], c[0][1], c[1][0], c[1][1], "bf16" if c[2] == torch.bfloat16 else "fp16", "x" if c[3] else ""))
def test_down_gemm_with_one_token_combine_matches_combine_launch(tris, cuda, case):
    """tris_grouped_forward_block_gr_predecoded_partials_combine (one token routed to two experts, the routed
    combine in the down GEMM's launch) gives tris_moe_combine's output over the partial-sum down GEMM's rows, bit
    for bit, in either pick order and output dtype."""
    experts, inv, dt, by_expert = case
    E, in_f, rank, n = 8, 14336, 512, 320
    note(f"down GEMM with the one-token combine experts={experts} inv={inv} {dt} by_expert={by_expert}")
    ext, ql = tris["ext"], tris["qlinear"]
    rng = np.random.default_rng(sum(experts) * 11 + inv[0])
    x = torch.from_numpy(rng.standard_normal((2, in_f)).astype(np.float16)).to(cuda)
    sv = torch.from_numpy((rng.standard_normal((rank, in_f)) * 0.02).astype(np.float16)).to(cuda)
    pay = ql.payload_to_device(make_projection(tris, 950 + experts[0], E, n, rank), cuda)
    eid = t_i32(list(experts), cuda)
    seg = t_i32([0, 1, 2], cuda)
    pr = int(pay["qweight1"].size(1))
    nblk = ((pr + 1) // 2) * ((n + 63) // 64)
    dec = torch.full((E if by_expert else 2, nblk, 128), -7, dtype=torch.int32, device=cuda)
    ids = torch.arange(E, dtype=torch.int32, device=cuda) if by_expert else eid
    ext.grouped_block_gr_predecode_multi([(dec, pay["q_gmap_gr_words"], pay["q_gmap_gr_offsets"],
                                           pay["q_gmap_gr_meta"], pr, n)], ids)
    inverse_perm = t_i32(list(inv), cuda)
    w16 = torch.from_numpy(rng.uniform(0.1, 0.9, (1, 2)).astype(np.float16)).to(cuda)
    pend = ext.backbone_linear_deferred(x, sv)
    assert isinstance(pend, ext.BackbonePartials)
    got = ext.grouped_forward_block_gr_predecoded_partials_combine(
        pend, eid, seg, 2, dec, *[pay[k] for k in NAMES], inverse_perm, w16, out_dtype=dt, decoded_by_expert=by_expert)
    rows = torch.empty((2, n), dtype=torch.float16, device=cuda)
    ext.grouped_forward_block_gr_predecoded_partials(pend, eid, seg, 2, dec, *[pay[k] for k in NAMES], True, out=rows,
                                                     decoded_by_expert=by_expert)
    want = ext.moe_combine(rows, inverse_perm, w16, out_dtype=dt)
    torch.cuda.synchronize()
    assert got.dtype == dt and tuple(got.shape) == (1, n)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_one_token_combine_rejects_other_routes_with_zeros(tris, cuda):
    """A route that is not one token on two experts with one row each (here both rows in one segment) gives a zero
    output row instead of reading past the route."""
    ext, ql = tris["ext"], tris["qlinear"]
    note("one-token combine: malformed route")
    rng = np.random.default_rng(3)
    x = torch.from_numpy(rng.standard_normal((2, 4096)).astype(np.float16)).to(cuda)
    sv = torch.from_numpy((rng.standard_normal((512, 4096)) * 0.02).astype(np.float16)).to(cuda)
    pay = ql.payload_to_device(make_projection(tris, 977, 4, 128, 512), cuda)
    pr = int(pay["qweight1"].size(1))
    dec = torch.zeros((2, ((pr + 1) // 2) * 2, 128), dtype=torch.int32, device=cuda)
    pend = ext.backbone_linear_deferred(x, sv)
    got = ext.grouped_forward_block_gr_predecoded_partials_combine(
        pend, t_i32([1, 2], cuda), t_i32([0, 2, 2], cuda), 1, dec, *[pay[k] for k in NAMES], t_i32([0, 1], cuda),
        torch.full((1, 2), 0.5, dtype=torch.float16, device=cuda))
    torch.cuda.synchronize()
    assert torch.equal(got, torch.zeros_like(got))


def test_block_one_token_combine_in_down_gemm_matches_combine_launch(tris, cuda, monkeypatch):
    """The decode step at T = 1 with the combine in the down GEMM's launch (moe.COMBINE_IN_DOWN_GEMM) gives the
    step with the combine's own launch bit for bit, on the C1 layer."""
    from tris_moe_amd.configs import C1_MIXTRAL_DECODE as SPEC

    note("block decode step, one-token combine in the down GEMM")
    syn, ql, moe = tris["synthetic"], tris["qlinear"], tris["moe"]
    layer = syn.make_layer(SPEC, 6701, tris["ext"].gr_encode)
    payloads = {p: ql.payload_to_device(layer[p], cuda) for p in ("gate", "up", "down")}
    backbones = {p: torch.from_numpy(layer["backbones"][p]).to(cuda) for p in ("gate", "up", "down")}
    rng = np.random.default_rng(71)
    router = torch.from_numpy((rng.standard_normal((SPEC.num_experts, SPEC.hidden)) * 0.015).astype(np.float32))
    block = moe.TrisSparseMoeBlock(SPEC.hidden, SPEC.num_experts, SPEC.top_k, payloads, backbones,
                                   router_weight=router.to(cuda))
    for seed in (6801, 6802, 6803):
        inp = syn.make_inputs(SPEC, 1, seed, layer["outlier_idx"])
        h = torch.from_numpy(inp["x"]).to(cuda).to(torch.bfloat16).reshape(1, 1, SPEC.hidden)
        with torch.no_grad():
            monkeypatch.setattr(moe, "COMBINE_IN_DOWN_GEMM", True)
            got, lg_got = block(h)
            monkeypatch.setattr(moe, "COMBINE_IN_DOWN_GEMM", False)
            want, lg_want = block(h)
        assert torch.equal(lg_got.view(torch.int16), lg_want.view(torch.int16))
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), seed
