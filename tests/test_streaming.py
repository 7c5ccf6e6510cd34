"""Whole-layer payload streaming (tris_moe_amd.streaming): the blob layout on the host, and on the GPU a
chain of streamed layers giving the resident path's bits (grouped_payload_sidecar.py:764-1153 semantics:
a slot is refilled only after the layer that used it has finished)."""
import numpy as np
import pytest
import torch

from tris_moe_amd import streaming
from tris_moe_amd.configs import MoELayerSpec

TINY = MoELayerSpec("tiny", hidden=256, num_experts=4, intermediate=384, top_k=2, rank=128, tokens=(3,))


def _layers(tris, n, seed0=500, gmap_p=None):
    ext, syn = tris["ext"], tris["synthetic"]
    return [syn.make_layer(TINY, seed0 + i, ext.gr_encode, gmap_p=gmap_p) for i in range(n)]


def test_layout_alignment_and_round_trip(tris):
    """Every tensor lands 256-byte aligned, in bounds, without overlap, and unpacks to its values;
    non-array payload fields are kept."""
    layer = _layers(tris, 1)[0]
    payloads = {p: layer[p] for p in streaming.PROJECTIONS}
    lay = streaming.layer_layout(payloads, layer["backbones"])
    ends = []
    for ent in lay.entries:
        assert ent.offset % streaming.ALIGN == 0
        ends.append((ent.offset, ent.offset + ent.nbytes))
    ends.sort()
    for (a0, a1), (b0, b1) in zip(ends, ends[1:]):
        assert a1 <= b0
    assert ends[-1][1] <= lay.nbytes and lay.nbytes % streaming.ALIGN == 0
    blob = np.zeros(lay.nbytes, dtype=np.uint8)
    streaming.pack_layer(payloads, layer["backbones"], lay, blob)
    views, bbs = streaming.unpack_views(lay, torch.from_numpy(blob))
    for p in streaming.PROJECTIONS:
        for key, val in payloads[p].items():
            if isinstance(val, np.ndarray):
                got = views[p][key].numpy()
                assert got.shape == val.shape, key
                np.testing.assert_array_equal(got.astype(np.float64), val.astype(np.float64), err_msg=key)
            else:
                assert views[p][key] == val, key
        np.testing.assert_array_equal(bbs[p].numpy(), layer["backbones"][p])


def test_layout_without_backbones(tris):
    layer = _layers(tris, 1)[0]
    payloads = {p: layer[p] for p in streaming.PROJECTIONS}
    with_bb = streaming.layer_layout(payloads, layer["backbones"])
    without = streaming.layer_layout(payloads, None)
    assert without.nbytes < with_bb.nbytes
    assert all(e.owner != "backbone" for e in without.entries)
    blob = np.zeros(without.nbytes, dtype=np.uint8)
    streaming.pack_layer(payloads, None, without, blob)
    _, bbs = streaming.unpack_views(without, torch.from_numpy(blob))
    assert bbs is None


def _resident_chain(tris, layers, x16, logits, dev):
    ql, moe = tris["qlinear"], tris["moe"]
    out = None
    for i, layer in enumerate(layers):
        pl = {p: ql.payload_to_device(layer[p], dev) for p in streaming.PROJECTIONS}
        bb = {p: torch.from_numpy(layer["backbones"][p]).to(dev) for p in streaming.PROJECTIONS}
        out = moe.grouped_moe_forward_from_logits(x16, logits[i], TINY.top_k, TINY.renormalize, pl, bb,
                                                  TINY.num_experts, torch.bfloat16)
        x16 = out.to(torch.float16)
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("slots,with_backbones", [(2, True), (1, True), (3, False)])
def test_streamed_chain_matches_resident(tris, cuda, slots, with_backbones):
    """Five layers through `slots` device slots (a slot reused while the copy stream runs ahead) give the
    resident chain's bits; the copies, bytes and slot reuses add up."""
    print(f"streamed chain slots={slots} backbones={with_backbones}", flush=True)
    layers = _layers(tris, 5)
    rng = np.random.default_rng(3)
    T = 3
    x16 = torch.from_numpy(rng.standard_normal((T, TINY.hidden)).astype(np.float16)).to(cuda)
    logits = [torch.from_numpy(rng.standard_normal((T, TINY.num_experts)).astype(np.float32)).to(cuda) for _ in layers]
    want = _resident_chain(tris, layers, x16, logits, cuda).cpu()
    host = [{p: l[p] for p in streaming.PROJECTIONS} for l in layers]
    bbs_host = [l["backbones"] for l in layers]
    st = streaming.GroupedPayloadStreamer(host, cuda, num_slots=slots, backbones=bbs_host if with_backbones else None)
    resident_bb = None
    if not with_backbones:
        resident_bb = [{p: torch.from_numpy(l["backbones"][p]).to(cuda) for p in streaming.PROJECTIONS} for l in layers]
    for rep in range(2):
        got = streaming.streamed_forward(st, x16, logits, TINY.top_k, TINY.renormalize, TINY.num_experts,
                                         backbones=resident_bb)
        torch.cuda.synchronize()
        assert torch.equal(got.cpu().view(torch.int16), want.view(torch.int16)), f"pass {rep}"
    assert st.stats["copies"] == 10
    assert st.stats["bytes"] == 2 * sum(st.layer_nbytes(i) for i in range(5))
    assert st.stats["slot_reuses"] == 10 - slots


@pytest.mark.gpu
def test_streamer_keeps_resident_layers(tris, cuda):
    """With as many slots as layers a second pass copies nothing."""
    print("streamer resident", flush=True)
    layers = _layers(tris, 2, seed0=900)
    host = [{p: l[p] for p in streaming.PROJECTIONS} for l in layers]
    st = streaming.GroupedPayloadStreamer(host, cuda, num_slots=2, backbones=[l["backbones"] for l in layers])
    rng = np.random.default_rng(4)
    x16 = torch.from_numpy(rng.standard_normal((2, TINY.hidden)).astype(np.float16)).to(cuda)
    logits = [torch.from_numpy(rng.standard_normal((2, TINY.num_experts)).astype(np.float32)).to(cuda) for _ in layers]
    a = streaming.streamed_forward(st, x16, logits, TINY.top_k, TINY.renormalize, TINY.num_experts)
    b = streaming.streamed_forward(st, x16, logits, TINY.top_k, TINY.renormalize, TINY.num_experts)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert st.stats["copies"] == 2 and st.stats["hits"] == 2


def _oracle_layer_check(oracle_mod, layer, x16, logits, got, spec, what):
    """One streamed layer's output against the oracle layer on the same input (the chain's fp16 input)."""
    w, sel = oracle_mod.route_topk(logits.cpu().numpy(), spec.top_k, spec.renormalize)
    want = oracle_mod.bf16_round(oracle_mod.moe_layer(
        x16.cpu().numpy(), w, sel, {p: layer[p] for p in streaming.PROJECTIONS}, layer["backbones"],
        spec.num_experts, weight_caches=layer.setdefault("_oracle_cache", {"gate": {}, "up": {}, "down": {}})))
    err = got.float().cpu().numpy().astype(np.float64) - want
    max_abs = float(np.abs(err).max())
    rel = float(np.linalg.norm(err) / np.linalg.norm(want))
    assert max_abs <= 2e-2 and rel <= 1e-3, f"{what}: max_abs={max_abs:.3g} rel_l2={rel:.3g}"


def _chain_against_oracle(oracle_mod, st, layers, x16, logits, spec, what, backbones=None):
    """The streamed chain with the residual stream (so activations stay O(1) over the layers: without it they
    shrink towards fp16 underflow); each layer's output against the oracle layer on that layer's input."""
    outs, ins = [], []
    streaming.streamed_forward(st, x16, logits, spec.top_k, spec.renormalize, spec.num_experts,
                               backbones=backbones, outputs=outs, inputs=ins, residual=True)
    torch.cuda.synchronize()
    assert len(outs) == len(layers) == len(ins)
    assert torch.equal(ins[0], x16)
    for i, out in enumerate(outs):
        assert float(out.float().abs().max()) > 6.2e-5, f"{what} layer {i}: output in the fp16 subnormal range"
        _oracle_layer_check(oracle_mod, layers[i], ins[i], logits[i], out, spec, f"{what} layer {i}")
        if i + 1 < len(ins):
            assert torch.equal(ins[i + 1], (ins[i].float() + out.float()).to(torch.float16))


@pytest.mark.gpu
@pytest.mark.parametrize("slots,with_backbones", [(2, True), (1, False)])
def test_streamed_chain_matches_oracle(tris, oracle_mod, cuda, slots, with_backbones):
    """Every layer of a five-layer streamed chain against the oracle layer on the same input."""
    print(f"streamed chain vs oracle slots={slots} backbones={with_backbones}", flush=True)
    layers = _layers(tris, 5, seed0=700)
    rng = np.random.default_rng(13)
    T = 3
    x16 = torch.from_numpy(rng.standard_normal((T, TINY.hidden)).astype(np.float16)).to(cuda)
    logits = [torch.from_numpy(rng.standard_normal((T, TINY.num_experts)).astype(np.float32)).to(cuda) for _ in layers]
    host = [{p: l[p] for p in streaming.PROJECTIONS} for l in layers]
    st = streaming.GroupedPayloadStreamer(host, cuda, num_slots=slots,
                                          backbones=[l["backbones"] for l in layers] if with_backbones else None)
    resident_bb = None
    if not with_backbones:
        resident_bb = [{p: torch.from_numpy(l["backbones"][p]).to(cuda) for p in streaming.PROJECTIONS} for l in layers]
    _chain_against_oracle(oracle_mod, st, layers, x16, logits, TINY, f"slots={slots}", backbones=resident_bb)


def test_split_bitmaps_partition(tris):
    """split_bitmaps: the split-bitmap tensors go to the streamed dicts, every other key stays resident, and the
    bitmap-only blob round-trips."""
    from gr_cases import to_sparse
    import oracle

    layer = tris["synthetic"].make_layer(TINY, 31, tris["ext"].gr_encode, keep_dense_gmap=True)
    for form in ("block_gr", "sparse"):
        host = {p: (to_sparse(oracle, layer[p], TINY.rank) if form == "sparse" else
                    {k: v for k, v in layer[p].items() if k != "gmap_dense"}) for p in streaming.PROJECTIONS}
        streamed, rest = streaming.split_bitmaps(host)
        for p in streaming.PROJECTIONS:
            assert set(streamed[p]) | set(rest[p]) == set(host[p]) and not set(streamed[p]) & set(rest[p])
            want = {"q_gmap_sparse", "q_gmap_sparse_prefix"} if form == "sparse" else \
                {"q_gmap_gr_words", "q_gmap_gr_offsets", "q_gmap_gr_meta"}
            assert set(streamed[p]) == want
        lay = streaming.layer_layout(streamed)
        blob = np.zeros(lay.nbytes, dtype=np.uint8)
        streaming.pack_layer(streamed, None, lay, blob)
        views, bb = streaming.unpack_views(lay, torch.from_numpy(blob))
        assert bb is None
        for p in streaming.PROJECTIONS:
            for k, v in streamed[p].items():
                np.testing.assert_array_equal(views[p][k].numpy(), v)


@pytest.mark.gpu
@pytest.mark.parametrize("form", ["sparse", "block_gr"])
def test_streamed_bitmaps_only_match_oracle(tris, oracle_mod, cuda, form):
    """The reference's staging mode (grouped_payload_sidecar.py:764-1146): only the split bitmaps stream
    through two slots, every other payload tensor and the backbones stay resident; sparse-form payloads
    (the format that mode serves) and block-GR ones; every layer against the oracle."""
    from gr_cases import to_sparse

    print(f"streamed bitmaps only, {form}", flush=True)
    q = tris["qlinear"]
    raw = [tris["synthetic"].make_layer(TINY, 900 + i, tris["ext"].gr_encode, keep_dense_gmap=True)
           for i in range(4)]
    layers = []
    for l in raw:
        conv = {p: (to_sparse(oracle_mod, l[p], TINY.rank) if form == "sparse" else
                    {k: v for k, v in l[p].items() if k != "gmap_dense"}) for p in streaming.PROJECTIONS}
        conv["backbones"] = l["backbones"]
        layers.append(conv)
    split = [streaming.split_bitmaps(l) for l in layers]
    resident = [{p: q.payload_to_device(rest[p], cuda) for p in streaming.PROJECTIONS} for _, rest in split]
    st = streaming.GroupedPayloadStreamer([s for s, _ in split], cuda, num_slots=2, resident=resident)
    rng = np.random.default_rng(17)
    T = 3
    x16 = torch.from_numpy(rng.standard_normal((T, TINY.hidden)).astype(np.float16)).to(cuda)
    logits = [torch.from_numpy(rng.standard_normal((T, TINY.num_experts)).astype(np.float32)).to(cuda)
              for _ in layers]
    bb = [{p: torch.from_numpy(l["backbones"][p]).to(cuda) for p in streaming.PROJECTIONS} for l in layers]
    _chain_against_oracle(oracle_mod, st, layers, x16, logits, TINY, f"bitmaps only {form}", backbones=bb)
    assert st.stats["copies"] == len(layers)


@pytest.mark.gpu
@pytest.mark.parametrize("p", [0.05, 0.15, 0.30])
def test_streamed_mixtral_layers_match_oracle(tris, oracle_mod, cuda, p):
    """C4 at its real layer shape: Mixtral-8x7B MoE layers (hidden 4096, 8 experts,
    intermediate 14336, rank 512) at decode T = 8 with split-bitmap density p, streamed from pinned host memory
    through two device slots (layers A, B, A: a slot mix-up changes the weights), every layer's output against
    the oracle layer on the same input."""
    from tris_moe_amd.configs import C4_STREAMING as SPEC

    print(f"C4 streamed Mixtral layers p={p}", flush=True)
    ext, syn = tris["ext"], tris["synthetic"]
    a = syn.make_layer(SPEC, 4100, ext.gr_encode, gmap_p=p)
    b = syn.make_layer(SPEC, 4200, ext.gr_encode, gmap_p=p)
    layers = [a, b, a]
    T = SPEC.tokens[0]
    inp = syn.make_inputs(SPEC, T, 4300, a["outlier_idx"])
    x16 = torch.from_numpy(inp["x"]).to(cuda).to(torch.bfloat16).to(torch.float16)
    rng = np.random.default_rng(int(p * 100))
    logits = [torch.from_numpy(rng.standard_normal((T, SPEC.num_experts)).astype(np.float32)).to(cuda)
              for _ in layers]
    host = [{q: l[q] for q in streaming.PROJECTIONS} for l in layers]
    st = streaming.GroupedPayloadStreamer(host, cuda, num_slots=2, backbones=[l["backbones"] for l in layers])
    _chain_against_oracle(oracle_mod, st, layers, x16, logits, SPEC, f"C4 p={p}")
    assert st.stats["copies"] == 3 and st.stats["slot_reuses"] == 1


@pytest.mark.gpu
def test_prefetch_never_refills_an_acquired_slot(tris, cuda):
    """A slot whose layer is acquired and not released is skipped by prefetch (its kernels may still read it);
    with every slot held, prefetch raises."""
    print("streamer held slots", flush=True)
    layers = _layers(tris, 3, seed0=950)
    host = [{p: l[p] for p in streaming.PROJECTIONS} for l in layers]
    st = streaming.GroupedPayloadStreamer(host, cuda, num_slots=2)
    st.prefetch(0)
    st.acquire(0)
    st.prefetch(1)
    st.prefetch(2)        # round-robin would take slot 0 (layer 0, held): it takes slot 1 instead
    assert st._where.get(0) == 0 and st._where.get(2) == 1 and 1 not in st._where
    st.acquire(2)
    with pytest.raises(RuntimeError, match="every slot"):
        st.prefetch(1)
    st.release(0)
    assert st.prefetch(1) == 0
    st.release(2)
    torch.cuda.synchronize()
