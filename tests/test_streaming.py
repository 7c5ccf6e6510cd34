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
