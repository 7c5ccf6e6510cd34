"""The in-kernel-decode MFMA grouped GEMM (tris_grouped_decode_forward_block_gr and the gate/up pair entry)
against the oracle: decode-sized segments, multi-tile segments, partial output tiles, output scale and bias,
dropped experts, rows gathered through an index, salient windows beyond one (and beyond 64 salient columns
in a slice), Rice k >= 4 and raw blocks, the C0 shape; exact weights through one-hot activations."""
import sys

import numpy as np
import pytest
import torch

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
                               salient_counts=salient_counts, output_scale=os_, bias=bs)


def segments(lengths, drop=None):
    ids = np.asarray([e for e, n in enumerate(lengths) if n > 0], dtype=np.int32)
    offs = np.concatenate([[0], np.cumsum([lengths[e] for e in ids])]).astype(np.int32)
    if drop is not None and ids.size:
        ids = ids.copy()
        ids[drop] = -1
    return ids, offs


def t32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(dev)


CASES = [
    dict(E=8, n=256, k=512, seg=[2, 0, 3, 1, 0, 0, 5, 2]),                # decode: a few rows per segment
    dict(E=4, n=200, k=512, seg=[17, 3, 0, 40]),                          # several row tiles, partial out tile
    dict(E=3, n=128, k=256, seg=[4, 4, 4], scale=True, bias=True),        # rank 256, epilogue
    dict(E=2, n=192, k=512, seg=[6, 9], salient_counts=[300, 40]),        # > 64 salient columns in a slice
    dict(E=3, n=64, k=512, seg=[5, 0, 3], p=0.05),                        # Rice k >= 4 blocks
    dict(E=3, n=64, k=512, seg=[5, 2, 3], p=0.6),                         # dense blocks (raw)
    dict(E=3, n=96, k=256, seg=[1, 1, 1]),                                # odd output tiles (a unit idle)
]


def case_id(c):
    extra = "".join(k[0] for k in ("scale", "bias") if c.get(k)) + (f"p{c['p']}" if "p" in c else "")
    return f"E{c['E']}n{c['n']}k{c['k']}{extra}" + ("sal" if c.get("salient_counts") else "")


@pytest.mark.parametrize("case", CASES, ids=case_id)
def test_decode_single_matches_oracle(tris, oracle_mod, cuda, case):
    note(f"decode single {case_id(case)}")
    case = dict(case)
    lengths = case.pop("seg")
    payload = make_projection(tris, 41, **case)
    dev = tris["qlinear"].payload_to_device(payload, cuda)
    assert tris["ext"].decode_payload_ok(dev)
    rows = int(sum(lengths))
    rng = np.random.default_rng(5)
    hidden = (rng.standard_normal((rows, case["k"])) * 1.5).astype(np.float16)
    ht = torch.from_numpy(hidden).to(cuda)
    for drop in (None, 0):
        ids, offs = segments(lengths, drop)
        got = tris["ext"].grouped_decode_forward(ht, dev, t32(ids, cuda), t32(offs, cuda), rows).cpu().numpy()
        want = oracle_mod.grouped_forward(payload, hidden, ids, offs, True)
        assert_close(got.astype(np.float32), want.astype(np.float32), f"drop={drop}")
        if drop is not None:
            assert not got[offs[0]:offs[1]].any()  # rows routed to no expert are zero
    # rows gathered through an index from a smaller activation tensor
    tokens = max(1, rows // 2)
    src = (rng.standard_normal((tokens, case["k"])) * 1.5).astype(np.float16)
    ridx = rng.integers(0, tokens, rows)
    ids, offs = segments(lengths)
    got = tris["ext"].grouped_decode_forward(torch.from_numpy(src).to(cuda), dev, t32(ids, cuda), t32(offs, cuda),
                                             rows, row_index=torch.from_numpy(ridx).to(cuda)).cpu().numpy()
    want = oracle_mod.grouped_forward(payload, src[ridx], ids, offs, True)
    assert_close(got.astype(np.float32), want.astype(np.float32), "row_index")


@pytest.mark.parametrize("swiglu", [False, True])
@pytest.mark.parametrize("shape", [(8, 512, 512, [2, 0, 3, 1, 4, 0, 5, 17]), (16, 1024, 256, None)],
                         ids=["mixtral-like", "olmoe-like"])
def test_decode_pair_matches_oracle(tris, oracle_mod, cuda, swiglu, shape):
    """Gate and up in one launch (units side by side): both outputs, or fp16(silu(g) * u) with g, u rounded to
    fp16 as the reference's two GEMM outputs are."""
    E, n, k, lengths = shape
    note(f"decode pair swiglu={swiglu} E={E} n={n} k={k}")
    rng = np.random.default_rng(6)
    if lengths is None:
        lengths = list(rng.integers(0, 5, E))
    pa = make_projection(tris, 51, E, n, k)
    pb = make_projection(tris, 52, E, n, k)
    da, db = (tris["qlinear"].payload_to_device(x, cuda) for x in (pa, pb))
    rows = int(sum(lengths))
    tokens = max(1, rows // 2)
    ha = rng.standard_normal((tokens, k)).astype(np.float16)
    hb = rng.standard_normal((tokens, k)).astype(np.float16)
    ridx = rng.integers(0, tokens, rows)
    ids, offs = segments(lengths)
    res = tris["ext"].grouped_decode_pair_forward(
        torch.from_numpy(ha).to(cuda), torch.from_numpy(hb).to(cuda), da, db, t32(ids, cuda), t32(offs, cuda), rows,
        row_index=torch.from_numpy(ridx).to(cuda), swiglu=swiglu)
    ga = oracle_mod.grouped_forward(pa, ha[ridx], ids, offs, True)
    ub = oracle_mod.grouped_forward(pb, hb[ridx], ids, offs, True)
    if swiglu:
        want = (oracle_mod.silu_f16(ga).astype(np.float32) * ub.astype(np.float32)).astype(np.float16)
        assert_close(res.cpu().numpy().astype(np.float32), want.astype(np.float32), "swiglu")
    else:
        assert_close(res[0].cpu().numpy().astype(np.float32), ga.astype(np.float32), "gate")
        assert_close(res[1].cpu().numpy().astype(np.float32), ub.astype(np.float32), "up")


@pytest.mark.parametrize("k,salient", [(512, None), (256, [90, 3]), (512, [300, 0])])
def test_decode_one_hot_weights_are_exact(tris, oracle_mod, cuda, k, salient):
    """One-hot activation rows read single weights: every output equals the oracle's exact fp16 weight (one
    product, no accumulation), for salient and non-salient columns alike."""
    note(f"decode one-hot k={k}")
    E, n = 2, 192
    payload = make_projection(tris, 61, E, n, k, salient_counts=salient)
    dev = tris["qlinear"].payload_to_device(payload, cuda)
    cols = np.arange(0, k, 3)
    hid = np.zeros((cols.size, k), dtype=np.float16)
    hid[np.arange(cols.size), cols] = 1.0
    ht = torch.from_numpy(hid).to(cuda)
    for e in range(E):
        ids = np.asarray([e], dtype=np.int32)
        offs = np.asarray([0, cols.size], dtype=np.int32)
        got = tris["ext"].grouped_decode_forward(ht, dev, t32(ids, cuda), t32(offs, cuda), cols.size).cpu().numpy()
        w = oracle_mod.dequant_grouped_expert(payload, e, True)   # [n, k]
        want = np.ascontiguousarray(w[:, cols].T)
        np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16), err_msg=f"expert {e}")
