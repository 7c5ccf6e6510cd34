"""GPU parity of the HIP path against the CPU oracle (run on the MI355X box: -m gpu).

Integer work (GR decode, predecode, route, dequantised fp16 weights) must be
bit-exact; fp16 GEMM outputs and layer outputs must be within
max-abs 2e-2 and relative-L2 1e-3 of the oracle.
"""
import math
import sys

import numpy as np
import pytest
import torch

from gr_cases import (block_from_positions, case_expected_words, case_positions, load_known_answers,
                      multi_block_dense, random_bitmap, structured_bitmap)

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


def ceil_div(a, b):
    return (a + b - 1) // b


def t_i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(dev)


def stacked_gr(oracle_mod, denses):
    coded = [oracle_mod.gr_encode(d) for d in denses]
    width = max(1, max(c[0].size for c in coded))
    words = np.zeros((len(denses), width), dtype=np.int32)
    for e, c in enumerate(coded):
        words[e, : c[0].size] = c[0]
    return words, np.stack([c[1] for c in coded]), np.stack([c[2] for c in coded])


def ulps(got, want, dtype):
    """|got - want| in units of the dtype's ulp at the larger magnitude (fp16 subnormals included)."""
    m = np.maximum(np.abs(got), np.abs(want)).astype(np.float64)
    if dtype == "fp16":
        ulp = np.spacing(m.astype(np.float16)).astype(np.float64)
    else:
        ulp = np.exp2(np.floor(np.log2(np.maximum(m, 2.0 ** -126))) - 7)
    return np.abs(got.astype(np.float64) - want.astype(np.float64)) / ulp


# --------------------------------------------------------------- GR decode
def test_gr_decode_known_answers(tris, oracle_mod, cuda):
    ext = tris["ext"]
    kats = load_known_answers()
    for case in kats["single_block"]:
        note(f"gr kat {case['name']}")
        dense = block_from_positions(case_positions(case))
        words = case_expected_words(case, dense)
        if words.size == 0:
            words = np.zeros(1, dtype=np.int32)
        got = ext.gr_decode_dense(t_i32(words[None], cuda), t_i32([[0, case_expected_words(case, dense).size]], cuda),
                                  t_i32([[case["meta"]]], cuda), t_i32([0], cuda), 2, 64)
        np.testing.assert_array_equal(got[0].cpu().numpy(), dense, err_msg=case["name"])
    for case in kats["multi_block"]:
        note(f"gr kat {case['name']}")
        dense = multi_block_dense(case)
        got = ext.gr_decode_dense(t_i32([case["words"]], cuda), t_i32([case["offsets"]], cuda),
                                  t_i32([case["meta"]], cuda), t_i32([0], cuda), case["packed_rows"],
                                  case["outfeatures"])
        np.testing.assert_array_equal(got[0].cpu().numpy(), dense)


@pytest.mark.parametrize("p", [0.0, 0.05, 0.15, 0.3, 0.6, 0.97])
def test_gr_decode_random_bit_exact(tris, oracle_mod, cuda, p):
    note(f"gr random p={p}")
    rng = np.random.default_rng(int(p * 1000) + 1)
    shape = (16, 448)
    denses = [random_bitmap(rng, *shape, p) for _ in range(3)]
    words, offsets, meta = stacked_gr(oracle_mod, denses)
    got = tris["ext"].gr_decode_dense(t_i32(words, cuda), t_i32(offsets, cuda), t_i32(meta, cuda),
                                      t_i32([2, 0, 1, 2], cuda), *shape).cpu().numpy()
    for i, e in enumerate([2, 0, 1, 2]):
        np.testing.assert_array_equal(got[i], denses[e])


@pytest.mark.parametrize("kind", ["full", "corners", "stripes", "sparse_long_runs"])
def test_gr_decode_structured_and_padded(tris, oracle_mod, cuda, kind):
    note(f"gr structured {kind}")
    dense = structured_bitmap(kind, 9, 131, np.random.default_rng(5))
    for kmin, kmax in ((0, 7), (3, 3), (7, 7), (0, 0)):
        words, offsets, meta = stacked_gr(oracle_mod, [dense])
        if (kmin, kmax) != (0, 7):
            w, o, m = oracle_mod.gr_encode(dense, kmin, kmax)
            words, offsets, meta = (w[None] if w.size else np.zeros((1, 1), np.int32)), o[None], m[None]
        got = tris["ext"].gr_decode_dense(t_i32(words, cuda), t_i32(offsets, cuda), t_i32(meta, cuda),
                                          t_i32([0], cuda), 9, 131)
        np.testing.assert_array_equal(got[0].cpu().numpy(), dense)


@pytest.mark.parametrize("k", list(range(16)))
def test_gr_decode_malformed_streams_follow_reference(tris, oracle_mod, cuda, k):
    """one_count disagreeing with the stream, unterminated runs, stray bits, k > 7: the GPU decoder
    reproduces the reference decoder exactly (serial rules)."""
    note(f"gr malformed k={k}")
    rng = np.random.default_rng(500 + k)
    nblk = 24
    words, offsets, meta = [], [0], []
    for b in range(nblk):
        nw = int(rng.integers(0, 150))
        w = rng.integers(-2**31, 2**31, size=nw, dtype=np.int64).astype(np.int32)
        if b % 3 == 0 and nw:
            w[-(nw // 2 + 1):] = 0
        if b % 4 == 1:
            w = (w & np.int32(0x11111111)).astype(np.int32)
        words.extend(w.tolist())
        offsets.append(len(words))
        meta.append(k | (int(rng.integers(0, 700)) << 8) if b % 7 else 16)
    words_a = np.asarray(words if words else [0], dtype=np.int32)[None]
    offsets_a = np.asarray(offsets, dtype=np.int32)[None]
    meta_a = np.asarray(meta, dtype=np.int32)[None]
    packed_rows, n = 2 * 4, 64 * 6  # 4 k-blocks x 6 out-blocks = 24 blocks
    want = oracle_mod.gr_predecode(words_a, offsets_a, meta_a, np.array([0]), nblk)
    buf = torch.zeros((1, nblk, 128), dtype=torch.int32, device=cuda)
    got = tris["ext"].compact3_tris_precomputed_grouped_block_gr_predecode(
        buf, t_i32([0], cuda), t_i32(words_a, cuda), t_i32(offsets_a, cuda), t_i32(meta_a, cuda), packed_rows, n)
    np.testing.assert_array_equal(got.cpu().numpy(), want)


def rice_completions(words, k: int) -> int:
    """Codewords (a 1 after any zeros, then k bits) completed within a Rice(k) stream read LSB first, k >= 1."""
    bits = np.unpackbits(np.asarray(words, dtype=np.int32).view(np.uint8), bitorder="little")
    count, state = 0, 0
    for b in bits.tolist():
        if state == 0:
            state = k if b else 0
        else:
            state -= 1
            count += state == 0
    return count


@pytest.mark.parametrize("k", [3, 4, 5, 6, 7])
def test_gr_decode_large_rice_parameter(tris, oracle_mod, cuda, k):
    """Rice k in [3, 7] (split maps sparser than p ~ 0.12) decode in parallel through the nibble tables: forced-k
    encodings of sparse, very sparse and clustered bitmaps (and denser ones, which the encoder stores raw at this
    k) decode bit-exactly through the predecode and dense entries."""
    note(f"gr large k={k}")
    rng = np.random.default_rng(700 + k)
    rows, n = 16, 448
    denses = [random_bitmap(rng, rows, n, p) for p in (0.003, 0.01, 0.03, 0.06, 0.12)]
    denses.append(structured_bitmap("sparse_long_runs", rows, n, rng))
    coded = [oracle_mod.gr_encode(d, k, k) for d in denses]
    width = max(1, max(c[0].size for c in coded))
    words = np.zeros((len(denses), width), dtype=np.int32)
    for e, c in enumerate(coded):
        words[e, : c[0].size] = c[0]
    offsets = np.stack([c[1] for c in coded])
    meta = np.stack([c[2] for c in coded])
    assert ((meta & 15) == k).any()
    ids = np.array([5, 0, 3, 1, 4, 2, 0], dtype=np.int32)
    nblk = (rows // 2) * (n // 64)
    want = oracle_mod.gr_predecode(words, offsets, meta, ids, nblk)
    buf = torch.empty((ids.size, nblk, 128), dtype=torch.int32, device=cuda)
    got = tris["ext"].compact3_tris_precomputed_grouped_block_gr_predecode(
        buf, t_i32(ids, cuda), t_i32(words, cuda), t_i32(offsets, cuda), t_i32(meta, cuda), rows, n)
    np.testing.assert_array_equal(got.cpu().numpy(), want)
    dense = tris["ext"].gr_decode_dense(t_i32(words, cuda), t_i32(offsets, cuda), t_i32(meta, cuda),
                                        t_i32(ids, cuda), rows, n).cpu().numpy()
    for i, e in enumerate(ids):
        np.testing.assert_array_equal(dense[i], denses[e])


@pytest.mark.parametrize("k", [3, 4, 5, 6, 7])
def test_gr_decode_large_rice_parameter_count_matching_streams(tris, oracle_mod, cuda, k):
    """Arbitrary streams whose one_count equals their completed codewords, which the parallel k >= 3 path accepts:
    positions run past bit 4095 (dropped, where the reference stops), unary runs and remainders cross words and
    lanes, long zero runs; one_count one above or below its count takes the serial rules.  Expected: the
    oracle's restatement of the reference decoder."""
    note(f"gr large k={k} count-matching")
    rng = np.random.default_rng(900 + k)
    nblk = 24
    words, offsets, meta = [], [0], []
    for b in range(nblk):
        nw = int(rng.integers(1, 129))
        w = rng.integers(-2**31, 2**31, size=nw, dtype=np.int64).astype(np.int32)
        if b % 4 == 1:
            w = (w & np.int32(0x01010101)).astype(np.int32)  # long unary runs
        elif b % 4 == 2:
            w = (w & np.int32(0x11111111)).astype(np.int32)
        elif b % 4 == 3:
            w[rng.random(nw) < 0.5] = 0  # whole zero words between codewords
        ones = rice_completions(w, k) + (0, 0, 0, 1, -1, 0)[b % 6]
        words.extend(w.tolist())
        offsets.append(len(words))
        meta.append(k | (max(ones, 0) << 8))
    words_a = np.asarray(words, dtype=np.int32)[None]
    offsets_a = np.asarray(offsets, dtype=np.int32)[None]
    meta_a = np.asarray(meta, dtype=np.int32)[None]
    packed_rows, n = 2 * 4, 64 * 6  # 4 k-blocks x 6 out-blocks = 24 blocks
    want = oracle_mod.gr_predecode(words_a, offsets_a, meta_a, np.array([0]), nblk)
    assert want.any()
    buf = torch.zeros((1, nblk, 128), dtype=torch.int32, device=cuda)
    got = tris["ext"].compact3_tris_precomputed_grouped_block_gr_predecode(
        buf, t_i32([0], cuda), t_i32(words_a, cuda), t_i32(offsets_a, cuda), t_i32(meta_a, cuda), packed_rows, n)
    np.testing.assert_array_equal(got.cpu().numpy(), want)


@pytest.mark.parametrize("experts,packed_rows,n", [(1, 64, 3200), (3, 128, 2048), (2, 128, 14336), (5, 128, 14336)],
                         ids=["1600blk", "6144blk", "28672blk", "71680blk"])
def test_predecode_large_grids(tris, oracle_mod, cuda, experts, packed_rows, n):
    """Block counts that select each lanes-per-block width of the decoder (32 lanes up to 8192 blocks, 16 above)."""
    note(f"predecode large E={experts} rows={packed_rows} n={n}")
    rng = np.random.default_rng(packed_rows + n + experts)
    denses = [random_bitmap(rng, packed_rows, n, (0.15, 0.02, 0.5, 0.3, 0.08)[i]) for i in range(experts)]
    words, offsets, meta = stacked_gr(oracle_mod, denses)
    ids = np.arange(experts, dtype=np.int32)[::-1].copy()
    nblk = (packed_rows // 2) * (n // 64)
    want = oracle_mod.gr_predecode(words, offsets, meta, ids, nblk)
    buf = torch.empty((experts, nblk, 128), dtype=torch.int32, device=cuda)
    got = tris["ext"].compact3_tris_precomputed_grouped_block_gr_predecode(
        buf, t_i32(ids, cuda), t_i32(words, cuda), t_i32(offsets, cuda), t_i32(meta, cuda), packed_rows, n)
    np.testing.assert_array_equal(got.cpu().numpy(), want)
    dense = tris["ext"].gr_decode_dense(t_i32(words, cuda), t_i32(offsets, cuda), t_i32(meta, cuda),
                                        t_i32(ids, cuda), packed_rows, n).cpu().numpy()
    for i, e in enumerate(ids):
        np.testing.assert_array_equal(dense[i], denses[e])


def test_predecode_large_grid_sparse_maps(tris, oracle_mod, cuda):
    """16 lanes per block (over 8192 blocks) on sparse maps: Rice k = 3 streams of 52-76 words (spans of up to 5
    words a lane), k = 4 and 5, mixed with k = 2 and 1 blocks in one launch."""
    note("predecode large grid sparse maps")
    rng = np.random.default_rng(31)
    packed_rows, n = 64, 14336
    ps = (0.1, 0.12, 0.05, 0.03, 0.2, 0.08)
    denses = [random_bitmap(rng, packed_rows, n, p) for p in ps]
    words, offsets, meta = stacked_gr(oracle_mod, denses)
    assert {3, 4, 5} <= set(np.unique(meta & 15).tolist())
    ids = np.array([0, 1, 2, 3, 4, 5], dtype=np.int32)
    nblk = (packed_rows // 2) * (n // 64)
    want = oracle_mod.gr_predecode(words, offsets, meta, ids, nblk)
    buf = torch.empty((ids.size, nblk, 128), dtype=torch.int32, device=cuda)
    got = tris["ext"].compact3_tris_precomputed_grouped_block_gr_predecode(
        buf, t_i32(ids, cuda), t_i32(words, cuda), t_i32(offsets, cuda), t_i32(meta, cuda), packed_rows, n)
    np.testing.assert_array_equal(got.cpu().numpy(), want)


def test_predecode_multi_matches_single_calls(tris, oracle_mod, cuda):
    """Three projections of different block counts in one launch give each projection's single-call
    result bit for bit (slots with expert -1 give zero blocks)."""
    note("predecode multi")
    rng = np.random.default_rng(12)
    shapes = [(16, 448, 0.15), (16, 448, 0.3), (32, 128, 0.05)]
    ids = np.array([2, 0, -1], dtype=np.int32)
    jobs, want = [], []
    for rows, n, p in shapes:
        denses = [random_bitmap(rng, rows, n, p) for _ in range(3)]
        words, offsets, meta = stacked_gr(oracle_mod, denses)
        nblk = (rows // 2) * ((n + 63) // 64)
        want.append(oracle_mod.gr_predecode(words, offsets, meta, ids, nblk))
        buf = torch.full((ids.size, nblk, 128), 7, dtype=torch.int32, device=cuda)
        jobs.append((buf, t_i32(words, cuda), t_i32(offsets, cuda), t_i32(meta, cuda), rows, n))
    got = tris["ext"].grouped_block_gr_predecode_multi(jobs, t_i32(ids, cuda))
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g.cpu().numpy(), w)


def test_predecode_layout_and_negative_slots(tris, oracle_mod, cuda):
    note("predecode layout")
    rng = np.random.default_rng(8)
    denses = [random_bitmap(rng, 6, 200, 0.15) for _ in range(4)]
    words, offsets, meta = stacked_gr(oracle_mod, denses)
    ids = np.array([3, -1, 0, 2], dtype=np.int32)
    nblk = 3 * 4
    want = oracle_mod.gr_predecode(words, offsets, meta, ids, nblk)
    buf = torch.full((4, nblk, 128), 7, dtype=torch.int32, device=cuda)
    got = tris["ext"].compact3_tris_precomputed_grouped_block_gr_predecode(
        buf, t_i32(ids, cuda), t_i32(words, cuda), t_i32(offsets, cuda), t_i32(meta, cuda), 6, 200)
    np.testing.assert_array_equal(got.cpu().numpy(), want)


# ------------------------------------------------------------------ dequant
def make_projection(tris, seed, E, n, k, p=0.15, salient_counts=None, scale=False, bias=False, g_idx=None):
    syn = tris["synthetic"]
    rng = syn.rng_for(seed)
    os_ = rng.uniform(0.5, 1.5, (E, n)).astype(np.float16) if scale else None
    bs = (rng.standard_normal((E, n)) * 0.1).astype(np.float16) if bias else None
    return syn.make_projection(rng, E, n, k, p, rng.random(k) + 0.5, tris["ext"].gr_encode,
                               salient_counts=salient_counts, output_scale=os_, bias=bs, g_idx=g_idx,
                               keep_dense_gmap=True)


DEQUANT_CASES = [
    dict(E=3, n=128, k=256),
    dict(E=2, n=100, k=96),                                 # partial out block, K not a multiple of 64
    dict(E=4, n=64, k=512, salient_counts=[0, 1, 40, 70]),  # ragged qweight2_sparse rows
    dict(E=2, n=96, k=256, g_idx="alternating"),            # non-uniform groups
    dict(E=2, n=64, k=128, p=0.9),
]


@pytest.mark.parametrize("case", DEQUANT_CASES, ids=lambda c: "-".join(f"{a}{b}" for a, b in c.items() if a != "salient_counts"))
def test_dequant_bit_exact(tris, oracle_mod, cuda, case):
    note(f"dequant {case}")
    case = dict(case)
    g_idx = None
    if case.pop("g_idx", None) == "alternating":
        g_idx = (np.arange(case["k"]) % 2).astype(np.int32)
    payload = make_projection(tris, 31, g_idx=g_idx, **case)
    dev = tris["qlinear"].payload_to_device(payload, cuda)
    E, k = case["E"], case["k"]
    ids = torch.tensor([E - 1, -1] + list(range(E)), dtype=torch.int32, device=cuda)
    for uniform in (False, True):
        got = tris["ext"].compact3_dequant(dev, k, ids, use_uniform_k64_groups=uniform).cpu().numpy()
        for i, e in enumerate(ids.tolist()):
            if e < 0:
                assert not got[i].any()
                continue
            want = oracle_mod.dequant_grouped_expert(payload, e, uniform)
            np.testing.assert_array_equal(got[i].view(np.uint16), want.view(np.uint16), err_msg=f"expert {e}")


# -------------------------------------------------------------------- route
@pytest.mark.parametrize("t,k,e", [(1, 2, 8), (4, 2, 8), (16, 2, 8), (16, 8, 64), (33, 8, 256), (2048, 2, 8)])
def test_route_matches_oracle(tris, oracle_mod, cuda, t, k, e):
    note(f"route t={t} k={k} e={e}")
    rng = np.random.default_rng(t + k + e)
    sel = np.stack([rng.choice(e, size=k, replace=False) for _ in range(t)]).astype(np.int64)
    want = oracle_mod.build_route(sel, e, 4)
    got = tris["qlinear"].build_grouped_route(torch.from_numpy(sel).to(cuda), e)
    for key in ("perm", "grouped_token_indices", "grouped_slots", "grouped_expert_ids", "expert_ids",
                "segment_offsets", "problem_offsets"):
        np.testing.assert_array_equal(got[key].cpu().numpy(), want[key], err_msg=key)
    assert got["total_problem_tiles_host"] == want["total_problem_tiles"]
    assert int(got["total_problem_tiles"][0]) == want["total_problem_tiles"]


ROUTE_TOPK_CASES = [(t, k, e, True) for t, k, e in [(1, 2, 8), (16, 2, 8), (32, 2, 64), (8, 8, 60), (4, 16, 16),
                                                    (3, 1, 64), (16, 8, 64), (33, 2, 8), (7, 8, 256), (256, 8, 128)]]
# top_k below its pick-list bucket on the one-wavefront router (buckets of 2, 8 and 16 picks), both weightings;
# the same top_k on the workgroup router; and the workgroup router without renormalisation (OLMoE's default)
ROUTE_TOPK_CASES += [(t, k, e, rn) for t, k, e in [(8, 4, 16), (4, 6, 12), (2, 12, 16), (5, 3, 16), (8, 4, 32),
                                                   (4, 6, 60), (2, 12, 64), (16, 8, 64)]
                     for rn in (False, True)]
ROUTE_TOPK_CASES += [(16, 8, 128, False), (64, 2, 8, False)]
# the workgroup router's expert-per-lane buckets (1, 2, 4, 8, 16 experts a lane), its largest shapes (2048
# routed rows, 1024 experts) and many 64-token scatter chunks
ROUTE_TOPK_CASES += [(t, k, e, True) for t, k, e in [(100, 3, 200), (40, 8, 512), (32, 8, 1024), (128, 16, 1024),
                                                     (2048, 1, 64), (1000, 2, 100), (9, 8, 60)]]


@pytest.mark.parametrize("t,k,e,renorm", ROUTE_TOPK_CASES)
def test_route_topk_fused_matches_oracle(tris, oracle_mod, cuda, t, k, e, renorm):
    """Fused softmax / top-k / route: the selection and the route are exactly the oracle's
    (stable argsort of the fp32 softmax), weights within one fp16 ulp.  Up to 64 routed rows and 8
    experts one wavefront does it (pick lists of 2, 8 or 16 entries, the smallest that holds top_k);
    otherwise one workgroup (one wavefront per token, 1, 2, 4, 8 or 16 experts a lane)."""
    note(f"route topk fused t={t} k={k} e={e} renorm={renorm}")
    rng = np.random.default_rng(t * 100 + e + k)
    logits = rng.standard_normal((t, e)).astype(np.float32)
    if t > 1:
        logits[1, : min(e, 4)] = 0.25  # exact ties among the top experts
    w, sel = oracle_mod.route_topk(logits, k, renorm)
    r = tris["ext"].route_topk_grouped(torch.from_numpy(logits).to(cuda), k, renorm, 4)
    np.testing.assert_array_equal(r["selected_experts"].cpu().numpy(), sel)
    want = oracle_mod.build_route(sel, e, 4)
    for key in ("perm", "grouped_token_indices", "grouped_slots"):
        np.testing.assert_array_equal(r[key].cpu().numpy(), np.asarray(want[key]), err_msg=key)
    na = len(want["expert_ids"])
    np.testing.assert_array_equal(r["expert_ids"].cpu().numpy()[:na], np.asarray(want["expert_ids"]))
    np.testing.assert_array_equal(r["segment_offsets"].cpu().numpy()[: na + 1], np.asarray(want["segment_offsets"]))
    np.testing.assert_array_equal(r["problem_offsets"].cpu().numpy()[: na + 1], np.asarray(want["problem_offsets"]))
    # padding to num_experts segments: no expert, empty segments at the end
    assert (r["expert_ids"].cpu().numpy()[na:] == -1).all()
    assert (r["segment_offsets"].cpu().numpy()[na:] == t * k).all()
    assert (r["problem_offsets"].cpu().numpy()[na:] == want["problem_offsets"][-1]).all()
    np.testing.assert_allclose(r["routing_weights"].cpu().numpy(), w, rtol=2e-6, atol=1e-7)
    got16 = r["routing_weights_f16"].cpu().numpy().view(np.int16).astype(np.int32)
    want16 = w.astype(np.float16).view(np.int16).astype(np.int32)
    assert np.abs(got16 - want16).max() <= 1
    inv = r["inverse_perm"].cpu().numpy()
    np.testing.assert_array_equal(r["perm"].cpu().numpy()[inv], np.arange(t * k))


@pytest.mark.parametrize("t,k,e,renorm", [(2048, 2, 8, True), (1024, 8, 256, True), (3000, 1, 64, False),
                                          (100, 16, 1024, True), (5, 3, 7, False), (40000, 2, 8, True),
                                          (257, 6, 60, False), (0, 2, 8, True)])
def test_route_topk_tokens_matches_oracle(tris, oracle_mod, cuda, t, k, e, renorm):
    """The token-parallel router (tris_route_topk, batches past the one-launch router: C2's 2048 tokens, C3's
    1024 tokens x top 8 of 256): selection exactly the oracle's, ties to the lower expert, weights within one
    fp16 ulp; 40000 tokens run the grid-stride loop; then the two-kernel route of its picks is the oracle's."""
    note(f"route topk tokens t={t} k={k} e={e} renorm={renorm}")
    rng = np.random.default_rng(t * 7 + e + k)
    logits = (rng.standard_normal((t, e)) * 1.5).astype(np.float32)
    if t > 3:
        logits[1, : min(e, 4)] = 0.25  # exact ties among the top experts
        logits[3, :] = -1.0            # every expert tied
    w, sel = oracle_mod.route_topk(logits, k, renorm)
    w32, got_sel, w16 = tris["ext"].route_topk(torch.from_numpy(logits).to(cuda), k, renorm)
    np.testing.assert_array_equal(got_sel.cpu().numpy(), sel)
    np.testing.assert_allclose(w32.cpu().numpy(), w, rtol=2e-6, atol=1e-7)
    got16 = w16.cpu().numpy().view(np.int16).astype(np.int32)
    want16 = w.astype(np.float16).view(np.int16).astype(np.int32)
    assert got16.size == 0 or np.abs(got16 - want16).max() <= 1
    if 0 < t <= 4096:
        route = tris["ext"].build_grouped_route_device(got_sel, e, 4)
        want = oracle_mod.build_route(sel, e, 4)
        for key in ("perm", "grouped_token_indices"):
            np.testing.assert_array_equal(route[key].cpu().numpy(), np.asarray(want[key]), err_msg=key)


def test_route_rejects_bad_expert_ids(tris, cuda):
    note("route bad ids")
    sel = torch.tensor([[0, 9]], dtype=torch.int64, device=cuda)
    with pytest.raises(RuntimeError):
        tris["qlinear"].build_grouped_route(sel, 8)


@pytest.mark.parametrize("t,k,e", [(6, 2, 8), (40, 4, 16)])
def test_route_device_bad_ids_stay_in_bounds(tris, oracle_mod, cuda, t, k, e):
    """The no-sync route with expert ids outside [0, E): counts[0] = -1; the valid picks are routed as the
    oracle routes them alone; the invalid ones fill the rows after every segment in flat order with their own
    token index and slot, grouped expert id -1 and inverse_perm -1; the combine skips them."""
    note(f"route bad ids device t={t} k={k} e={e}")
    rng = np.random.default_rng(t + k)
    sel = np.stack([rng.choice(e, size=k, replace=False) for _ in range(t)]).astype(np.int64)
    bad = rng.random(sel.shape) < 0.2
    bad[0, 0] = True
    sel[bad] = np.where(rng.random(int(bad.sum())) < 0.5, -1, e + 3)
    r = tris["ext"].build_grouped_route_device(torch.from_numpy(sel).to(cuda), e, 4)
    flat = sel.reshape(-1)
    valid = (flat >= 0) & (flat < e)
    nv = int(valid.sum())
    assert int(r["counts"][0]) == -1
    # valid picks: a stable sort by expert, as the oracle's route of the valid entries alone
    order = np.argsort(np.where(valid, flat, e), kind="stable")[:nv]
    perm = r["perm"].cpu().numpy()
    np.testing.assert_array_equal(perm[:nv], order)
    gexp = r["grouped_expert_ids"].cpu().numpy()
    np.testing.assert_array_equal(gexp[:nv], flat[order])
    ids = sorted(set(flat[valid].tolist()))
    np.testing.assert_array_equal(r["expert_ids"].cpu().numpy()[: len(ids)], ids)
    segs = r["segment_offsets"].cpu().numpy()
    counts = [int((flat[valid] == i).sum()) for i in ids]
    np.testing.assert_array_equal(segs[: len(ids) + 1], np.concatenate([[0], np.cumsum(counts)]))
    assert (segs[len(ids):] == nv).all()
    # invalid picks: the tail rows, flat order
    tail = np.nonzero(~valid)[0]
    np.testing.assert_array_equal(perm[nv:], tail)
    np.testing.assert_array_equal(r["grouped_token_indices"].cpu().numpy(), perm // k)
    np.testing.assert_array_equal(r["grouped_slots"].cpu().numpy(), perm % k)
    assert (gexp[nv:] == -1).all()
    inv = r["inverse_perm"].cpu().numpy()
    assert (inv[~valid] == -1).all()
    np.testing.assert_array_equal(perm[inv[valid]], np.nonzero(valid)[0])
    # the combine adds only the valid picks
    hidden = 64
    eo = torch.from_numpy(rng.standard_normal((t * k, hidden)).astype(np.float16)).to(cuda)
    wts = torch.from_numpy(rng.uniform(0.1, 1.0, (t, k)).astype(np.float16)).to(cuda)
    out = tris["ext"].moe_combine(eo, r["inverse_perm"], wts, None).float().cpu().numpy()
    eon, wn = eo.cpu().numpy().astype(np.float32), wts.cpu().numpy()
    want = np.zeros((t, hidden), np.float32)
    for i in np.nonzero(valid)[0]:
        want[i // k] += (eon[inv[i]] * np.float32(wn[i // k, i % k])).astype(np.float16).astype(np.float32)
    np.testing.assert_allclose(out, oracle_mod.bf16_round(want), rtol=0, atol=0)


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("tokens,hidden,experts", [(1, 4096, 8), (16, 4096, 8), (37, 2048, 256), (300, 1024, 60),
                                                   (2048, 4096, 8), (40, 8448, 12)])
def test_router_linear_matches_oracle(tris, oracle_mod, cuda, dtype, tokens, hidden, experts):
    """tris_router_linear (the block's router Linear and fp16 input cast in one launch; rows of more than 8192
    columns take the MFMA tile kernel) against the oracle's router_logits: the model-dtype logits equal the exact sum rounded once except where the fp32 summation
    order decides a rounding tie (a tiny fraction, each one ulp), the fp32 logits are those values widened, and
    x16 is torch's x.to(float16) bit for bit (bf16 model; an fp16 model passes x itself)."""
    note(f"router linear {dtype} T={tokens} H={hidden} E={experts}")
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    rng = np.random.default_rng(tokens * 7 + experts)
    x = torch.from_numpy(rng.standard_normal((tokens, hidden)).astype(np.float32) * 2).to(tdt).to(cuda)
    w = torch.from_numpy((rng.standard_normal((experts, hidden)) / math.sqrt(hidden)).astype(np.float32)).to(tdt)
    w = w.to(cuda)
    logits, logits32, x16 = tris["ext"].router_linear(x, w)
    assert logits.dtype == tdt and logits32.dtype == torch.float32 and x16.dtype == torch.float16
    got = logits.float().cpu().numpy()
    want = oracle_mod.router_logits(x.float().cpu().numpy(), w.float().cpu().numpy(), dtype)
    eq = got == want
    assert (~eq).sum() <= max(1, 0.002 * eq.size), f"{(~eq).sum()} of {eq.size} logits differ"
    # one ulp of the dtype, or (a sum that cancels to a tiny value) a few fp32 ulps of its terms' magnitudes:
    # any fp32 summation order is that far from the exact sum
    l1 = np.abs(x.float().cpu().numpy()).astype(np.float64) @ np.abs(w.float().cpu().numpy()).astype(np.float64).T
    d = ulps(got, want, dtype)
    ok = (d <= 1) | (np.abs(got - want) <= 16 * 2.0 ** -24 * l1)
    worst = np.unravel_index(np.argmax(np.where(ok, 0, d)), d.shape)
    assert ok.all(), f"{d[worst]} ulps at {worst}: got {got[worst]!r} want {want[worst]!r}"
    np.testing.assert_array_equal(logits32.cpu().numpy(), got)
    if dtype == "bf16":
        assert torch.equal(x16.view(torch.int16), x.to(torch.float16).view(torch.int16))
    else:
        assert x16.data_ptr() == x.data_ptr()


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("hidden", [100, 2048, 4096])
def test_combine_gated_shared_expert(tris, oracle_mod, cuda, dtype, hidden):
    """tris_moe_combine_gated against the oracle's gated join (oracle.shared_expert_gate, round_dtype): the
    routed sum in the output dtype plus dt(gate * dt(shared)), the gate's dot product reduced inside each
    workgroup (hidden 4096: two workgroups per token), a ragged hidden size (scalar loads), both dtypes; and
    without the gate, the ungated sum rounded once to the dtype."""
    note(f"combine gated {dtype} hidden={hidden}")
    rng = np.random.default_rng(hidden + (1 if dtype == "bf16" else 2))
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    t, k = 5, 3
    eo = rng.standard_normal((t * k, hidden)).astype(np.float16)
    inv = rng.permutation(t * k).astype(np.int32)
    wts = rng.uniform(0.1, 1.0, (t, k)).astype(np.float16)
    sh = rng.standard_normal((t, hidden)).astype(np.float16)
    x = torch.from_numpy(rng.standard_normal((t, hidden)).astype(np.float32)).to(tdt)
    wg = torch.from_numpy((rng.standard_normal(hidden) * (1.0 / math.sqrt(hidden))).astype(np.float32)).to(tdt)
    dev = lambda a: torch.from_numpy(a).to(cuda)
    got = tris["ext"].moe_combine(dev(eo), dev(inv), dev(wts), dev(sh), shared_gate_input=x.to(cuda),
                                  shared_gate_weight=wg.to(cuda), out_dtype=tdt)
    assert got.dtype == tdt
    routed = np.zeros((t, hidden), np.float32)
    for i in range(t * k):
        routed[i // k] += (eo[inv[i]].astype(np.float32) * np.float32(wts[i // k, i % k])).astype(
            np.float16).astype(np.float32)
    gate = oracle_mod.shared_expert_gate(x.float().numpy(), wg.float().numpy(), dtype)
    assert 0.01 < gate.min() and gate.max() < 0.99  # the data keep the gate away from 0 and 1
    rd = lambda v: oracle_mod.round_dtype(v, dtype)
    want = rd(rd(routed) + rd(gate * rd(sh.astype(np.float32))))
    out = got.float().cpu().numpy()
    assert_close(out, want, f"gated combine {dtype} {hidden}")
    # the gate's fp32 sum runs in another order than the oracle's float64 one: a rounding of the logit may
    # differ near a tie, and then a whole token moves by an ulp; every other value is bit-exact
    assert (out == want).mean() > 0.99
    plain = tris["ext"].moe_combine(dev(eo), dev(inv), dev(wts), dev(sh), out_dtype=tdt).float().cpu().numpy()
    np.testing.assert_array_equal(plain, rd(routed + sh.astype(np.float32)))


# ----------------------------------------------------------- grouped GEMM
def oracle_grouped(oracle_mod, payload, hidden, expert_ids, seg, uniform):
    return oracle_mod.grouped_forward(payload, hidden, expert_ids, seg, uniform)


GEMM_CASES = [
    dict(E=8, n=256, k=512, seg=[1, 0, 1, 0, 0, 0, 0, 0]),              # decode: one row per segment
    dict(E=4, n=192, k=256, seg=[3, 17, 0, 40]),                         # multi-tile segments, an empty one
    dict(E=3, n=100, k=96, seg=[5, 2, 9]),                               # ragged shapes
    dict(E=3, n=128, k=256, seg=[4, 4, 4], scale=True, bias=True),       # epilogue
    dict(E=2, n=128, k=256, seg=[6, 6], g_idx="alternating"),            # non-uniform groups
    dict(E=3, n=200, k=512, seg=[130, 0, 75], scale=True, bias=True, salient_counts=[64, 0, 33]),  # long
]


def _segments(seg_lengths, E, drop=None):
    ids = [e for e in range(E) if seg_lengths[e] > 0]
    offs = np.concatenate([[0], np.cumsum([seg_lengths[e] for e in ids])]).astype(np.int32)
    ids = np.asarray(ids, dtype=np.int32)
    if drop is not None and ids.size:
        ids = ids.copy()
        ids[drop] = -1
    return ids, offs


@pytest.mark.parametrize("case", GEMM_CASES, ids=lambda c: f"E{c['E']}n{c['n']}k{c['k']}" + ("s" if c.get("scale") else ""))
def test_grouped_forward_block_gr(tris, oracle_mod, cuda, case):
    note(f"grouped block_gr {case}")
    case = dict(case)
    g_idx = None
    if case.pop("g_idx", None) == "alternating":
        g_idx = (np.arange(case["k"]) % 2).astype(np.int32)
    seg_len = case.pop("seg")
    payload = make_projection(tris, 41, g_idx=g_idx, **case)
    dev = tris["qlinear"].payload_to_device(payload, cuda)
    ext = tris["ext"]
    rows = int(sum(seg_len))
    rng = np.random.default_rng(3)
    hidden = (rng.standard_normal((rows, case["k"])) * 1.5).astype(np.float16)
    for drop in (None, 0):
        ids, offs = _segments(seg_len, case["E"], drop)
        prob = np.concatenate([[0], np.cumsum((np.diff(offs) + 3) // 4)]).astype(np.int32)
        for uniform in ((False, True) if g_idx is None else (False,)):
            got = ext.compact3_tris_precomputed_grouped_forward_block_gr(
                torch.from_numpy(hidden).to(cuda), t_i32(ids, cuda), t_i32(offs, cuda), t_i32(prob, cuda),
                torch.tensor([int(prob[-1])]), dev["qweight1"], dev["qweight2_sparse"], dev["qweight2_sparse_prefix"],
                dev["q_gmap_gr_words"], dev["q_gmap_gr_offsets"], dev["q_gmap_gr_meta"], dev["c_map"], dev["g_idx"],
                dev["col_pack3"], dev["row_pack3"], dev["output_scale"], dev["has_output_scale"],
                dev["bias"] if dev["has_bias"] else torch.empty(0, device=cuda, dtype=torch.float16),
                dev["has_bias"], uniform).cpu().numpy()
            want = oracle_grouped(oracle_mod, payload, hidden, ids, offs, uniform)
            assert_close(got.astype(np.float32), want.astype(np.float32), f"drop={drop} uniform={uniform}")


def test_dual_and_predecoded_match(tris, oracle_mod, cuda):
    note("dual + predecoded")
    ext = tris["ext"]
    E, k = 4, 256
    pa = make_projection(tris, 51, E, 320, k)
    pb = make_projection(tris, 52, E, 320, k)
    da = tris["qlinear"].payload_to_device(pa, cuda)
    db = tris["qlinear"].payload_to_device(pb, cuda)
    ids, offs = _segments([2, 37, 0, 5], E)
    prob = np.concatenate([[0], np.cumsum((np.diff(offs) + 3) // 4)]).astype(np.int32)
    rng = np.random.default_rng(4)
    rows = int(offs[-1])
    ha = torch.from_numpy((rng.standard_normal((rows, k)) * 1.5).astype(np.float16)).to(cuda)
    hb = torch.from_numpy((rng.standard_normal((rows, k)) * 1.5).astype(np.float16)).to(cuda)
    args = (t_i32(ids, cuda), t_i32(offs, cuda), t_i32(prob, cuda), torch.tensor([int(prob[-1])]))
    empty = torch.empty(0, device=cuda, dtype=torch.float16)

    def single(d, h):
        return ext.compact3_tris_precomputed_grouped_forward_block_gr(
            h, *args, d["qweight1"], d["qweight2_sparse"], d["qweight2_sparse_prefix"], d["q_gmap_gr_words"],
            d["q_gmap_gr_offsets"], d["q_gmap_gr_meta"], d["c_map"], d["g_idx"], d["col_pack3"], d["row_pack3"],
            d["output_scale"], False, empty, False, True)

    oa, ob = ext.compact3_tris_precomputed_grouped_dual_forward_block_gr(
        ha, hb, *args, *[da[x] for x in ("qweight1", "qweight2_sparse", "qweight2_sparse_prefix", "q_gmap_gr_words",
                                         "q_gmap_gr_offsets", "q_gmap_gr_meta", "c_map", "g_idx", "col_pack3",
                                         "row_pack3", "output_scale")], False, empty,
        *[db[x] for x in ("qweight1", "qweight2_sparse", "qweight2_sparse_prefix", "q_gmap_gr_words",
                          "q_gmap_gr_offsets", "q_gmap_gr_meta", "c_map", "g_idx", "col_pack3", "row_pack3",
                          "output_scale")], False, empty, True)
    assert torch.equal(oa, single(da, ha)) and torch.equal(ob, single(db, hb))
    assert_close(oa.cpu().numpy(), oracle_grouped(oracle_mod, pa, ha.cpu().numpy(), ids, offs, True), "dual a")
    assert_close(ob.cpu().numpy(), oracle_grouped(oracle_mod, pb, hb.cpu().numpy(), ids, offs, True), "dual b")
    nblk = tris["synthetic"].packing.num_gr_blocks(k, 320)
    deca = torch.empty((ids.size, nblk, 128), dtype=torch.int32, device=cuda)
    deca = ext.compact3_tris_precomputed_grouped_block_gr_predecode(
        deca, t_i32(ids, cuda), da["q_gmap_gr_words"], da["q_gmap_gr_offsets"], da["q_gmap_gr_meta"], k // 32, 320)
    for uniform in (True, False):  # MFMA kernel / per-weight VALU kernel
        pre = ext.compact3_tris_precomputed_grouped_forward_block_gr_predecoded(
            ha, *args, deca, da["qweight1"], da["qweight2_sparse"], da["qweight2_sparse_prefix"], da["c_map"],
            da["g_idx"], da["col_pack3"], da["row_pack3"], uniform)
        assert_close(pre.cpu().numpy(), oracle_grouped(oracle_mod, pa, ha.cpu().numpy(), ids, offs, True),
                     f"predecoded uniform={uniform}")
    decb = torch.empty((ids.size, nblk, 128), dtype=torch.int32, device=cuda)
    decb = ext.compact3_tris_precomputed_grouped_block_gr_predecode(
        decb, t_i32(ids, cuda), db["q_gmap_gr_words"], db["q_gmap_gr_offsets"], db["q_gmap_gr_meta"], k // 32, 320)
    pa2, pb2 = ext.compact3_tris_precomputed_grouped_dual_forward_block_gr_predecoded(
        ha, hb, *args, deca, *[da[x] for x in ("qweight1", "qweight2_sparse", "qweight2_sparse_prefix", "c_map",
                                               "g_idx", "col_pack3", "row_pack3")],
        decb, *[db[x] for x in ("qweight1", "qweight2_sparse", "qweight2_sparse_prefix", "c_map", "g_idx",
                                "col_pack3", "row_pack3")], True)
    assert_close(pa2.cpu().numpy(), oracle_grouped(oracle_mod, pa, ha.cpu().numpy(), ids, offs, True), "dual pre a")
    assert_close(pb2.cpu().numpy(), oracle_grouped(oracle_mod, pb, hb.cpu().numpy(), ids, offs, True), "dual pre b")


@pytest.mark.parametrize("split", [None, 16], ids=["whole", "split16"])
@pytest.mark.parametrize("rank,n,salient", [(256, 128, None), (512, 192, [0, 40]), (128, 64, [7, 0]),
                                            (512, 136, [64, 17])])
def test_predecoded_mfma_one_hot_is_bit_exact(tris, oracle_mod, cuda, rank, n, salient, split):
    """With one-hot activation rows the MFMA grouped GEMM returns single dequantised weights, which
    must equal the reference's fp16 weights bit for bit: every lane group, packed row, split bit,
    sign and salient column of the operand construction is checked.  Each expert gets `rank` rows (row r
    is e_r), as one segment (long segments: the weight-stationary kernel) or as segments of `split` rows
    of the same expert (the row-tile kernel)."""
    note(f"mfma one-hot rank={rank} n={n} split={split}")
    ext = tris["ext"]
    E = 2
    pay = make_projection(tris, 70 + rank, E, n, rank, salient_counts=salient)
    d = tris["qlinear"].payload_to_device(pay, cuda)
    step = rank if split is None else split
    ids = np.repeat(np.arange(E, dtype=np.int32), ceil_div(rank, step))
    offs = np.concatenate([[0], np.cumsum([min(step, rank - c) for _ in range(E) for c in range(0, rank, step)])])
    offs = offs.astype(np.int32)
    rows = E * rank
    h = np.zeros((rows, rank), dtype=np.float16)
    for e in range(E):
        for r in range(rank):
            h[e * rank + r, r] = 1.0
    hd = torch.from_numpy(h).to(cuda)
    prob = np.concatenate([[0], np.cumsum((np.diff(offs) + 3) // 4)]).astype(np.int32)
    nblk = tris["synthetic"].packing.num_gr_blocks(rank, n)
    dec = torch.empty((ids.size, nblk, 128), dtype=torch.int32, device=cuda)
    ext.compact3_tris_precomputed_grouped_block_gr_predecode(
        dec, t_i32(ids, cuda), d["q_gmap_gr_words"], d["q_gmap_gr_offsets"], d["q_gmap_gr_meta"], rank // 32, n)
    got = ext.compact3_tris_precomputed_grouped_forward_block_gr_predecoded(
        hd, t_i32(ids, cuda), t_i32(offs, cuda), t_i32(prob, cuda), int(prob[-1]), dec, d["qweight1"],
        d["qweight2_sparse"], d["qweight2_sparse_prefix"], d["c_map"], d["g_idx"], d["col_pack3"], d["row_pack3"],
        True).cpu().numpy()
    for e in range(E):
        w = oracle_mod.dequant_grouped_expert(pay, e, True)   # [n, rank] fp16
        np.testing.assert_array_equal(got[e * rank:(e + 1) * rank].view(np.uint16),
                                      w.T.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("drop", [None, 0])
def test_predecoded_long_segments(tris, oracle_mod, cuda, drop):
    """Segments of 64 rows and more (the weight-stationary MFMA kernel): ragged N (a partial output tile),
    rows not a multiple of 16, a full second salient window (64 salient columns) and, with drop=0, a
    segment routed to no expert (zero rows)."""
    note(f"predecoded long segments drop={drop}")
    ext = tris["ext"]
    E, n, k = 3, 200, 512
    pay = make_projection(tris, 81, E, n, k, salient_counts=[64, 0, 33])
    d = tris["qlinear"].payload_to_device(pay, cuda)
    ids, offs = _segments([130, 0, 75], E, drop)
    prob = np.concatenate([[0], np.cumsum((np.diff(offs) + 3) // 4)]).astype(np.int32)
    rng = np.random.default_rng(12)
    rows = int(offs[-1])
    h = (rng.standard_normal((rows, k)) * 1.5).astype(np.float16)
    nblk = tris["synthetic"].packing.num_gr_blocks(k, n)
    dec = torch.empty((ids.size, nblk, 128), dtype=torch.int32, device=cuda)
    ext.compact3_tris_precomputed_grouped_block_gr_predecode(
        dec, t_i32(ids, cuda), d["q_gmap_gr_words"], d["q_gmap_gr_offsets"], d["q_gmap_gr_meta"], k // 32, n)
    got = ext.compact3_tris_precomputed_grouped_forward_block_gr_predecoded(
        torch.from_numpy(h).to(cuda), t_i32(ids, cuda), t_i32(offs, cuda), t_i32(prob, cuda), int(prob[-1]), dec,
        d["qweight1"], d["qweight2_sparse"], d["qweight2_sparse_prefix"], d["c_map"], d["g_idx"], d["col_pack3"],
        d["row_pack3"], True).cpu().numpy()
    want = oracle_grouped(oracle_mod, pay, h, ids, offs, True)
    assert_close(got.astype(np.float32), want.astype(np.float32), f"long segments drop={drop}")
    if drop is not None:
        assert not got[offs[drop]:offs[drop + 1]].any()


@pytest.mark.parametrize("seg", [[3, 21, 0, 9], [90, 150, 0, 70]], ids=["short", "long"])
def test_swiglu_fused_matches_dual_then_silu(tris, oracle_mod, cuda, seg):
    """The fused gate/up GEMM + SwiGLU equals silu(g) * u computed from the dual kernel's own fp16
    outputs with the oracle's fp16 roundings; exp may differ in its last fp32 bit from numpy's,
    so a rare one-ulp difference is allowed.  Long segments run the weight-stationary kernel, whose
    dual outputs are also checked against the oracle."""
    note(f"swiglu fused seg={seg}")
    ext = tris["ext"]
    E, k, n = 4, 256, 320
    pa = make_projection(tris, 61, E, n, k)
    pb = make_projection(tris, 62, E, n, k)
    da = tris["qlinear"].payload_to_device(pa, cuda)
    db = tris["qlinear"].payload_to_device(pb, cuda)
    ids, offs = _segments(seg, E)
    prob = np.concatenate([[0], np.cumsum((np.diff(offs) + 3) // 4)]).astype(np.int32)
    rng = np.random.default_rng(9)
    rows = int(offs[-1])
    ha = torch.from_numpy((rng.standard_normal((rows, k)) * 3).astype(np.float16)).to(cuda)
    hb = torch.from_numpy((rng.standard_normal((rows, k)) * 3).astype(np.float16)).to(cuda)
    args = (t_i32(ids, cuda), t_i32(offs, cuda), t_i32(prob, cuda), int(prob[-1]))
    nblk = tris["synthetic"].packing.num_gr_blocks(k, n)
    dec = []
    for d in (da, db):
        buf = torch.empty((ids.size, nblk, 128), dtype=torch.int32, device=cuda)
        dec.append(ext.compact3_tris_precomputed_grouped_block_gr_predecode(
            buf, t_i32(ids, cuda), d["q_gmap_gr_words"], d["q_gmap_gr_offsets"], d["q_gmap_gr_meta"], k // 32, n))
    names = ("qweight1", "qweight2_sparse", "qweight2_sparse_prefix", "c_map", "g_idx", "col_pack3", "row_pack3")
    g, u = ext.compact3_tris_precomputed_grouped_dual_forward_block_gr_predecoded(
        ha, hb, *args, dec[0], *[da[x] for x in names], dec[1], *[db[x] for x in names], True)
    fused = ext.compact3_tris_precomputed_grouped_swiglu_forward_block_gr_predecoded(
        ha, hb, *args, dec[0], *[da[x] for x in names], dec[1], *[db[x] for x in names]).cpu().numpy()
    g, u = g.cpu().numpy(), u.cpu().numpy()
    assert_close(g, oracle_grouped(oracle_mod, pa, ha.cpu().numpy(), ids, offs, True), "dual gate")
    assert_close(u, oracle_grouped(oracle_mod, pb, hb.cpu().numpy(), ids, offs, True), "dual up")
    want = (oracle_mod.silu_f16(g).astype(np.float32) * u.astype(np.float32)).astype(np.float16)
    ulp = np.abs(fused.view(np.int16).astype(np.int32) - want.view(np.int16).astype(np.int32))
    assert ulp.max() <= 1 and (ulp > 0).mean() < 0.01, (int(ulp.max()), float((ulp > 0).mean()))
    # the standalone act_fn(g) * u kernel gives the fused kernel's bits exactly
    sep = ext.swiglu_mul(torch.from_numpy(g).to(cuda), torch.from_numpy(u).to(cuda)).cpu().numpy()
    np.testing.assert_array_equal(sep.view(np.uint16), fused.view(np.uint16))


def test_swiglu_mul_edge_cases(tris, oracle_mod, cuda):
    """act_fn(g) * u over a ragged length (a 16-byte body and an element-wise tail), zeros, infinities
    and large magnitudes, against the oracle's fp16 roundings (one ulp allowed for exp)."""
    note("swiglu_mul edges")
    ext = tris["ext"]
    rng = np.random.default_rng(31)
    count = 1003
    g = (rng.standard_normal(count) * 6).astype(np.float16)
    u = (rng.standard_normal(count) * 6).astype(np.float16)
    g[:6] = np.array([0.0, -0.0, 60000.0, -60000.0, np.inf, -np.inf], dtype=np.float16)
    u[6:9] = np.array([0.0, 65504.0, -65504.0], dtype=np.float16)
    gt, ut = torch.from_numpy(g).to(cuda), torch.from_numpy(u).to(cuda)
    out = ext.swiglu_mul(gt, ut).cpu().numpy()
    with np.errstate(over="ignore", invalid="ignore"):
        want = (oracle_mod.silu_f16(g).astype(np.float32) * u.astype(np.float32)).astype(np.float16)
    fin = np.isfinite(want)
    np.testing.assert_array_equal(np.isfinite(out), fin)
    ulp = np.abs(out[fin].view(np.int16).astype(np.int32) - want[fin].view(np.int16).astype(np.int32))
    assert ulp.max() <= 1, int(ulp.max())
    assert ext.swiglu_mul(gt[:0], ut[:0]).numel() == 0


def test_run_grouped_structured_api(tris, oracle_mod, cuda):
    """qlinear-level API: route dict, segment-length lists, predecode policy for long segments."""
    note("run_grouped_structured api")
    ql = tris["qlinear"]
    E, k, n = 4, 256, 192
    payload = make_projection(tris, 61, E, n, k)
    dev = ql.payload_to_device(payload, cuda)
    rng = np.random.default_rng(6)
    for lengths in ([1, 0, 1, 0], [70, 80, 0, 90]):
        rows = sum(lengths)
        hidden = torch.from_numpy((rng.standard_normal((rows, k)) * 1.5).astype(np.float16)).to(cuda)
        out = ql.run_grouped_structured_expert_forward(dev, hidden, hidden, lengths)
        ids, offs = _segments(lengths, E)
        want = oracle_grouped(oracle_mod, payload, hidden.cpu().numpy(), ids, offs, True)
        assert_close(out.cpu().numpy(), want, f"lengths={lengths}")
    assert ql.run_grouped_structured_expert_forward(dev, hidden.cpu(), hidden.cpu(), lengths) is None


# ------------------------------------------------------------------ backbone
@pytest.mark.parametrize("tokens,in_f,rank", [(1, 4096, 512), (16, 4096, 512), (5, 14336, 512), (37, 2048, 256),
                                              (4, 1000, 100), (64, 4096, 512), (70, 1001, 48), (300, 4096, 512),
                                              (512, 4096, 512), (1000, 14336, 512), (2048, 4096, 512),
                                              (600, 2048, 256), (4096, 512, 256), (700, 1000, 128),
                                              (520, 1056, 128), (513, 96, 256)])
def test_backbone_matches_fp32(tris, cuda, tokens, in_f, rank, monkeypatch):
    """Decode-sized inputs run the split-K MFMA kernel (1 to 4 token tiles per workgroup: 37 tokens are 3,
    64 are 4, 70 are a group of 4 and a partial one; 1001 columns take the element-wise loads); from
    ext.BACKBONE_GEMM_MIN_ROWS rows with rank a multiple of 128 and in_features of 32 the tiled split-K GEMM
    (partial 256-row tiles, 1 to 16 slices, an odd stage count at K = 1056, one slice that writes fp16 directly
    at K = 96 and K = 512); otherwise from ext.BACKBONE_LIBRARY_MIN_ROWS rows and ext.BACKBONE_LIBRARY_MIN_ELEMS
    activation elements (300 x 4096, and 700 x 1000 columns) the library GEMM.  Gathered rows past the token
    count project the tokens, then gather."""
    note(f"backbone T={tokens} in={in_f} rank={rank}")
    # the layer sends a shape to the tiled GEMM only when its launch fills the GPU; here every eligible shape goes
    monkeypatch.setattr(tris["ext"], "BACKBONE_GEMM_MIN_WORKGROUPS", 1)
    rng = np.random.default_rng(tokens + in_f)
    x = rng.standard_normal((tokens, in_f)).astype(np.float16)
    sv = (rng.standard_normal((rank, in_f)) * 0.02).astype(np.float16)
    want = (x.astype(np.float32) @ sv.astype(np.float32).T).astype(np.float16)
    xt, st = torch.from_numpy(x).to(cuda), torch.from_numpy(sv).to(cuda)
    first = tris["ext"].backbone_linear(xt, st)
    assert_close(first.cpu().numpy(), want, "backbone")
    assert torch.equal(tris["ext"].backbone_linear(xt, st), first)  # deterministic
    idx = torch.from_numpy(rng.integers(0, tokens, 2 * tokens)).to(cuda)
    got = tris["ext"].backbone_linear(xt, st, row_index=idx)
    assert_close(got.cpu().numpy(), want[idx.cpu().numpy()], "backbone gathered")
    if in_f % 8 == 0:
        sv2 = torch.from_numpy((rng.standard_normal((rank, in_f)) * 0.02).astype(np.float16)).to(cuda)
        pa, pb = tris["ext"].backbone_linear_pair(xt, st, sv2, row_index=idx)
        assert torch.equal(pa, got) and torch.equal(pb, tris["ext"].backbone_linear(xt, sv2, row_index=idx))
    if in_f % 8 == 0:
        s = rng.uniform(0.5, 1.5, in_f).astype(np.float16)
        xs = (x.astype(np.float32) * s.astype(np.float32)).astype(np.float16)
        want_s = (xs.astype(np.float32) @ sv.astype(np.float32).T).astype(np.float16)
        got = tris["ext"].backbone_linear(xt, st, in_scale=torch.from_numpy(s).to(cuda)).cpu().numpy()
        assert_close(got, want_s, "backbone scaled")


# --------------------------------------------------------------------- layer
def _run_layer(tris, oracle_mod, cuda, spec, tokens, seed, expert_path="auto", steps=None):
    """The layer on `steps` independent batches of `tokens` (each its own forward call), outputs and oracle
    outputs concatenated.  Single-token cases take four steps: the bf16 output of one token is 4096 values, and
    rel-L2 over so few is dominated by a handful of whole-ulp flips that any fp32-accumulating evaluation makes
    (measured: two fp32 orders of the oracle itself differ by up to 1.2e-3 on one token, ~8e-4 on average)."""
    syn = tris["synthetic"]
    ql = tris["qlinear"]
    steps = steps if steps is not None else (4 if tokens == 1 else 1)
    layer = syn.make_layer(spec, seed, tris["ext"].gr_encode)
    payloads = {p: ql.payload_to_device(layer[p], cuda) for p in ("gate", "up", "down")}
    backbones = {p: torch.from_numpy(layer["backbones"][p]).to(cuda) for p in ("gate", "up", "down")}
    shared = gate_w = None
    if "shared_expert" in layer:
        shared = tuple(torch.from_numpy(w).to(cuda) for w in layer["shared_expert"])
        gate_w = torch.from_numpy(layer["shared_expert_gate"]).to(cuda).to(torch.bfloat16)
    block = tris["moe"].TrisSparseMoeBlock(spec.hidden, spec.num_experts, spec.top_k, payloads, backbones,
                                           renormalize=spec.renormalize, shared_expert=shared,
                                           shared_expert_gate=gate_w)
    caches = {"gate": {}, "up": {}, "down": {}}
    outs, wants = [], []
    for i in range(steps):
        inp = syn.make_inputs(spec, tokens, seed + 1 + i, layer["outlier_idx"])
        x = torch.from_numpy(inp["x"]).to(cuda).to(torch.bfloat16)
        logits = torch.from_numpy(inp["router_logits"]).to(cuda)
        if expert_path == "auto":
            out = block.forward_routed(x, logits).float().cpu().numpy()
        else:
            wt, st = tris["moe"].route_topk(logits, spec.top_k, spec.renormalize)
            sh = (*shared, gate_w) if shared is not None else None
            out = tris["moe"].grouped_moe_forward(x.to(torch.float16), wt, st, payloads, backbones, spec.num_experts,
                                                  torch.bfloat16, sh, expert_path=expert_path,
                                                  x_model=x).float().cpu().numpy()
        w, sel = oracle_mod.route_topk(inp["router_logits"], spec.top_k, spec.renormalize)
        want = oracle_mod.moe_layer(inp["x"].astype(np.float16), w, sel, {p: layer[p] for p in ("gate", "up", "down")},
                                    layer["backbones"], spec.num_experts, layer.get("shared_expert"),
                                    weight_caches=caches, shared_gate=layer.get("shared_expert_gate"),
                                    x_model=inp["x"], out_dtype="bf16")
        outs.append(out)
        wants.append(oracle_mod.bf16_round(want))
    return np.concatenate(outs), np.concatenate(wants)


def test_layer_a3b_c3_shared_expert_in_own_launches(tris, oracle_mod, cuda, monkeypatch):
    """C3 at T = 1 with the shared expert in launches of its own (moe.FOLD_SHARED_EXPERT off): the path the block
    takes when its weights do not stack; the default runs it as extra columns of the routed launches."""
    from tris_moe_amd.configs import C3_A3B

    note("layer C3 A3B T=1, shared expert unfolded")
    monkeypatch.setattr(tris["moe"], "FOLD_SHARED_EXPERT", False)
    out, want = _run_layer(tris, oracle_mod, cuda, C3_A3B, 1, 3001)
    assert_close(out, want, "C3 layer T=1 (shared expert unfolded)")


@pytest.mark.parametrize("tokens", [1, 3, 20])
def test_layer_ungated_shared_expert_in_routed_launches(tris, oracle_mod, cuda, tokens):
    """A smaller A3B-shaped layer (1024 hidden, 32 experts, top-8) with an ungated shared expert (the three weights,
    no gate: final + shared(h)), run through the block, so its shared expert rides in the routed launches
    (SharedExpertStack: at T = 20, 160 routed rows, its down projection runs apart), against the oracle."""
    from tris_moe_amd.configs import C3_A3B

    spec = C3_A3B.with_(name="a3b_small", hidden=1024, num_experts=32)
    note(f"layer with an ungated shared expert in the routed launches T={tokens}")
    syn, ql, moe = tris["synthetic"], tris["qlinear"], tris["moe"]
    layer = syn.make_layer(spec, 3300 + tokens, tris["ext"].gr_encode)
    payloads = {p: ql.payload_to_device(layer[p], cuda) for p in ("gate", "up", "down")}
    backbones = {p: torch.from_numpy(layer["backbones"][p]).to(cuda) for p in ("gate", "up", "down")}
    shared = tuple(torch.from_numpy(w).to(cuda) for w in layer["shared_expert"])
    block = moe.TrisSparseMoeBlock(spec.hidden, spec.num_experts, spec.top_k, payloads, backbones,
                                   renormalize=spec.renormalize, shared_expert=shared)
    assert block.shared_stack is not None
    outs, wants = [], []
    for i in range(4):
        inp = syn.make_inputs(spec, tokens, 3400 + 10 * tokens + i, layer["outlier_idx"])
        x = torch.from_numpy(inp["x"]).to(cuda).to(torch.bfloat16)
        logits = torch.from_numpy(inp["router_logits"]).to(cuda)
        outs.append(block.forward_routed(x, logits).float().cpu().numpy())
        w, sel = oracle_mod.route_topk(inp["router_logits"], spec.top_k, spec.renormalize)
        want = oracle_mod.moe_layer(inp["x"].astype(np.float16), w, sel, {p: layer[p] for p in ("gate", "up", "down")},
                                    layer["backbones"], spec.num_experts, layer["shared_expert"], out_dtype="bf16")
        wants.append(oracle_mod.bf16_round(want))
    assert_close(np.concatenate(outs), np.concatenate(wants), f"ungated shared expert layer T={tokens}")


def test_layer_olmoe_c0(tris, oracle_mod, cuda):
    from tris_moe_amd.configs import C0_OLMOE

    note("layer C0 OLMoE T=16")
    out, want = _run_layer(tris, oracle_mod, cuda, C0_OLMOE, 16, 1000)
    assert_close(out, want, "C0 layer")


@pytest.mark.parametrize("tokens,path", [(1, "auto"), (4, "auto"), (16, "predecoded"), (4, "fused")])
def test_layer_mixtral_c1_decode(tris, oracle_mod, cuda, tokens, path):
    from tris_moe_amd.configs import C1_MIXTRAL_DECODE

    note(f"layer C1 Mixtral T={tokens} path={path}")
    out, want = _run_layer(tris, oracle_mod, cuda, C1_MIXTRAL_DECODE, tokens, 2000 + tokens, path)
    assert_close(out, want, f"C1 layer T={tokens} {path}")


@pytest.mark.parametrize("tokens", [160, 512, 2048])
def test_layer_mixtral_prefill_shape(tris, oracle_mod, cuda, tokens):
    """C2's layer shape at 160 tokens (320 routed rows: multi-tile segments, the row-tile MFMA kernel),
    512 tokens (about 128 rows per expert: the weight-stationary kernel) and C2 itself (2048 tokens, N(0, 1)
    router logits: the histogram / scatter route over 4096 routed rows), with the library GEMM for the
    backbones."""
    from tris_moe_amd.configs import C2_MIXTRAL_PREFILL

    note(f"layer C2 Mixtral prefill shape T={tokens}")
    out, want = _run_layer(tris, oracle_mod, cuda, C2_MIXTRAL_PREFILL, tokens, 4000 + tokens)
    assert_close(out, want, f"C2-shape layer T={tokens}")


@pytest.mark.parametrize("tokens", [1, 32, 1024])
def test_layer_a3b_c3_with_shared_expert(tris, oracle_mod, cuda, tokens):
    """C3: 256 experts, top-8, an always-on fp16 shared expert joined through its
    sigmoid gate (modeling_qwen2_moe.py:815-818), N(0, 1.5) router logits, at its three batches (1024 tokens:
    8192 routed rows over nearly every expert)."""
    from tris_moe_amd.configs import C3_A3B

    note(f"layer C3 A3B T={tokens}")
    out, want = _run_layer(tris, oracle_mod, cuda, C3_A3B, tokens, 3000 + tokens)
    assert_close(out, want, f"C3 layer T={tokens}")
