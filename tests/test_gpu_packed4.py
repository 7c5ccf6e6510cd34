"""GPU parity of the 4-bit packed backbone (PackedQuantMatrix4bit, qlinear_cuda.py:2637-2786): dequantised
weights bit-exact against the oracle; projections within max-abs 2e-2 / rel-L2 1e-3 of the fp32-accumulated
product of those weights; a Mixtral layer with packed backbones against the oracle layer."""
import numpy as np
import pytest
import torch

from test_gpu_parity import assert_close, note

pytestmark = pytest.mark.gpu


def _quantised(oracle_mod, rows, cols, group, seed, act_order=False):
    """A packed payload of a random matrix (GPTQ-style asymmetric 4-bit, the producer
    utils/pack_utils.py:126-180) and its exact fp16 dequantisation."""
    rng = np.random.default_rng(seed)
    m = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
    g_idx = (np.arange(cols) // group).astype(np.int32)
    if act_order:
        g_idx = g_idx[rng.permutation(cols)]
    G = int(g_idx.max()) + 1
    lo = np.minimum(np.stack([m[:, g_idx == g].min(axis=1) for g in range(G)]), -1e-3)
    hi = np.maximum(np.stack([m[:, g_idx == g].max(axis=1) for g in range(G)]), 1e-3)
    scale = ((hi - lo) / 15.0).astype(np.float16).astype(np.float32)
    zero = np.round(-lo / scale)
    pl = oracle_mod.packed4_build_payload(m, scale, zero, g_idx)
    w = oracle_mod.packed4_dequant(pl["qweight"], pl["qzeros"], pl["scales"], pl["g_idx"], rows, cols)
    return pl, w


def _module(tris, pl, dev):
    m = tris["qlinear"].PackedQuantMatrix4bit()
    m.set_quantized(pl["qweight"], pl["qzeros"], pl["scales"], pl["g_idx"], pl["rows"], pl["cols"])
    return m.to(dev)


@pytest.mark.parametrize("rows,cols,group,act", [(512, 4096, 128, False), (37, 90, 16, False), (64, 200, 32, True),
                                                 (8, 8, 8, False)])
def test_dequant_bit_exact(tris, oracle_mod, cuda, rows, cols, group, act):
    note(f"packed4 dequant {rows}x{cols} g{group} act={act}")
    pl, want = _quantised(oracle_mod, rows, cols, group, 11 + rows, act)
    m = _module(tris, pl, cuda)
    got = m.dequantize(cuda, torch.float16).cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("tokens,cols,rows,gather,scaled", [(1, 4096, 512, False, False), (16, 4096, 512, True, False),
                                                            (5, 14336, 512, True, True), (3, 200, 40, False, False),
                                                            (300, 4096, 512, True, False)])
def test_projection_matches_fp32(tris, oracle_mod, cuda, tokens, cols, rows, gather, scaled):
    """Fused kernel (uniform groups, < 256 rows) or the cached dequantised matrix on the library GEMM (>= 256
    rows): x[row_index] (* in_scale) . W^T against the fp32 product of the oracle's fp16 weights."""
    note(f"packed4 projection T={tokens} {cols}->{rows} gather={gather} scaled={scaled}")
    pl, w = _quantised(oracle_mod, rows, cols, 8 if cols == 200 else 128, 5 + tokens)
    m = _module(tris, pl, cuda)
    rng = np.random.default_rng(tokens)
    src = 7 if gather else tokens
    x = (rng.standard_normal((src, cols)) * 2).astype(np.float16)
    idx = rng.integers(0, src, tokens).astype(np.int64) if gather else None
    s = (rng.random(cols) + 0.5).astype(np.float16) if scaled else None
    got = m.project(torch.from_numpy(x).to(cuda), in_scale=None if s is None else torch.from_numpy(s).to(cuda),
                    row_index=None if idx is None else torch.from_numpy(idx).to(cuda)).cpu().numpy()
    xs = x[idx] if gather else x
    if scaled:
        xs = (xs.astype(np.float32) * s.astype(np.float32)).astype(np.float16)
    want = oracle_mod.linear_f16(xs, w)
    assert_close(got, want, "packed4 projection")


def test_pair_and_reference_entry(tris, oracle_mod, cuda):
    """The gate/up pair in one launch gives the bits of two single calls; packed4_linear_forward (the
    reference's extension signature) takes the fused kernel for uniform groups and the dequantised fp16 path
    for act-order groups, both within tolerance."""
    note("packed4 pair + packed4_linear_forward")
    ql, ext = tris["qlinear"], tris["ext"]
    pa, wa = _quantised(oracle_mod, 512, 4096, 128, 1)
    pb, wb = _quantised(oracle_mod, 512, 4096, 128, 2)
    ma, mb = _module(tris, pa, cuda), _module(tris, pb, cuda)
    rng = np.random.default_rng(3)
    x = torch.from_numpy(rng.standard_normal((6, 4096)).astype(np.float16)).to(cuda)
    idx = torch.tensor([5, 0, 0, 3, 1, 2, 4, 5], dtype=torch.int64, device=cuda)
    ga, gb = ql.shared_projection_pair(x, ma, mb, row_index=idx)
    assert torch.equal(ga, ma.project(x, row_index=idx)) and torch.equal(gb, mb.project(x, row_index=idx))
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    out = ext.packed4_linear_forward(x, t(pa["qweight"]), t(pa["qzeros"]), t(pa["scales"]), t(pa["g_idx"]))
    assert_close(out.cpu().numpy(), oracle_mod.linear_f16(x.cpu().numpy(), wa), "packed4_linear_forward uniform")
    pc, wc = _quantised(oracle_mod, 96, 256, 32, 4, act_order=True)
    xc = torch.from_numpy(rng.standard_normal((3, 256)).astype(np.float16)).to(cuda)
    out = ext.packed4_linear_forward(xc, t(pc["qweight"]), t(pc["qzeros"]), t(pc["scales"]), t(pc["g_idx"]))
    assert_close(out.cpu().numpy(), oracle_mod.linear_f16(xc.cpu().numpy(), wc), "packed4_linear_forward act order")


@pytest.mark.parametrize("tokens", [4, 16])
def test_layer_mixtral_packed_backbones(tris, oracle_mod, cuda, tokens):
    """C1's layer with every backbone a 4-bit packed matrix (group 128): the decode path through the fused
    packed projections against the oracle layer on the dequantised backbones."""
    from tris_moe_amd.configs import C1_MIXTRAL_DECODE as spec

    note(f"layer C1 packed backbones T={tokens}")
    syn, ql = tris["synthetic"], tris["qlinear"]
    layer = syn.make_layer(spec, 6000 + tokens, tris["ext"].gr_encode)
    inp = syn.make_inputs(spec, tokens, 6001 + tokens, layer["outlier_idx"])
    payloads = {p: ql.payload_to_device(layer[p], cuda) for p in ("gate", "up", "down")}
    backbones, deq = {}, {}
    for i, p in enumerate(("gate", "up", "down")):
        sv = layer["backbones"][p].astype(np.float32)
        rows, cols = sv.shape
        g_idx = (np.arange(cols) // 128).astype(np.int32)
        G = cols // 128
        lo = np.minimum(sv.reshape(rows, G, 128).min(axis=2).T, -1e-3)
        hi = np.maximum(sv.reshape(rows, G, 128).max(axis=2).T, 1e-3)
        scale = ((hi - lo) / 15.0).astype(np.float16).astype(np.float32)
        pl = oracle_mod.packed4_build_payload(sv, scale, np.round(-lo / scale), g_idx)
        deq[p] = oracle_mod.packed4_dequant(pl["qweight"], pl["qzeros"], pl["scales"], pl["g_idx"], rows, cols)
        backbones[p] = _module(tris, pl, cuda)
    block = tris["moe"].TrisSparseMoeBlock(spec.hidden, spec.num_experts, spec.top_k, payloads, backbones,
                                           renormalize=spec.renormalize)
    x = torch.from_numpy(inp["x"]).to(cuda).to(torch.bfloat16)
    out = block.forward_routed(x, torch.from_numpy(inp["router_logits"]).to(cuda)).float().cpu().numpy()
    w, sel = oracle_mod.route_topk(inp["router_logits"], spec.top_k, spec.renormalize)
    want = oracle_mod.moe_layer(inp["x"].astype(np.float16), w, sel, {p: layer[p] for p in ("gate", "up", "down")},
                                deq, spec.num_experts)
    assert_close(out, oracle_mod.bf16_round(want), f"C1 packed backbones T={tokens}")
