"""Non-expert compact3 linears (compact3_linear_forward / _dual_ / _qkv_, TriSMoE_cuda.cpp:497-700,
kernel.cu:2146-3744 and 10781-11740): the oracle's composition on the CPU, and on the GPU the single, dual
and Q/K/V bindings against the oracle, with input and output scales, bias, the matrix-mode null-space
term, and ragged batches."""
import numpy as np
import pytest
import torch

from tris_moe_amd import synthetic
from tris_moe_amd.packing import pack_4bit

MODULE_KEYS = ("qweight1", "qweight2_sparse", "qweight2_sparse_prefix", "q_gmap_gr_words", "q_gmap_gr_offsets",
               "q_gmap_gr_meta", "c_map", "g_idx", "col_pack3", "row_pack3")


def _modules(ext, count, n, k, seed):
    """count one-matrix modules (a synthetic projection's experts, each without its expert dimension)."""
    rng = np.random.default_rng(seed)
    col_norm = rng.random(k).astype(np.float32) + 0.5
    proj = synthetic.make_projection(rng, count, n, k, 0.15, col_norm, ext.gr_encode)
    return [{key: np.ascontiguousarray(proj[key][e]) for key in MODULE_KEYS} for e in range(count)], rng


def _ns(rng, n, k, ns_rank, gs):
    c2 = pack_4bit(rng.standard_normal((ns_rank, k)).astype(np.float32) * 0.05, gs)
    c1 = pack_4bit(rng.standard_normal((n, ns_rank)).astype(np.float32) * 0.05, min(ns_rank, gs))
    return c2, c1


def test_oracle_linear_is_the_composition(oracle_mod, tris):
    """oracle.compact3_linear against the same products taken by torch on the CPU: (x' W^T + C1 (C2 x)) *
    output_scale + bias in fp32, one rounding; without extras it is the grouped oracle over one segment.
    Two plausible slips (the null-space term after the output scale; the input scale applied to the term's
    input too) give other bits on this data, so the check sees them."""
    import torch.nn.functional as F

    mods, rng = _modules(tris["ext"], 1, 96, 128, 5)
    m = mods[0]
    x = (rng.standard_normal((6, 128)) * 2).astype(np.float16)
    s_in = (rng.random(128) + 0.5).astype(np.float16)
    s_out = (rng.random(96) * 2 + 0.25).astype(np.float16)
    bias = rng.standard_normal(96).astype(np.float16)
    c2p, c1p = _ns(rng, 96, 128, 16, 32)
    c2 = oracle_mod.packed4_dequant(c2p["qweight"], c2p["qzeros"], c2p["scales"], c2p["g_idx"], 16, 128)
    c1 = oracle_mod.packed4_dequant(c1p["qweight"], c1p["qzeros"], c1p["scales"], c1p["g_idx"], 96, 16)
    got = oracle_mod.compact3_linear(x, m, s_in, s_out, bias, c2, c1)
    w = torch.from_numpy(oracle_mod.dequant_grouped_expert(oracle_mod.module_as_payload(m), 0)).float()
    xt, xs = torch.from_numpy(x).float(), (torch.from_numpy(x) * torch.from_numpy(s_in)).float()
    ns = F.linear(F.linear(xt, torch.from_numpy(c2).float()), torch.from_numpy(c1).float())
    want = ((F.linear(xs, w) + ns) * torch.from_numpy(s_out).float() + torch.from_numpy(bias).float()).half().numpy()
    np.testing.assert_array_equal(got, want)
    slip1 = ((F.linear(xs, w) * torch.from_numpy(s_out).float() + ns) + torch.from_numpy(bias).float()).half().numpy()
    ns2 = F.linear(F.linear(xs, torch.from_numpy(c2).float()), torch.from_numpy(c1).float())
    slip2 = ((F.linear(xs, w) + ns2) * torch.from_numpy(s_out).float() + torch.from_numpy(bias).float()).half().numpy()
    assert not np.array_equal(slip1, want) and not np.array_equal(slip2, want)
    plain = oracle_mod.compact3_linear(x, m)
    grouped = oracle_mod.grouped_forward(oracle_mod.module_as_payload(m), x, np.asarray([0]), np.asarray([0, 6]))
    np.testing.assert_array_equal(plain, grouped)


# ------------------------------------------------------------------------------------------------ GPU
def _dev(mod, cuda):
    return {k: torch.from_numpy(v).to(cuda) for k, v in mod.items()}


def _linear(ext, x, m, s_in=None, s_out=None, bias=None, ns=None):
    empty = x.new_empty((0,))
    ns_args = ([ns[1]["qweight"], ns[1]["qzeros"], ns[1]["scales"], ns[1]["g_idx"], ns[0]["qweight"],
                ns[0]["qzeros"], ns[0]["scales"], ns[0]["g_idx"], True] if ns is not None else [empty] * 8 + [False])
    return ext.compact3_linear_forward(
        x, m["qweight1"], m["qweight2_sparse"], m["qweight2_sparse_prefix"], empty, empty, m["q_gmap_gr_words"],
        m["q_gmap_gr_offsets"], m["q_gmap_gr_meta"], m["c_map"], m["g_idx"], m["col_pack3"], m["row_pack3"],
        s_in if s_in is not None else empty, s_out if s_out is not None else empty,
        bias if bias is not None else empty, s_in is not None, s_out is not None, bias is not None, *ns_args, 1, False)


@pytest.mark.gpu
@pytest.mark.parametrize("batch", [1, 7, 70])
@pytest.mark.parametrize("extras", ["plain", "scales_bias", "ns"])
def test_linear_matches_oracle(tris, oracle_mod, cuda, batch, extras):
    """compact3_linear_forward: one row, a ragged tile and several tiles; no extras, input / output scales
    with bias, and all of them with a null-space term (act-order-free groups of 32 and 16)."""
    from test_gpu_parity import assert_close, note

    note(f"compact3 linear batch={batch} extras={extras}")
    ext = tris["ext"]
    n, k = 200, 192
    mods, rng = _modules(ext, 1, n, k, 40 + batch)
    m = mods[0]
    x = (rng.standard_normal((batch, k)) * 1.5).astype(np.float16)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    s_in = s_out = bias = ns = None
    c2 = c1 = None
    if extras != "plain":
        s_in = (rng.random(k) + 0.5).astype(np.float16)
        s_out = (rng.random(n) * 2 + 0.25).astype(np.float16)
        bias = rng.standard_normal(n).astype(np.float16)
    if extras == "ns":
        c2p, c1p = _ns(rng, n, k, 24, 32)
        c2 = oracle_mod.packed4_dequant(c2p["qweight"], c2p["qzeros"], c2p["scales"], c2p["g_idx"], 24, k)
        c1 = oracle_mod.packed4_dequant(c1p["qweight"], c1p["qzeros"], c1p["scales"], c1p["g_idx"], n, 24)
        ns = ({kk: t(v) for kk, v in c2p.items()}, {kk: t(v) for kk, v in c1p.items()})
    got = _linear(ext, t(x), _dev(m, cuda), *(t(a) if a is not None else None for a in (s_in, s_out, bias)), ns=ns)
    want = oracle_mod.compact3_linear(x, m, s_in, s_out, bias, c2, c1)
    assert_close(got.cpu().numpy(), want, f"compact3_linear_forward {extras}")


@pytest.mark.gpu
def test_dual_and_qkv_match_single_calls(tris, oracle_mod, cuda):
    """compact3_dual_linear_forward and compact3_qkv_linear_forward (with biases): the bits of single calls,
    within tolerance of the oracle; a sparse-format payload is refused with a message."""
    from test_gpu_parity import assert_close, note

    note("compact3 dual / qkv")
    ext = tris["ext"]
    n, k, batch = 128, 256, 9
    mods, rng = _modules(ext, 3, n, k, 77)
    dm = [_dev(m, cuda) for m in mods]
    x = torch.from_numpy((rng.standard_normal((batch, k)) * 1.5).astype(np.float16)).to(cuda)
    args = lambda m: [m[key] for key in MODULE_KEYS]
    dual = ext.compact3_dual_linear_forward(x, *args(dm[0]), *args(dm[1]), 1, False)
    for i in range(2):
        assert torch.equal(dual[i], _linear(ext, x, dm[i]))
        assert_close(dual[i].cpu().numpy(), oracle_mod.compact3_linear(x.cpu().numpy(), mods[i]), f"dual[{i}]")
    biases = [torch.from_numpy(rng.standard_normal(n).astype(np.float16)).to(cuda) for _ in range(3)]
    qkv = ext.compact3_qkv_linear_forward(x, *args(dm[0]), biases[0], *args(dm[1]), biases[1], *args(dm[2]), biases[2],
                                          1, False)
    for i in range(3):
        assert torch.equal(qkv[i], _linear(ext, x, dm[i], bias=biases[i]))
        want = oracle_mod.compact3_linear(x.cpu().numpy(), mods[i], bias=biases[i].cpu().numpy())
        assert_close(qkv[i].cpu().numpy(), want, f"qkv[{i}]")
    sparse = dict(dm[0], q_gmap_gr_offsets=dm[0]["q_gmap_gr_offsets"][:-1])
    with pytest.raises(RuntimeError, match="block-GR"):
        _linear(ext, x, sparse)


@pytest.mark.gpu
def test_module_and_fused_runners(tris, oracle_mod, cuda):
    """qlinear.Compact3Linear (mode-4 QuantLinear) with every extra, and the Q/K/V and shared-expert gate/up
    runners: the bits of the modules run one by one; a module with scales is left to the caller (None)."""
    from test_gpu_parity import assert_close, note

    note("Compact3Linear module and fused runners")
    ext, ql = tris["ext"], tris["qlinear"]
    n, k = 160, 128
    mods, rng = _modules(ext, 3, n, k, 91)
    c2p, c1p = _ns(rng, n, k, 16, 32)
    full = ql.Compact3Linear(k, n).load_tensors(dict(mods[0], input_scale=(rng.random(k) + 0.5).astype(np.float16),
                                                     output_scale=(rng.random(n) + 0.5).astype(np.float16),
                                                     bias=rng.standard_normal(n).astype(np.float16),
                                                     ns_c1=c1p, ns_c2=c2p)).to(cuda)
    x = torch.from_numpy((rng.standard_normal((2, 3, k)) * 1.5).astype(np.float16)).to(cuda)
    y = full(x)
    assert y.shape == (2, 3, n)
    c2 = oracle_mod.packed4_dequant(c2p["qweight"], c2p["qzeros"], c2p["scales"], c2p["g_idx"], 16, k)
    c1 = oracle_mod.packed4_dequant(c1p["qweight"], c1p["qzeros"], c1p["scales"], c1p["g_idx"], n, 16)
    want = oracle_mod.compact3_linear(x.reshape(-1, k).cpu().numpy(), mods[0], full.input_scale.cpu().numpy(),
                                      full.output_scale.cpu().numpy(), full.bias.cpu().numpy(), c2, c1)
    assert_close(y.reshape(-1, n).cpu().numpy(), want, "Compact3Linear")
    plain = [ql.Compact3Linear(k, n).load_tensors(dict(m, bias=rng.standard_normal(n).astype(np.float16))).to(cuda)
             for m in mods]
    q, kk, v = ql.run_compact3_qkv_block_gr_forward(*plain, x)
    for got, m in zip((q, kk, v), plain):
        assert torch.equal(got, m(x))
    nobias = [ql.Compact3Linear(k, n).load_tensors(m).to(cuda) for m in mods[:2]]
    g, u = ql.run_compact3_shared_expert_gate_up_forward(*nobias, x)
    assert torch.equal(g, nobias[0](x)) and torch.equal(u, nobias[1](x))
    assert ql.run_compact3_qkv_block_gr_forward(full, plain[1], plain[2], x) is None
