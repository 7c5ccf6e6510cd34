"""Grouped payload checkpoints (tris_moe_amd.checkpoint): the reference's safetensors key scheme and scalar
encoding (grouped_payload_sidecar.py:18-135, 172-193), its load-time repair (:248-337), sparse-bitmap payloads
converted to block-GR, shared backbones (fp16 and 4-bit packed); on the GPU a layer loaded from a checkpoint
gives the bits of the same layer built in memory."""
import numpy as np
import pytest
import torch

from tris_moe_amd import checkpoint as ck
from tris_moe_amd.configs import MoELayerSpec

TINY = MoELayerSpec("tiny", hidden=256, num_experts=4, intermediate=384, top_k=2, rank=128, tokens=(3,))


def _input_scales(n):
    """ns_mode 1 input scales for layer 1's gate and down projections (layer 0 has none)."""
    rng = np.random.default_rng(77)
    return [None] + [{"gate": rng.uniform(0.5, 1.5, TINY.hidden).astype(np.float16),
                      "down": rng.uniform(0.5, 1.5, TINY.intermediate).astype(np.float16)}] * (n - 1)


def _save(tris, tmp_path, n=2, packed_down=False, family="mixtral", input_scales=None):
    layers = [tris["synthetic"].make_layer(TINY, 100 + i, tris["ext"].gr_encode) for i in range(n)]
    bbs = []
    for L in layers:
        bb = dict(L["backbones"])
        if packed_down:
            from tris_moe_amd.packing import pack_4bit
            bb["down"] = pack_4bit(bb["down"].astype(np.float32), 64)
        bbs.append(bb)
    path = str(tmp_path / ck.GROUPED_PAYLOAD_SIDECAR_BASENAME)
    ck.save_grouped_checkpoint(path, [{p: L[p] for p in ck.GROUPED_PRECOMPUTED_KEYS} for L in layers], family,
                               bbs, metadata={"model": "tiny"}, input_scales=input_scales)
    return path, layers, bbs


def test_key_scheme_and_scalars(tris, tmp_path):
    from safetensors import safe_open

    path, layers, _ = _save(tris, tmp_path)
    with safe_open(path, framework="pt") as f:
        keys = set(f.keys())
        meta = f.metadata()
        assert meta["format"] == "olmoe_grouped_runtime_payload_v1" and meta["model"] == "tiny"
        assert "model.layers.0.block_sparse_moe.grouped_payload.gate.qweight1" in keys
        assert "model.layers.1.block_sparse_moe.grouped_payload.down.q_gmap_gr_words" in keys
        assert "model.layers.0.TriS_shared_up_proj.shared_sv" in keys
        assert not any(k.split(".")[-1].startswith("_") for k in keys)   # derived caches stay out
        t = f.get_tensor("model.layers.0.block_sparse_moe.grouped_payload.gate.is_compact3")
        assert t.dtype == torch.bool and tuple(t.shape) == (1,) and bool(t[0])
        assert f.get_tensor("model.layers.0.block_sparse_moe.grouped_payload.gate.bias").numel() == 0
    assert ck.split_payload_tensor_name("model.layers.3.mlp.grouped_payload.up_ns.ns_c1_qweight") == \
        ("model.layers.3.mlp", "up_ns", "ns_c1_qweight")
    assert ck.split_payload_tensor_name("model.layers.3.mlp.experts.0.w1") is None
    assert ck.moe_layer_prefix(5, "olmoe") == "model.layers.5.mlp"


def test_round_trip_on_host(tris, tmp_path):
    path, layers, bbs = _save(tris, tmp_path, packed_down=True)
    c = ck.GroupedCheckpoint(path)
    assert c.compatibility() == (True, None)
    assert c.layer_prefixes() == ["model.layers.0.block_sparse_moe", "model.layers.1.block_sparse_moe"]
    for i, lp in enumerate(c.layer_prefixes()):
        got = c.load_layer(lp, "cpu")
        for proj in ck.GROUPED_PRECOMPUTED_KEYS:
            want = layers[i][proj]
            for key, val in want.items():
                if key == "gmap_dense":
                    continue
                if isinstance(val, np.ndarray):
                    np.testing.assert_array_equal(got[proj][key].numpy(), val, err_msg=f"{lp} {proj} {key}")
                else:
                    assert got[proj][key] == val, (proj, key)
        host = c.load_layer_numpy(lp)   # the host form the streaming loader packs
        for proj in ck.GROUPED_PRECOMPUTED_KEYS:
            np.testing.assert_array_equal(host[proj]["q_gmap_gr_words"], layers[i][proj]["q_gmap_gr_words"])
            assert host[proj]["bias"] is None and host[proj]["is_compact3"] is True
        bb = c.load_backbones(i, "cpu")
        np.testing.assert_array_equal(bb["gate"].numpy(), bbs[i]["gate"])
        assert bb["down"].is_quantized() and bb["down"].group_size == 64
        np.testing.assert_array_equal(bb["down"].qweight.numpy(), bbs[i]["down"]["qweight"])


def test_zero_output_scale_is_repaired(tris, tmp_path):
    """A compact3 payload saved with an all-zero output_scale loads with ones and has_output_scale False,
    and repair_grouped_payload_tensors fixes the tensors in place (grouped_payload_sidecar.py:248-337)."""
    layer = tris["synthetic"].make_layer(TINY, 7, tris["ext"].gr_encode)
    pls = {p: dict(layer[p]) for p in ck.GROUPED_PRECOMPUTED_KEYS}
    pls["up"]["output_scale"] = np.zeros_like(pls["up"]["output_scale"])
    pls["up"]["has_output_scale"] = True
    path = str(tmp_path / "c.safetensors")
    ck.save_grouped_checkpoint(path, [pls])
    got = ck.GroupedCheckpoint(path).load_layer("model.layers.0.block_sparse_moe", "cpu")
    assert got["up"]["has_output_scale"] is False and bool((got["up"]["output_scale"] == 1).all())
    tensors = ck.payload_tensors("L", "up", pls["up"])
    assert ck.repair_grouped_payload_tensors(tensors) == 1
    assert bool((tensors["L.grouped_payload.up.output_scale"] == 1).all())
    assert not bool(tensors["L.grouped_payload.up.has_output_scale"][0])


def test_sparse_bitmap_payload_converts_to_block_gr(tris, tmp_path):
    """A payload in the sparse split-bitmap format (q_gmap_sparse over the non-salient columns + prefix, no GR
    words) loads as block-GR with the words this build's encoder gives for the same dense bitmap."""
    from tris_moe_amd.packing import pack_sparse_bool_matrix, sparse_prefix, pack_bool_matrix

    syn, ext = tris["synthetic"], tris["ext"]
    layer = syn.make_layer(TINY, 9, ext.gr_encode)
    rng = np.random.default_rng(1)
    pls = {}
    for proj in ck.GROUPED_PRECOMPUTED_KEYS:
        p = dict(layer[proj])
        E, _, n = p["qweight1"].shape
        rank = p["g_idx"].shape[1]
        sparse, prefix, dense_words = [], [], []
        for e in range(E):
            sal = ((p["c_map"][e].astype(np.uint32)[np.arange(rank) // 32] >> (np.arange(rank) % 32).astype(np.uint32))
                   & 1).astype(bool)
            dense = (rng.random((n, rank)) < 0.2) & ~sal[None, :]
            sparse.append(pack_sparse_bool_matrix(dense, ~sal))
            prefix.append(sparse_prefix(~sal))
            dense_words.append(pack_bool_matrix(dense))
        rows = max(s.shape[0] for s in sparse)
        p["q_gmap_sparse"] = np.stack([np.pad(s, ((0, rows - s.shape[0]), (0, 0))) for s in sparse])
        p["q_gmap_sparse_prefix"] = np.stack(prefix)
        for k in ("q_gmap_gr_words", "q_gmap_gr_offsets", "q_gmap_gr_meta"):
            del p[k]
        p["compact3_use_block_gr"] = False
        p["_dense"] = dense_words
        pls[proj] = p
    path = str(tmp_path / "sparse.safetensors")
    ck.save_grouped_checkpoint(path, [pls], family="olmoe")
    got = ck.GroupedCheckpoint(path).load_layer("model.layers.0.mlp", "cpu")
    for proj in ck.GROUPED_PRECOMPUTED_KEYS:
        g = got[proj]
        assert g["compact3_use_block_gr"] is True and "q_gmap_sparse" not in g
        for e, dw in enumerate(pls[proj]["_dense"]):
            words, offsets, meta = ext.gr_encode(dw)
            np.testing.assert_array_equal(g["q_gmap_gr_offsets"][e].numpy(), offsets)
            np.testing.assert_array_equal(g["q_gmap_gr_meta"][e].numpy(), meta)
            np.testing.assert_array_equal(g["q_gmap_gr_words"][e, : words.size].numpy(), words)


def test_null_space_payloads_round_trip(tris, tmp_path):
    """gate_ns / up_ns / down_ns payloads are written under their cache keys, pass the compatibility check and
    load back with the same tensors and Python scalars; an inconsistent one is refused."""
    from safetensors.torch import load_file, save_file

    syn = tris["synthetic"]
    layer = syn.make_layer(TINY, 11, tris["ext"].gr_encode)
    rng = np.random.default_rng(0)
    pls = {p: layer[p] for p in ck.GROUPED_PRECOMPUTED_KEYS}
    pls["gate_ns"] = syn.make_ns_payload(rng, 4, TINY.hidden, TINY.intermediate, [8, 0, 16, 8], 64)
    pls["down_ns"] = syn.make_ns_payload(rng, 4, TINY.intermediate, TINY.hidden, [0, 0, 0, 0], 64)
    path = str(tmp_path / "ns.safetensors")
    ck.save_grouped_checkpoint(path, [pls])
    c = ck.GroupedCheckpoint(path)
    assert c.compatibility() == (True, None)
    got = c.load_layer("model.layers.0.block_sparse_moe", "cpu")
    assert "up_ns" not in got and got["gate_ns"]["max_ns_rank"] == 16 and got["down_ns"]["max_ns_rank"] == 0
    for k in ("ns_c2_qweight", "ns_c1_scales", "ns_c1_group_offsets"):
        np.testing.assert_array_equal(got["gate_ns"][k].numpy(), pls["gate_ns"][k])
    tensors = load_file(path)
    tensors["model.layers.0.block_sparse_moe.grouped_payload.gate_ns.ns_c1_qweight"] = torch.zeros((1, TINY.intermediate),
                                                                                                 dtype=torch.int32)
    save_file(tensors, path)
    c = ck.GroupedCheckpoint(path)
    assert c.compatibility()[0] is False
    with pytest.raises(ValueError, match="gate_ns"):
        c.load_layer("model.layers.0.block_sparse_moe", "cpu")


@pytest.mark.parametrize("family", ["mixtral", "olmoe"])
def test_input_scales_round_trip(tris, tmp_path, family):
    """experts[0]'s ns_mode / expert_input_scale (the per-expert state a deployment-only checkpoint keeps,
    grouped_payload_sidecar.py:38-46) load as the layer's backbone input scales; ns_mode 1 without a scale is
    an error."""
    from safetensors.torch import save_file

    scales = _input_scales(2)
    path, _, _ = _save(tris, tmp_path, input_scales=scales, family=family)
    c = ck.GroupedCheckpoint(path)
    mod = {"mixtral": ("w1", "w2"), "olmoe": ("gate_proj", "down_proj")}[family]
    lp1 = ck.moe_layer_prefix(1, family)
    assert f"{lp1}.experts.0.{mod[0]}.expert_input_scale" in c.keys()
    assert f"{lp1}.experts.0.{mod[1]}.ns_mode" in c.keys()
    bb0, bb1 = c.load_backbones(0, "cpu"), c.load_backbones(1, "cpu")
    assert not any(k.endswith("_in_scale") for k in bb0)
    assert sorted(k for k in bb1 if k.endswith("_in_scale")) == ["down_in_scale", "gate_in_scale"]
    for proj in ("gate", "down"):
        got = bb1[f"{proj}_in_scale"]
        assert got.dtype == torch.float16 and np.array_equal(got.numpy().view(np.uint16), scales[1][proj].view(np.uint16))
    # ns_mode 1 with the scale missing
    bad = {k: c._f.get_tensor(k) for k in c.keys() if not k.endswith("expert_input_scale")}
    path2 = str(tmp_path / "bad.safetensors")
    save_file(bad, path2)
    with pytest.raises(ValueError, match="ns_mode 1"):
        ck.GroupedCheckpoint(path2).load_backbones(1, "cpu")


def test_incomplete_checkpoint_is_reported(tris, tmp_path):
    from safetensors.torch import save_file

    path = str(tmp_path / "bad.safetensors")
    save_file({"model.layers.0.mlp.grouped_payload.gate.qweight1": torch.zeros(1, dtype=torch.int32)}, path)
    ok, reason = ck.GroupedCheckpoint(path).compatibility()
    assert not ok and "model.layers.0.mlp:gate" in reason
    save_file({"x": torch.zeros(1)}, path)
    assert ck.GroupedCheckpoint(path).compatibility()[0] is False


@pytest.mark.gpu
def test_checkpoint_layer_runs_like_memory(tris, oracle_mod, cuda, tmp_path):
    """Two layers loaded from a checkpoint (packed down backbones; layer 1 with ns_mode 1 input scales on its
    gate and down projections) match the oracle layer, and give the bits of the same layers built from the
    in-memory payloads."""
    print("checkpoint layer", flush=True)
    scales = _input_scales(2)
    path, layers, bbs = _save(tris, tmp_path, packed_down=True, input_scales=scales)
    c = ck.GroupedCheckpoint(path)
    ql, moe = tris["qlinear"], tris["moe"]
    rng = np.random.default_rng(5)
    x16 = torch.from_numpy(rng.standard_normal((3, TINY.hidden)).astype(np.float16)).to(cuda)
    logits = torch.from_numpy(rng.standard_normal((3, TINY.num_experts)).astype(np.float32)).to(cuda)
    for i, lp in enumerate(c.layer_prefixes()):
        loaded = c.load_layer(lp, cuda)
        lbb = c.load_backbones(i, cuda)
        mem = {p: ql.payload_to_device(layers[i][p], cuda) for p in ck.GROUPED_PRECOMPUTED_KEYS}
        mbb = {p: torch.from_numpy(bbs[i][p]).to(cuda) for p in ("gate", "up")}
        mbb["down"] = ql.PackedQuantMatrix4bit().set_from_payload(bbs[i]["down"]).to(cuda)
        for proj, sc in (scales[i] or {}).items():
            mbb[f"{proj}_in_scale"] = torch.from_numpy(sc).to(cuda)
        a = moe.grouped_moe_forward_from_logits(x16, logits, TINY.top_k, TINY.renormalize, loaded, lbb,
                                                TINY.num_experts, torch.bfloat16)
        b = moe.grouped_moe_forward_from_logits(x16, logits, TINY.top_k, TINY.renormalize, mem, mbb,
                                                TINY.num_experts, torch.bfloat16)
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), lp
        # the oracle layer on the host copies (the packed down backbone dequantised by the oracle)
        pk = bbs[i]["down"]
        down_sv = oracle_mod.packed4_dequant(pk["qweight"], pk["qzeros"], pk["scales"], pk["g_idx"], int(pk["rows"]),
                                             int(pk["cols"]))
        w, sel = oracle_mod.route_topk(logits.cpu().numpy(), TINY.top_k, TINY.renormalize)
        want = oracle_mod.bf16_round(oracle_mod.moe_layer(
            x16.cpu().numpy(), w, sel, {p: layers[i][p] for p in ck.GROUPED_PRECOMPUTED_KEYS},
            {"gate": bbs[i]["gate"], "up": bbs[i]["up"], "down": down_sv}, TINY.num_experts,
            input_scales=scales[i]))
        got = a.float().cpu().numpy().astype(np.float64)
        err = got - want
        rel = float(np.linalg.norm(err) / np.linalg.norm(want))
        assert float(np.abs(err).max()) <= 2e-2 and rel <= 1e-3, (lp, rel)


def _mode4_tensors(tris, rng, n=96, rank=128, sparse_form=False):
    """A non-expert compact3 module's state-dict tensors (QuantLinear mode 4), block-GR or sparse split
    bitmaps, with ns_mode 1 scales and packed null-space matrices."""
    from tris_moe_amd.packing import pack_4bit, pack_bool_matrix, pack_sparse_bool_matrix, sparse_prefix

    syn, ext = tris["synthetic"], tris["ext"]
    col_norm = rng.random(rank).astype(np.float32) + 0.5
    proj = syn.make_projection(rng, 1, n, rank, 0.15, col_norm, ext.gr_encode)
    t = {k: np.ascontiguousarray(proj[k][0]) for k in ("qweight1", "qweight2_sparse", "qweight2_sparse_prefix",
                                                       "c_map", "g_idx", "col_pack3", "row_pack3")}
    sal = ((t["c_map"].astype(np.uint32)[np.arange(rank) // 32] >> (np.arange(rank) % 32).astype(np.uint32)) & 1
           ).astype(bool)
    dense = (rng.random((n, rank)) < 0.2) & ~sal[None, :]
    words, offsets, meta = ext.gr_encode(pack_bool_matrix(dense))
    if sparse_form:
        t["q_gmap_sparse"] = pack_sparse_bool_matrix(dense, ~sal)
        t["q_gmap_sparse_prefix"] = sparse_prefix(~sal)
    else:
        t.update(q_gmap_gr_words=words, q_gmap_gr_offsets=offsets, q_gmap_gr_meta=meta)
    t["ns_mode"] = np.asarray([1], np.int32)
    t["ns_vector_col"] = (rng.random(rank) + 0.5).astype(np.float16)
    t["ns_vector_row"] = (rng.random(n) + 0.5).astype(np.float16)
    t["bias"] = rng.standard_normal(n).astype(np.float16)
    for key, mat, gs in (("ns_c2", rng.standard_normal((16, rank)), 32), ("ns_c1", rng.standard_normal((n, 16)), 16)):
        for name, v in pack_4bit(mat.astype(np.float32) * 0.05, gs).items():
            t[f"{key}_quant.{name}"] = v
    return t, (words, offsets, meta)


def test_compact3_linear_module_loads(tris, tmp_path):
    """load_compact3_linear: a mode-4 module's keys, block-GR or sparse split bitmaps (converted to the words
    this build's encoder gives), with its ns_mode 1 scales, bias and packed null-space matrices."""
    from safetensors.torch import save_file

    rng = np.random.default_rng(4)
    for sparse_form in (False, True):
        t, (words, offsets, meta) = _mode4_tensors(tris, rng, sparse_form=sparse_form)
        path = str(tmp_path / f"m4_{int(sparse_form)}.safetensors")
        save_file({f"model.layers.0.self_attn.q_proj.{k}": torch.from_numpy(np.ascontiguousarray(v))
                   for k, v in t.items()}, path)
        m = ck.GroupedCheckpoint(path).load_compact3_linear("model.layers.0.self_attn.q_proj", "cpu")
        np.testing.assert_array_equal(m.q_gmap_gr_offsets.numpy(), offsets)
        np.testing.assert_array_equal(m.q_gmap_gr_meta.numpy(), meta)
        np.testing.assert_array_equal(m.q_gmap_gr_words.numpy()[: words.size], words)
        np.testing.assert_array_equal(m.input_scale.numpy(), t["ns_vector_col"])
        np.testing.assert_array_equal(m.output_scale.numpy(), t["ns_vector_row"])
        assert m._ns_mode_host == 2 and m.ns_c1["qweight"].shape == t["ns_c1_quant.qweight"].shape


@pytest.mark.gpu
def test_compact3_linear_from_checkpoint_runs(tris, oracle_mod, cuda, tmp_path):
    """A mode-4 module loaded from a sparse-form checkpoint computes what the same module built from the
    block-GR tensors computes (bit for bit), within tolerance of the oracle."""
    from safetensors.torch import save_file
    from test_gpu_parity import assert_close, note

    note("compact3 linear from checkpoint")
    rng = np.random.default_rng(6)
    t, _ = _mode4_tensors(tris, rng, sparse_form=True)
    path = str(tmp_path / "m4.safetensors")
    save_file({f"mlp.shared_expert.gate_proj.{k}": torch.from_numpy(np.ascontiguousarray(v)) for k, v in t.items()},
              path)
    loaded = ck.GroupedCheckpoint(path).load_compact3_linear("mlp.shared_expert.gate_proj", cuda)
    rng2 = np.random.default_rng(6)
    tb, _ = _mode4_tensors(tris, rng2, sparse_form=False)
    direct = tris["qlinear"].Compact3Linear(128, 96).load_tensors(dict(
        {k: tb[k] for k in tris["qlinear"].COMPACT3_MODULE_KEYS}, input_scale=tb["ns_vector_col"],
        output_scale=tb["ns_vector_row"], bias=tb["bias"],
        ns_c1={n: tb[f"ns_c1_quant.{n}"] for n in ("qweight", "qzeros", "scales", "g_idx")},
        ns_c2={n: tb[f"ns_c2_quant.{n}"] for n in ("qweight", "qzeros", "scales", "g_idx")})).to(cuda)
    x = torch.from_numpy((np.random.default_rng(8).standard_normal((5, 128)) * 1.5).astype(np.float16)).to(cuda)
    y = loaded(x)
    assert torch.equal(y, direct(x))
    c2 = oracle_mod.packed4_dequant(tb["ns_c2_quant.qweight"], tb["ns_c2_quant.qzeros"], tb["ns_c2_quant.scales"],
                                    tb["ns_c2_quant.g_idx"], 16, 128)
    c1 = oracle_mod.packed4_dequant(tb["ns_c1_quant.qweight"], tb["ns_c1_quant.qzeros"], tb["ns_c1_quant.scales"],
                                    tb["ns_c1_quant.g_idx"], 96, 16)
    module = {k: tb[k] for k in tris["qlinear"].COMPACT3_MODULE_KEYS}
    want = oracle_mod.compact3_linear(x.cpu().numpy(), module, tb["ns_vector_col"], tb["ns_vector_row"], tb["bias"],
                                      c2, c1)
    assert_close(y.cpu().numpy(), want, "compact3 linear from checkpoint")
