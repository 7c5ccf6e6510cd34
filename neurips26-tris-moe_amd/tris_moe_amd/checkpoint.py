"""Grouped runtime payload checkpoints (safetensors).

Reads and writes the reference's checkpoint layout for the grouped expert path
(``grouped_payload_sidecar.py:18-135`` key scheme and scalar encoding, ``:160-337``
decoding, compatibility checks and repair, ``:340-361`` inspection, ``:586-698``
loading), so that exported TriS-MoE checkpoints load into this build without the
AutoGPTQ loader:

* expert payloads: ``{layer_prefix}.grouped_payload.{gate|up|down}.{name}`` with
  ``layer_prefix`` ``model.layers.{i}.block_sparse_moe`` (Mixtral) or
  ``model.layers.{i}.mlp`` (OLMoE / Qwen-MoE); Python scalars are stored as
  one-element tensors (bool or int32), ``None`` as an empty tensor; names
  starting with ``_`` (derived caches) are never written;
* shared backbones (the ``ExpertSharedMatrix`` banks of a layer,
  ``modeling/_utils.py:135-177``): ``model.layers.{i}.TriS_shared_{proj}_proj.shared_sv``
  (fp16 [rank, in]) or ``....shared_sv_quant.{qweight,qzeros,scales,g_idx,rows,cols}``
  (4-bit packed, ``qlinear_cuda.py:2637-2786``).

Loading returns the stacked payload dicts the grouped kernels take (device
tensors, scalars as Python values, the uniform-K64 proof taken once).  Payloads
stored with the sparse split bitmap (``q_gmap_sparse`` + prefix, no block-GR
words) are converted to block-GR on load: the bitmap is expanded to its dense
form and GR-coded with this build's encoder (the format the kernels read).
Matrix-mode null-space payloads (``gate_ns`` / ``up_ns`` / ``down_ns`` cache keys,
``build_grouped_ns_compensation_payload`` layout) load next to them, checked like
the reference's ``_sidecar_payload_is_compatible`` (:196-245) and bounds-checked
before they reach a kernel.  Host-side I/O only; nothing here runs on the GPU
except the final copies.
"""
from __future__ import annotations

import os

import numpy as np
import torch

GROUPED_PAYLOAD_SIDECAR_BASENAME = "grouped_runtime_payload.safetensors"
GROUPED_PAYLOAD_METADATA = {"format": "olmoe_grouped_runtime_payload_v1"}
GROUPED_PAYLOAD_EMBEDDED_METADATA_KEY = "olmoe_grouped_runtime_payload"
GROUPED_PRECOMPUTED_KEYS = ("gate", "up", "down")
GROUPED_QGMAP_PAYLOAD_NAMES = frozenset({"q_gmap_sparse", "q_gmap_sparse_prefix"})
SCALAR_NAMES = frozenset({"is_compact3", "compact3_use_block_gr", "has_output_scale", "has_bias", "max_ns_rank",
                          "infeatures", "outfeatures", "group_size"})
BOOL_NAMES = frozenset({"is_compact3", "compact3_use_block_gr", "has_output_scale", "has_bias"})
PROJ_MODULE = {"gate": "gate_proj", "up": "up_proj", "down": "down_proj"}
# Expert module of each projection under a MoE block's ``experts.{e}`` (grouped_payload_sidecar.py:467-495):
# Mixtral's w1 / w3 / w2, else gate_proj / up_proj / down_proj.
EXPERT_MODULE = {"mixtral": {"gate": "w1", "up": "w3", "down": "w2"}, "other": PROJ_MODULE}
PACKED4_NAMES = ("qweight", "qzeros", "scales", "g_idx", "rows", "cols")
MARKER = ".grouped_payload."


# ------------------------------------------------------------------------------------------------ names
def payload_tensor_name(layer_prefix: str, cache_key: str, name: str) -> str:
    """grouped_payload_sidecar.py:104-105."""
    return f"{layer_prefix}{MARKER}{cache_key}.{name}"


def split_payload_tensor_name(name: str):
    """(layer_prefix, cache_key, payload_name) of a payload tensor key, else None (:112-122)."""
    if MARKER not in name:
        return None
    layer_prefix, rest = name.split(MARKER, 1)
    if "." not in rest:
        return None
    cache_key, payload_name = rest.split(".", 1)
    if not cache_key or not payload_name:
        return None
    return layer_prefix, cache_key, payload_name


def moe_layer_prefix(layer_idx: int, family: str = "mixtral") -> str:
    """The MoE block of decoder layer i (grouped_payload_sidecar.py:54-80)."""
    return f"model.layers.{layer_idx}.block_sparse_moe" if family == "mixtral" else f"model.layers.{layer_idx}.mlp"


def expert_module_prefix(layer_prefix: str, expert: int, proj: str) -> str:
    """The state-dict prefix of one expert's projection module under a MoE block."""
    family = "mixtral" if layer_prefix.endswith("block_sparse_moe") else "other"
    return f"{layer_prefix}.experts.{expert}.{EXPERT_MODULE[family][proj]}"


def shared_bank_prefix(layer_idx: int, proj: str) -> str:
    """The ExpertSharedMatrix of (layer, projection): attribute TriS_shared_{gate|up|down}_proj of the
    decoder layer (modeling/_utils.py:135-177)."""
    return f"model.layers.{layer_idx}.TriS_shared_{PROJ_MODULE[proj]}"


# ------------------------------------------------------------------------------------------------ write
def encode_payload_tensor(value):
    """A payload value as a checkpoint tensor (grouped_payload_sidecar.py:172-184): arrays as they are
    (0-d made 1-element), bool -> bool [1], int -> int32 [1], None -> empty fp16."""
    if isinstance(value, torch.Tensor):
        value = value.detach().to("cpu").contiguous()
        return value.reshape(1) if value.ndim == 0 else value
    if isinstance(value, np.ndarray):
        t = torch.from_numpy(np.ascontiguousarray(value))
        return t.reshape(1) if t.ndim == 0 else t
    if value is None:
        return torch.empty((0,), dtype=torch.float16)
    if isinstance(value, (bool, np.bool_)):
        return torch.tensor([bool(value)], dtype=torch.bool)
    if isinstance(value, (int, np.integer)):
        return torch.tensor([int(value)], dtype=torch.int32)
    raise TypeError(f"unsupported grouped payload value {type(value)!r}")


def payload_tensors(layer_prefix: str, cache_key: str, payload: dict) -> dict:
    """Checkpoint tensors of one stacked payload; derived caches (names starting with '_') and the
    host-only dense split bitmap are left out."""
    out = {}
    for name, value in payload.items():
        if name.startswith("_") or name == "gmap_dense":
            continue
        out[payload_tensor_name(layer_prefix, cache_key, name)] = encode_payload_tensor(value)
    return out


def backbone_tensors(layer_idx: int, proj: str, backbone) -> dict:
    """Checkpoint tensors of one shared backbone: an fp16 SV [rank, in], or a packed 4-bit payload dict
    (qweight, qzeros, scales, g_idx, rows, cols)."""
    prefix = shared_bank_prefix(layer_idx, proj)
    if isinstance(backbone, dict):
        out = {}
        for k in PACKED4_NAMES:
            v = backbone[k]
            if k in ("rows", "cols"):  # 0-d int32 buffers, as PackedQuantMatrix4bit registers them
                out[f"{prefix}.shared_sv_quant.{k}"] = torch.tensor(int(v), dtype=torch.int32)
            else:
                out[f"{prefix}.shared_sv_quant.{k}"] = encode_payload_tensor(v)
        return out
    return {f"{prefix}.shared_sv": encode_payload_tensor(np.asarray(backbone, dtype=np.float16))}


def save_grouped_checkpoint(path: str, layers: list, family: str = "mixtral", backbones: list | None = None,
                            metadata: dict | None = None, input_scales: list | None = None) -> str:
    """Write decoder layers' grouped payloads (``layers[i] = {"gate": payload, "up": ..., "down": ...}``,
    host arrays) and optionally their shared backbones (``backbones[i] = {proj: SV or packed payload}``) in the
    reference's key scheme, with the sidecar metadata (:542-557).  ``input_scales[i] = {proj: fp16 [in]}``
    writes experts[0]'s ``mode`` (5), ``ns_mode`` (1) and ``expert_input_scale`` for those projections, the
    per-expert state a deployment-only checkpoint keeps (grouped_payload_sidecar.py:38-46)."""
    from safetensors.torch import save_file

    tensors = {}
    for i, layer in enumerate(layers):
        for proj, scale in ((input_scales[i] or {}) if input_scales is not None else {}).items():
            prefix = expert_module_prefix(moe_layer_prefix(i, family), 0, proj)
            tensors[f"{prefix}.mode"] = torch.tensor([5], dtype=torch.int32)
            tensors[f"{prefix}.ns_mode"] = torch.tensor([1], dtype=torch.int32)
            tensors[f"{prefix}.expert_input_scale"] = encode_payload_tensor(np.asarray(scale, dtype=np.float16))
        for key in GROUPED_PRECOMPUTED_KEYS:
            tensors.update(payload_tensors(moe_layer_prefix(i, family), key, layer[key]))
            if layer.get(f"{key}_ns") is not None:
                tensors.update(payload_tensors(moe_layer_prefix(i, family), f"{key}_ns", layer[f"{key}_ns"]))
        if backbones is not None:
            for proj in GROUPED_PRECOMPUTED_KEYS:
                tensors.update(backbone_tensors(i, proj, backbones[i][proj]))
    meta = dict(GROUPED_PAYLOAD_METADATA)
    if metadata:
        meta.update({str(k): str(v) for k, v in metadata.items()})
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    save_file(tensors, path, metadata=meta)
    return path


# ------------------------------------------------------------------------------------------------ repair
def repair_grouped_payload_tensors(tensors: dict) -> int:
    """In place: a compact3 payload whose output_scale is all zeros gets ones and has_output_scale False
    (grouped_payload_sidecar.py:307-337).  Returns the number of payloads repaired."""
    groups = {}
    for name in tensors:
        split = split_payload_tensor_name(name)
        if split is None or split[1] not in GROUPED_PRECOMPUTED_KEYS:
            continue
        groups.setdefault(split[:2], {})[split[2]] = name
    repaired = 0
    for names in groups.values():
        c3, osn = names.get("is_compact3"), names.get("output_scale")
        if c3 is None or osn is None:
            continue
        is_c3, scale = tensors[c3], tensors[osn]
        if is_c3.numel() == 0 or not bool(is_c3.reshape(-1)[0]) or scale.numel() == 0 or bool((scale != 0).any()):
            continue
        tensors[osn] = torch.ones_like(scale)
        if "has_output_scale" in names:
            tensors[names["has_output_scale"]] = torch.zeros_like(tensors[names["has_output_scale"]],
                                                                   dtype=torch.bool)
        repaired += 1
    return repaired


def sparse_gmap_to_dense(q_gmap_sparse: np.ndarray, prefix: np.ndarray, c_map: np.ndarray, rank: int) -> np.ndarray:
    """The dense split bitmap (int32 [rank/32, N], zeros at salient columns) of one expert from its sparse
    form: the j-th non-salient column (k order) has its bits in word j // 32, bit j % 32
    (TriSMoE_cuda_kernel.cu:619-637; the inverse of pack_sparse_bool_matrix)."""
    from .packing import pack_bool_matrix

    words = np.asarray(q_gmap_sparse).astype(np.uint32)
    n = words.shape[1]
    cm = np.asarray(c_map).astype(np.uint32)
    salient = ((cm[np.arange(rank) // 32] >> (np.arange(rank) % 32).astype(np.uint32)) & 1).astype(bool)
    active = np.flatnonzero(~salient)
    pre = np.asarray(prefix, dtype=np.int64)
    if active.size and pre.size > 1 and int(pre[-1]) != active.size:
        raise ValueError(f"q_gmap_sparse_prefix counts {int(pre[-1])} non-salient columns, c_map {active.size}")
    dense = np.zeros((n, rank), dtype=bool)
    if active.size:
        j = np.arange(active.size)
        dense[:, active] = ((words[j // 32] >> (j % 32).astype(np.uint32)[:, None]) & 1).astype(bool).T
    return pack_bool_matrix(dense)


def _to_block_gr(payload: dict) -> dict:
    """A sparse-bitmap compact3 payload as block-GR: per expert dense bitmap, GR-coded, stacked with zero
    padding (qlinear_cuda.py:1551-1601)."""
    from . import ext

    qs = payload["q_gmap_sparse"].cpu().numpy()
    pre = payload["q_gmap_sparse_prefix"].cpu().numpy()
    cmap = payload["c_map"].cpu().numpy()
    rank = int(payload["g_idx"].shape[1])
    coded = [ext.gr_encode(sparse_gmap_to_dense(qs[e], pre[e], cmap[e], rank)) for e in range(qs.shape[0])]
    width = max(c[0].size for c in coded)
    words = np.zeros((len(coded), width), dtype=np.int32)
    for e, c in enumerate(coded):
        words[e, : c[0].size] = c[0]
    dev = payload["qweight1"].device
    out = {k: v for k, v in payload.items() if k not in GROUPED_QGMAP_PAYLOAD_NAMES}
    out["q_gmap_gr_words"] = torch.from_numpy(words).to(dev)
    out["q_gmap_gr_offsets"] = torch.from_numpy(np.stack([c[1] for c in coded])).to(dev)
    out["q_gmap_gr_meta"] = torch.from_numpy(np.stack([c[2] for c in coded])).to(dev)
    out["compact3_use_block_gr"] = True
    return out


def _k64_uniform(g_idx: torch.Tensor) -> bool:
    """Every 64-column K tile of every expert lies in one group (qlinear_cuda.py:364-381)."""
    rank = int(g_idx.shape[-1])
    first = g_idx[..., (torch.arange(rank, device=g_idx.device) // 64) * 64]
    return bool(torch.equal(first, g_idx))


def decode_payload(raw: dict, device, dtype=torch.float16) -> dict | None:
    """One stacked payload from its checkpoint tensors (grouped_payload_sidecar.py:187-193, 248-304,
    630-643): floating tensors to ``dtype``, integer tensors to int32/int64 as stored, 1-element scalars to
    Python values, an all-zero output_scale repaired to ones, empty bias to None, sparse bitmaps converted to
    block-GR; None when it is not a compact3 payload this path runs."""
    p = {}
    for name, t in raw.items():
        if name in SCALAR_NAMES and t.numel() == 1:
            v = t.reshape(-1)[0].item()
            p[name] = bool(v) if name in BOOL_NAMES else int(v)
        elif t.is_floating_point():
            p[name] = t.to(device=device, dtype=dtype).contiguous()
        else:
            p[name] = t.to(device=device).contiguous()
    if not p.get("is_compact3", False):
        return None
    scale = p.get("output_scale")
    if isinstance(scale, torch.Tensor) and scale.numel() and not bool((scale != 0).any()):
        p["output_scale"] = torch.ones_like(scale)
        p["has_output_scale"] = False
    bias = p.get("bias")
    if isinstance(bias, torch.Tensor) and bias.numel() == 0:
        p["bias"] = None
        p["has_bias"] = False
    if not p.get("compact3_use_block_gr", False) or "q_gmap_gr_words" not in p:
        if not GROUPED_QGMAP_PAYLOAD_NAMES <= set(p):
            return None
        p = _to_block_gr(p)
    for key in ("qweight1", "qweight2_sparse", "qweight2_sparse_prefix", "c_map", "g_idx", "col_pack3", "row_pack3",
                "output_scale"):
        if key not in p:
            raise ValueError(f"grouped payload lacks {key}")
    if "has_output_scale" not in p:
        p["has_output_scale"] = not bool(torch.all(p["output_scale"] == 1).item())
    p.setdefault("has_bias", p.get("bias") is not None)
    p["_compact3_k64_groups_uniform"] = _k64_uniform(p["g_idx"])
    return p


# ------------------------------------------------------------------------------------------------ read
class GroupedCheckpoint:
    """A safetensors checkpoint (sidecar or full model file) holding grouped payloads and shared banks.

    ``layer_prefixes()`` lists the MoE blocks with payloads; ``load_layer(prefix, device)`` returns
    ``{"gate", "up", "down"}`` payload dicts; ``load_backbones(i, device)`` the layer's shared backbones (fp16
    tensors or ``qlinear.PackedQuantMatrix4bit`` modules)."""

    def __init__(self, path: str):
        from safetensors import safe_open

        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.path = path
        self._f = safe_open(path, framework="pt", device="cpu")
        self.metadata = dict(self._f.metadata() or {})
        self._keys = list(self._f.keys())
        self._payload_keys = {}
        for k in self._keys:
            split = split_payload_tensor_name(k)
            if split is not None:
                self._payload_keys.setdefault(split[:2], {})[split[2]] = k

    def keys(self):
        return list(self._keys)

    def layer_prefixes(self) -> list:
        def order(prefix):
            parts = prefix.split(".")
            return (int(parts[2]) if len(parts) > 2 and parts[2].isdigit() else -1, prefix)
        return sorted({lp for lp, key in self._payload_keys if key in GROUPED_PRECOMPUTED_KEYS}, key=order)

    def ns_compatible(self, layer_prefix: str, cache_key: str) -> bool:
        """grouped_payload_sidecar.py:196-245: every null-space tensor present, offsets one per expert, block
        shapes consistent with infeatures, outfeatures, group_size and the per-expert ranks."""
        names = self._payload_keys.get((layer_prefix, cache_key), {})
        need = ("ns_rank_per_expert", "ns_c2_rank_offsets", "ns_c2_rank_word_offsets", "ns_c1_rank_word_offsets",
                "ns_c1_group_offsets", "max_ns_rank", "group_size", "infeatures", "outfeatures", "ns_c2_qweight",
                "ns_c2_qzeros", "ns_c2_scales", "ns_c1_qweight", "ns_c1_qzeros", "ns_c1_scales")
        if any(n not in names for n in need):
            return False
        t = {n: self._f.get_tensor(names[n]) for n in need}
        scal = {n: int(t[n].reshape(-1)[0]) if t[n].numel() else 0 for n in ("group_size", "infeatures", "outfeatures")}
        gs, inf, outf = scal["group_size"], scal["infeatures"], scal["outfeatures"]
        if gs <= 0 or inf < 0 or outf < 0:
            return False
        E = int(t["ns_rank_per_expert"].numel())
        if any(int(t[n].numel()) != E for n in ("ns_c2_rank_offsets", "ns_c2_rank_word_offsets",
                                               "ns_c1_rank_word_offsets", "ns_c1_group_offsets")):
            return False
        if t["ns_c2_qweight"].ndim != 2 or int(t["ns_c2_qweight"].shape[0]) != (inf + 7) // 8:
            return False
        if t["ns_c2_qzeros"].ndim != 2 or t["ns_c2_scales"].ndim != 2:
            return False
        if int(t["ns_c2_qzeros"].shape[0]) != int(t["ns_c2_scales"].shape[0]) or \
                int(t["ns_c2_qzeros"].shape[0]) != ((inf + gs - 1) // gs if inf > 0 else 0):
            return False
        if t["ns_c1_qweight"].ndim != 2 or int(t["ns_c1_qweight"].shape[1]) != outf:
            return False
        if t["ns_c1_qzeros"].ndim != 2 or int(t["ns_c1_qzeros"].shape[1]) != (outf + 7) // 8:
            return False
        if t["ns_c1_scales"].ndim != 2 or int(t["ns_c1_scales"].shape[1]) != outf:
            return False
        ranks = t["ns_rank_per_expert"].reshape(-1).to(torch.int64)
        pos = ranks[ranks > 0]
        words = int(((pos + 7) // 8).sum()) if pos.numel() else 0
        groups = int(((pos + gs - 1) // gs).sum()) if pos.numel() else 0
        return (int(t["ns_c1_qweight"].shape[0]) == words and int(t["ns_c1_qzeros"].shape[0]) == groups
                and int(t["ns_c1_scales"].shape[0]) == groups)

    def compatibility(self):
        """(ok, reason) like inspect_grouped_payload_sidecar_compatibility (grouped_payload_sidecar.py:340-361),
        for the block-GR/sparse compact3 payloads this path loads."""
        if not self._payload_keys:
            return False, "checkpoint contains no grouped payload tensors"
        for (lp, key), names in sorted(self._payload_keys.items()):
            if key.endswith("_ns") and key[:-3] in GROUPED_PRECOMPUTED_KEYS:
                if not self.ns_compatible(lp, key):
                    return False, f"incompatible grouped payload: {lp}:{key}"
                continue
            if key not in GROUPED_PRECOMPUTED_KEYS:
                continue
            need = {"is_compact3", "qweight1", "qweight2_sparse", "qweight2_sparse_prefix", "c_map", "g_idx",
                    "col_pack3", "row_pack3", "output_scale"}
            gr = {"q_gmap_gr_words", "q_gmap_gr_offsets", "q_gmap_gr_meta"}
            if not need <= set(names) or not (gr <= set(names) or GROUPED_QGMAP_PAYLOAD_NAMES <= set(names)):
                return False, f"incomplete grouped payload: {lp}:{key}"
        return True, None

    def raw_payload(self, layer_prefix: str, cache_key: str) -> dict | None:
        names = self._payload_keys.get((layer_prefix, cache_key))
        if names is None:
            return None
        return {n: self._f.get_tensor(k) for n, k in names.items()}

    def load_payload(self, layer_prefix: str, cache_key: str, device, dtype=torch.float16) -> dict | None:
        raw = self.raw_payload(layer_prefix, cache_key)
        return None if raw is None else decode_payload(raw, device, dtype)

    def load_ns_payload(self, layer_prefix: str, cache_key: str, device, dtype=torch.float16) -> dict | None:
        """The null-space payload of ``cache_key`` (gate / up / down) on the device, or None when the checkpoint
        has none; raises ValueError when it is present but inconsistent."""
        from .qlinear import ns_payload_to_device

        key = f"{cache_key}_ns"
        raw = self.raw_payload(layer_prefix, key)
        if raw is None:
            return None
        if not self.ns_compatible(layer_prefix, key):
            raise ValueError(f"{self.path}: incompatible null-space payload {layer_prefix}:{key}")
        host = {n: (int(t.reshape(-1)[0]) if n in SCALAR_NAMES and t.numel() == 1 else t) for n, t in raw.items()}
        return ns_payload_to_device(host, device, dtype)

    def load_layer(self, layer_prefix: str, device, dtype=torch.float16) -> dict:
        """{"gate", "up", "down"} payloads, plus "gate_ns" / "up_ns" / "down_ns" where the checkpoint has them."""
        out = {}
        for key in GROUPED_PRECOMPUTED_KEYS:
            p = self.load_payload(layer_prefix, key, device, dtype)
            if p is None:
                raise KeyError(f"{self.path}: no compact3 grouped payload {layer_prefix}:{key}")
            out[key] = p
            ns = self.load_ns_payload(layer_prefix, key, device, dtype)
            if ns is not None:
                out[f"{key}_ns"] = ns
        return out

    def load_layer_numpy(self, layer_prefix: str) -> dict:
        """load_layer on the host with numpy arrays (the form ``streaming.GroupedPayloadStreamer`` packs into
        pinned layer blobs)."""
        layer = self.load_layer(layer_prefix, "cpu")
        return {proj: {k: (v.numpy() if isinstance(v, torch.Tensor) else v) for k, v in p.items()}
                for proj, p in layer.items() if proj in GROUPED_PRECOMPUTED_KEYS}

    def load_compact3_linear(self, prefix: str, device):
        """A non-expert compact3 linear (the reference's QuantLinear in mode 4: attention projections,
        dense or shared-expert MLPs) from its state-dict keys ``{prefix}.qweight1`` ... ``{prefix}.row_pack3``,
        as a ``qlinear.Compact3Linear`` on ``device``.  A sparse split bitmap (``q_gmap_sparse`` +
        prefix) is converted to block-GR here; ``ns_mode == 1`` brings the input / output scales
        ``ns_vector_col`` / ``ns_vector_row`` and packed ``ns_c1_quant`` / ``ns_c2_quant`` matrices the
        null-space term, as the reference's forward uses them (qlinear_cuda.py:4238-4360, 3998-4022)."""
        from .packing import num_gr_blocks
        from .qlinear import COMPACT3_MODULE_KEYS, Compact3Linear

        get = lambda name: self._f.get_tensor(f"{prefix}.{name}") if f"{prefix}.{name}" in self._keys else None
        t = {k: get(k) for k in COMPACT3_MODULE_KEYS}
        rank = int(t["g_idx"].numel())
        n = int(t["qweight1"].size(1))
        gro, grm = t.get("q_gmap_gr_offsets"), t.get("q_gmap_gr_meta")
        if gro is None or grm is None or int(grm.numel()) != num_gr_blocks(rank, n):
            sparse, sprefix = get("q_gmap_sparse"), get("q_gmap_sparse_prefix")
            if sparse is None or sprefix is None:
                raise KeyError(f"{self.path}: {prefix} has neither block-GR nor sparse split bitmaps")
            one = {"q_gmap_sparse": sparse[None], "q_gmap_sparse_prefix": sprefix[None], "c_map": t["c_map"][None],
                   "g_idx": t["g_idx"][None], "qweight1": t["qweight1"][None]}
            gr = _to_block_gr(one)
            for k in ("q_gmap_gr_words", "q_gmap_gr_offsets", "q_gmap_gr_meta"):
                t[k] = torch.as_tensor(gr[k])[0]
        extras = {}
        ns_mode = get("ns_mode")
        if ns_mode is not None and int(ns_mode.reshape(-1)[0]) == 1:
            extras["input_scale"] = get("ns_vector_col")
            extras["output_scale"] = get("ns_vector_row")
        bias = get("bias")
        if bias is not None and bias.numel() > 0:
            extras["bias"] = bias
        for key in ("ns_c1", "ns_c2"):
            q = {name: get(f"{key}_quant.{name}") for name in ("qweight", "qzeros", "scales", "g_idx")}
            if all(v is not None and v.numel() > 0 for v in q.values()):
                extras[key] = q
        if ("ns_c1" in extras) != ("ns_c2" in extras):
            extras.pop("ns_c1", None)
            extras.pop("ns_c2", None)
        return Compact3Linear(rank, n).load_tensors(dict(t, **extras)).to(device)

    def load_input_scales(self, layer_prefix: str, device) -> dict:
        """``{proj}_in_scale`` for the projections whose experts[0] module has ``ns_mode == 1``: the fp16 [in]
        vector compute_shared_hidden multiplies the backbone input by (``expert_input_scale`` for expert_compact3
        modules, mode 5; ``ns_vector_col`` otherwise, qlinear_cuda.py:3918-3923, 4477-4480).  The grouped
        forward projects every expert's input through experts[0] (modeling_mixtral.py:469-470, 497), so only
        expert 0's scale is read.  Raises ValueError when ns_mode is 1 and the scale is missing."""
        out = {}
        for proj in GROUPED_PRECOMPUTED_KEYS:
            prefix = expert_module_prefix(layer_prefix, 0, proj)
            key = f"{prefix}.ns_mode"
            if key not in self._keys or int(self._f.get_tensor(key).reshape(-1)[0]) != 1:
                continue
            mode_key = f"{prefix}.mode"
            mode = int(self._f.get_tensor(mode_key).reshape(-1)[0]) if mode_key in self._keys else 5
            name = f"{prefix}.expert_input_scale" if mode == 5 else f"{prefix}.ns_vector_col"
            if name not in self._keys or self._f.get_tensor(name).numel() == 0:
                raise ValueError(f"{self.path}: {prefix} has ns_mode 1 but no {name.rsplit('.', 1)[1]}")
            out[f"{proj}_in_scale"] = self._f.get_tensor(name).to(device=device, dtype=torch.float16).contiguous()
        return out

    def load_backbones(self, layer_idx: int, device, layer_prefix: str | None = None) -> dict:
        """The layer's shared backbones {gate, up, down}, plus ``{proj}_in_scale`` entries for the projections
        that scale their input (``load_input_scales`` of ``layer_prefix``, by default the layer's Mixtral or
        OLMoE block, whichever the checkpoint holds)."""
        from .qlinear import PackedQuantMatrix4bit

        out = {}
        if layer_prefix is None:
            cands = [moe_layer_prefix(layer_idx, f) for f in ("mixtral", "other")]
            held = [c for c in cands if any(k.startswith(c + ".") for k in self._keys)]
            layer_prefix = held[0] if held else None
        if layer_prefix is not None:
            out.update(self.load_input_scales(layer_prefix, device))
        for proj in GROUPED_PRECOMPUTED_KEYS:
            prefix = shared_bank_prefix(layer_idx, proj)
            quant = {n: f"{prefix}.shared_sv_quant.{n}" for n in PACKED4_NAMES}
            if all(k in self._keys for k in quant.values()) and self._f.get_tensor(quant["qweight"]).numel() > 0:
                t = {n: self._f.get_tensor(k) for n, k in quant.items()}
                out[proj] = PackedQuantMatrix4bit().set_quantized(
                    t["qweight"], t["qzeros"], t["scales"].to(torch.float16), t["g_idx"], int(t["rows"].reshape(-1)[0]),
                    int(t["cols"].reshape(-1)[0])).to(device)
            elif f"{prefix}.shared_sv" in self._keys:
                out[proj] = self._f.get_tensor(f"{prefix}.shared_sv").to(device=device, dtype=torch.float16).contiguous()
            else:
                raise KeyError(f"{self.path}: no shared backbone {prefix}")
        return out
