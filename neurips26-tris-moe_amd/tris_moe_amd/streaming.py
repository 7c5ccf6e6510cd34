"""Streaming of whole compressed MoE layer payloads from pinned host memory into device slots.

Generalises the reference's ``GroupedQGmapCPUStagingManager`` (grouped_payload_sidecar.py:764-1153), which
streams only the sparse split bitmap of non-GR payloads into one reused workspace, to block-GR payloads with
every tensor of a layer (gate, up and down payloads, optionally the backbones): a layer is one pinned host
blob, copied with one asynchronous host-to-device transfer on a copy stream into one of ``num_slots`` device
slots, so that the next layer's copy overlaps the current layer's kernels when a device budget keeps the
model off the GPU.  The reference's own mode, only the split bitmaps streamed (sparse or block-GR) and every
other tensor resident, is ``split_bitmaps`` plus the streamer's ``resident`` argument.

Ordering (as the reference's per-slot ready/done events, :1093-1134):

* ``prefetch(i)`` picks a slot for layer i; the copy stream first waits for that slot's ``done`` event, which
  ``release`` of the slot's previous layer recorded on the compute stream, then copies and records ``ready``.
* ``acquire(i)`` makes the compute stream wait for ``ready`` and returns device payload dicts whose tensors
  are views into the slot (the kernels read them in place).
* ``release(i)`` records ``done`` on the compute stream after the layer's kernels were queued.

The manager is host-side orchestration; the transfer is the DMA engine's hipMemcpyAsync from page-locked
memory (torch ``pin_memory=True`` allocates it), and nothing here synchronises the host.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

PROJECTIONS = ("gate", "up", "down")
ALIGN = 256  # byte alignment of every tensor in a blob (and of the fp16 activations' 16-byte loads)

_TORCH_DTYPES = {
    np.dtype(np.int32): torch.int32,
    np.dtype(np.int64): torch.int64,
    np.dtype(np.float16): torch.float16,
    np.dtype(np.float32): torch.float32,
}


@dataclass(frozen=True)
class BlobEntry:
    """One tensor of a layer blob: projection (or "backbone"), key, dtype, shape, byte offset."""

    owner: str
    key: str
    dtype: np.dtype
    shape: tuple
    offset: int

    @property
    def nbytes(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize


@dataclass
class LayerLayout:
    entries: list = field(default_factory=list)
    nbytes: int = 0
    scalars: dict = field(default_factory=dict)  # owner -> non-array payload values


def _host_array(key: str, val: np.ndarray) -> np.ndarray:
    """The dtype a payload tensor has on the device (qlinear.payload_to_device)."""
    if key in ("output_scale", "bias"):
        return np.ascontiguousarray(val, dtype=np.float16)
    if val.dtype == np.int64:
        return np.ascontiguousarray(val)
    return np.ascontiguousarray(val, dtype=np.int32)


def layer_layout(payloads: dict, backbones: dict | None = None) -> LayerLayout:
    """Blob layout of one layer: every array of the gate, up and down payloads (in key order), then the
    backbones if given; offsets are ALIGN-aligned."""
    lay = LayerLayout()
    off = 0

    def add(owner, key, arr):
        nonlocal off
        off = (off + ALIGN - 1) // ALIGN * ALIGN
        lay.entries.append(BlobEntry(owner, key, arr.dtype, tuple(arr.shape), off))
        off += arr.nbytes

    for proj in PROJECTIONS:
        pl = payloads[proj]
        lay.scalars[proj] = {}
        for key in sorted(pl):
            val = pl[key]
            if isinstance(val, np.ndarray):
                add(proj, key, _host_array(key, val))
            else:
                lay.scalars[proj][key] = val
    if backbones is not None:
        for proj in PROJECTIONS:
            add("backbone", proj, np.ascontiguousarray(backbones[proj], dtype=np.float16))
    lay.nbytes = (off + ALIGN - 1) // ALIGN * ALIGN
    return lay


def pack_layer(payloads: dict, backbones: dict | None, layout: LayerLayout, out: np.ndarray) -> None:
    """Write one layer's arrays into ``out`` (a uint8 view of at least layout.nbytes) at the layout's offsets."""
    for ent in layout.entries:
        arr = backbones[ent.key] if ent.owner == "backbone" else payloads[ent.owner][ent.key]
        arr = np.ascontiguousarray(arr, dtype=ent.dtype) if ent.owner == "backbone" else _host_array(ent.key, arr)
        out[ent.offset:ent.offset + ent.nbytes] = arr.reshape(-1).view(np.uint8)


def unpack_views(layout: LayerLayout, buf: torch.Tensor) -> tuple[dict, dict | None]:
    """Payload dicts (and backbones) whose tensors view ``buf`` (uint8, on any device) at the layout."""
    payloads = {proj: dict(layout.scalars[proj]) for proj in PROJECTIONS}
    backbones = None
    for ent in layout.entries:
        t = buf[ent.offset:ent.offset + ent.nbytes].view(_TORCH_DTYPES[ent.dtype]).view(ent.shape)
        if ent.owner == "backbone":
            backbones = backbones if backbones is not None else {}
            backbones[ent.key] = t
        else:
            payloads[ent.owner][ent.key] = t
    return payloads, backbones


# the split-bitmap tensors of a payload: what the reference's staging manager streams
# (grouped_payload_sidecar.py:764-1146 streams q_gmap_sparse(+prefix)); for block-GR payloads their GR streams
BITMAP_KEYS = frozenset({"q_gmap_sparse", "q_gmap_sparse_prefix", "q_gmap_gr_words", "q_gmap_gr_offsets",
                         "q_gmap_gr_meta"})


def split_bitmaps(layer: dict) -> tuple[dict, dict]:
    """One layer's host payloads split into (split bitmaps, the rest): stream the first with
    ``GroupedPayloadStreamer`` and keep the second resident (``resident=``), as the reference's staging
    manager keeps every other payload tensor on the device."""
    streamed, rest = {}, {}
    for proj in PROJECTIONS:
        pl = layer[proj]
        streamed[proj] = {k: v for k, v in pl.items() if k in BITMAP_KEYS}
        rest[proj] = {k: v for k, v in pl.items() if k not in BITMAP_KEYS}
    return streamed, rest


def _uniform_k64(g_idx: np.ndarray) -> bool:
    """Every 64-column K tile of every expert lies in one group (qlinear_cuda.py:364-381)."""
    rank = g_idx.shape[-1]
    first = g_idx[..., (np.arange(rank) // 64) * 64]
    return bool(np.array_equal(first, g_idx))


class GroupedPayloadStreamer:
    """Whole-layer payload streaming into ``num_slots`` device slots (two by default: one layer computing,
    the next one copying).

    ``layers``: per layer ``{"gate": payload, "up": payload, "down": payload}`` with numpy arrays (the host
    format of ``synthetic.make_layer`` / the sidecar loader); ``backbones``: per layer ``{"gate": SV, "up": SV,
    "down": SV}`` fp16 arrays to stream as well, or None to keep them out of the blob.  ``resident``: per layer
    the same dicts of device tensors that stay on the GPU (``split_bitmaps`` and ``qlinear.payload_to_device``);
    acquire merges them under the streamed tensors, so ``layers`` may hold only the split bitmaps.
    """

    def __init__(self, layers: list, device, num_slots: int = 2, backbones: list | None = None,
                 resident: list | None = None):
        if num_slots < 1:
            raise ValueError("num_slots must be at least 1")
        if not layers:
            raise ValueError("no layers to stream")
        if backbones is not None and len(backbones) != len(layers):
            raise ValueError("one backbone dict per layer")
        if resident is not None and len(resident) != len(layers):
            raise ValueError("one resident payload dict per layer")
        self.resident = resident
        self.device = torch.device(device)
        self.layouts = [layer_layout(layers[i], None if backbones is None else backbones[i]) for i in range(len(layers))]
        self.slot_bytes = max(l.nbytes for l in self.layouts)
        self.num_slots = num_slots
        # page-locked host blobs (hipHostMalloc through torch), one per layer
        self.host = []
        for i, lay in enumerate(self.layouts):
            blob = torch.empty(lay.nbytes, dtype=torch.uint8, pin_memory=True)
            pack_layer(layers[i], None if backbones is None else backbones[i], lay, blob.numpy())
            self.host.append(blob)
        # the uniform 64-column group proof is taken once on the host (a device check would synchronise)
        def g_idx(i, p):
            if "g_idx" in layers[i][p]:
                return np.asarray(layers[i][p]["g_idx"])
            return resident[i][p]["g_idx"].cpu().numpy()

        self._uniform = [{p: _uniform_k64(g_idx(i, p)) for p in PROJECTIONS} for i in range(len(layers))]
        self.slots = [torch.empty(self.slot_bytes, dtype=torch.uint8, device=self.device) for _ in range(num_slots)]
        self.copy_stream = torch.cuda.Stream(device=self.device)
        self._ready = [torch.cuda.Event() for _ in range(num_slots)]
        self._done = [torch.cuda.Event() for _ in range(num_slots)]
        self._used = [False] * num_slots
        self._held = [False] * num_slots     # acquired and not yet released: the slot must not be refilled
        self._owner = [-1] * num_slots       # layer held (or being copied) by each slot
        self._where = {}                      # layer -> slot
        self._next = 0
        self.stats = {"prefetches": 0, "copies": 0, "bytes": 0, "slot_reuses": 0, "hits": 0}

    @property
    def num_layers(self) -> int:
        return len(self.layouts)

    def layer_nbytes(self, i: int) -> int:
        return self.layouts[i].nbytes

    def prefetch(self, i: int) -> int:
        """Queue layer i's copy into a slot (no-op when it is already resident); returns the slot.  The slots are
        taken round-robin, skipping slots whose layer is acquired and not yet released (kernels queued on it may
        still read it); RuntimeError when every slot is held."""
        if not 0 <= i < self.num_layers:
            raise IndexError(f"layer {i} out of range")
        self.stats["prefetches"] += 1
        if i in self._where:
            self.stats["hits"] += 1
            return self._where[i]
        for _ in range(self.num_slots):
            s = self._next
            self._next = (self._next + 1) % self.num_slots
            if not self._held[s]:
                break
        else:
            raise RuntimeError(f"prefetch of layer {i}: every slot holds an acquired layer (release one first)")
        old = self._owner[s]
        if old >= 0:
            del self._where[old]
        self._owner[s] = i
        self._where[i] = s
        with torch.cuda.stream(self.copy_stream):
            if self._used[s]:
                self.copy_stream.wait_event(self._done[s])  # the slot's previous layer has finished
                self.stats["slot_reuses"] += 1
            n = self.layouts[i].nbytes
            self.slots[s][:n].copy_(self.host[i], non_blocking=True)
            self._ready[s].record(self.copy_stream)
        self.stats["copies"] += 1
        self.stats["bytes"] += self.layouts[i].nbytes
        return s

    def acquire(self, i: int, stream: torch.cuda.Stream | None = None):
        """Device payloads (and backbones, or None) of layer i; ``stream`` (default: current) waits for the copy."""
        s = self._where.get(i)
        if s is None:
            s = self.prefetch(i)
        stream = stream if stream is not None else torch.cuda.current_stream(self.device)
        stream.wait_event(self._ready[s])
        self._held[s] = True
        # the slot's memory is used by `stream` (caching allocator bookkeeping for the views)
        self.slots[s].record_stream(stream)
        payloads, backbones = unpack_views(self.layouts[i], self.slots[s])
        if self.resident is not None:
            payloads = {p: {**self.resident[i][p], **payloads[p]} for p in PROJECTIONS}
        for p in PROJECTIONS:
            payloads[p]["_compact3_k64_groups_uniform"] = self._uniform[i][p]
        return payloads, backbones

    def release(self, i: int, stream: torch.cuda.Stream | None = None) -> None:
        """Layer i's kernels are queued on ``stream``: its slot may be refilled once they finish."""
        s = self._where.get(i)
        if s is None:
            raise RuntimeError(f"layer {i} is not resident")
        stream = stream if stream is not None else torch.cuda.current_stream(self.device)
        self._done[s].record(stream)
        self._used[s] = True
        self._held[s] = False


def streamed_forward(streamer: GroupedPayloadStreamer, x16: torch.Tensor, router_logits: list, top_k: int,
                     renormalize: bool, num_experts: int, backbones: list | None = None,
                     outputs: list | None = None, residual: bool = False, inputs: list | None = None):
    """Run the layers in order, prefetching layer i + 1 while layer i computes.  Layer i + 1's input is layer
    i's output (fp16), or with ``residual`` the residual stream fp16(x_i + out_i) that a decoder stack feeds
    its next layer (keeps activations O(1) across many layers).  ``router_logits[i]``: the [T, E] fp32 logits
    of layer i; ``backbones[i]``: resident backbones when the blobs do not carry them; ``outputs`` /
    ``inputs``: lists that receive every layer's output (bf16) / input (fp16).  Returns the last output."""
    from . import moe

    n = streamer.num_layers
    streamer.prefetch(0)
    out = None
    for i in range(n):
        if i + 1 < n and streamer.num_slots > 1:  # with one slot the next copy waits for this layer anyway
            streamer.prefetch(i + 1)
        payloads, bb = streamer.acquire(i)
        if bb is None:
            bb = backbones[i]
        if inputs is not None:
            inputs.append(x16)
        out = moe.grouped_moe_forward_from_logits(x16, router_logits[i], top_k, renormalize, payloads, bb,
                                                  num_experts, torch.bfloat16)
        streamer.release(i)
        if outputs is not None:
            outputs.append(out)
        x16 = (x16.float() + out.float()).to(torch.float16) if residual else out.to(torch.float16)
    return out
