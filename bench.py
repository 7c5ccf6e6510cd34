#!/usr/bin/env python3
"""Benchmark of the TriS-MoE grouped expert path on one MI355X.

Headline workload: one Mixtral-8x7B-shaped MoE layer
at decode (hidden 4096, 8 experts, intermediate 14336, top-2, rank-512 fp16
backbones, binarised compact3 experts with a block-GR split bitmap at
p = 0.15), T = 16 tokens.  A step is the whole block (TrisSparseMoeBlock.forward,
modeling_mixtral.py:539-608) from the bf16 activations: the router Linear (its
weight drawn so the logits are N(0, 1) as the config states), the bf16 -> fp16
cast, fused softmax / top-k / route, the gate/up backbone pair, the grouped
gate/up GEMM with the SwiGLU product, the down backbone, the grouped down GEMM
and the weighted scatter-add.  Synthetic seeded data; the steps cycle through
--layers identical-content layer copies resident in HBM (so weights come from
HBM, not the 256 MB last-level cache).  One HIP graph holds one step per layer
copy (as a model's decode graph holds its layers), and the timed region
replays it.

Prints ONE JSON line.  ``value`` is MoE-layer tokens/s at T = 16; ``hbm_gbps``
the step's algorithmic bytes (the active experts' compressed
payload + backbones + layer input/output) / step time, ``step_roofline_frac``
that over 8 TB/s; ``roofline`` is for the dominant kernel, timed live with HIP
events on its own stream over the same algorithmic (compressed) bytes of the
work it covers; ``cpu_baseline`` times the CPU oracle (GR decode + exact fp16
dequant + fp32 GEMMs, every host core) on the same layer.  The other configs
(C0, C2, C3, C4) are reported under their own keys.
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
PKG = ROOT / "neurips26-tris-moe_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBPS = 8000.0
MFMA_FP16_PEAK_TFLOPS = 2500.0  # dense fp16 MFMA, MI355X
PROJS = ("gate", "up", "down")


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=192, help="timed C1 steps at T = 16 (a multiple of --layers)")
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--tokens", type=int, default=16, help="decode batch of the reported line (1, 4 or 16)")
    ap.add_argument("--sweep", default="1,4", help="extra decode batches measured into 'sweep' ('' for none)")
    ap.add_argument("--layers", type=int, default=16, help="HBM-resident layer copies cycled through")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--cpu-baseline", type=int, default=1)
    ap.add_argument("--cpu-reps", type=int, default=20, help="timed CPU-baseline repetitions (median reported)")
    ap.add_argument("--configs", default="c0,c3,c4", help="other configs measured into their keys ('' for none)")
    ap.add_argument("--gmap-p", type=float, default=None, help="split-bitmap density of the reported C1 line "
                    "(default: the config's 0.15)")
    ap.add_argument("--expert-path", default="auto", choices=("auto", "predecoded", "fused"),
                    help="expert GEMM path of the reported C1 line (moe.grouped_moe_forward's expert_path)")
    ap.add_argument("--density-sweep", default="0.05,0.3",
                    help="split-bitmap densities p at which the C1 step is also measured, into 'gmap_density'")
    ap.add_argument("--stream-layers", type=int, default=32)
    ap.add_argument("--prefill", type=int, default=2048, help="C2 prefill tokens measured into 'prefill' (0: none)")
    ap.add_argument("--packed4", type=int, default=1,
                    help="also time the decode step with 4-bit packed backbones into 'packed4_backbones'")
    ap.add_argument("--ns", type=int, default=1,
                    help="also time the decode step with null-space compensation into 'ns_compensation'")
    ap.add_argument("--profile-kernel", action="store_true",
                    help="only run the dominant kernel eagerly --kernel-reps times (a target for rocprofv3 --pmc)")
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="only run a device-to-device copy of this many bytes 5 times (counter calibration)")
    ap.add_argument("--streaming", action="store_true", help="only measure C4 and print its JSON object")
    ap.add_argument("--prefill-only", action="store_true", help="only measure C2 and print its JSON object")
    return ap.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main():
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU; --gpus must be 1 "
                          "(sharding across GPUs is designed, not built)"}))
        sys.exit(2)
    import torch

    if args.copy_bytes > 0:
        dev = torch.device("cuda:0")
        src = torch.ones(args.copy_bytes // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": int(src.numel() * 4), "launches": 5}))
        return

    import tris_moe_amd
    from tris_moe_amd import ext, synthetic
    from tris_moe_amd.configs import C1_MIXTRAL_DECODE as SPEC

    tris_moe_amd.load_library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.streaming:
        print(json.dumps(streaming_bench(args, dev)), flush=True)
        return
    t0 = time.time()
    if args.gmap_p is not None:
        SPEC = dataclasses.replace(SPEC, gmap_p=args.gmap_p)
    layer = synthetic.make_layer(SPEC, args.seed, ext.gr_encode)
    log(f"synthetic C1 layer generated in {time.time() - t0:.1f}s (p = {SPEC.gmap_p:g})")
    lb = LayerBench(SPEC, layer, args.layers, dev, seed=args.seed)
    lb.expert_path = args.expert_path
    if args.profile_kernel:
        profile_dominant_kernel(args, lb)
        return
    if args.prefill_only:
        print(json.dumps(prefill_bench(args, lb)), flush=True)
        return

    main_res = lb.measure(args.tokens, args.steps, args.warmup, args.seed + args.tokens)
    log(f"C1 T={args.tokens}: {main_res['ms_per_step'] * 1e3:.1f} us/step, {main_res['tokens_per_s']:.0f} tok/s, "
        f"{main_res['hbm_gbps']:.0f} GB/s")
    sweep = {}
    for tok in [int(t) for t in args.sweep.split(",") if t.strip()]:
        if tok == args.tokens:
            continue
        r = lb.measure(tok, max(args.steps // 2, 2 * args.layers), args.warmup, args.seed + tok)
        sweep[f"T{tok}"] = summary(r)
        log(f"C1 T={tok}: {r['ms_per_step'] * 1e3:.1f} us/step, {r['tokens_per_s']:.0f} tok/s, {r['hbm_gbps']:.0f} GB/s")

    roofline = dominant_kernel_roofline(args, lb, main_res)
    log(f"dominant kernel {roofline['kernel']}: {roofline['kernel_us']:.1f} us/launch, "
        f"{roofline['achieved']:.0f} GB/s on compressed bytes (frac {roofline['frac']:.3f})")

    density = {}
    for p in [float(v) for v in args.density_sweep.split(",") if v.strip()]:
        if p == SPEC.gmap_p:
            continue
        dl = synthetic.make_layer(SPEC, args.seed, ext.gr_encode, gmap_p=p)
        db = LayerBench(SPEC, dl, args.layers, dev, seed=args.seed)
        r = db.measure(args.tokens, max(args.steps // 2, 2 * args.layers), args.warmup, args.seed + args.tokens)
        db.release()
        density[f"p{p:g}"] = summary(r)
        log(f"C1 T={args.tokens} at p={p:g}: {r['ms_per_step'] * 1e3:.1f} us/step, {r['tokens_per_s']:.0f} tok/s")

    packed4 = packed4_bench(args, lb) if args.packed4 else None
    ns_line = ns_bench(args, lb) if args.ns else None
    prefill = prefill_bench(args, lb) if args.prefill > 0 else None
    lb.release()
    others = {}
    wanted = {c.strip() for c in args.configs.split(",") if c.strip()}
    if "c0" in wanted:
        others["c0_olmoe"] = config_bench(args, "c0", dev)
    if "c3" in wanted:
        others["c3_a3b"] = config_bench(args, "c3", dev)
    if "c4" in wanted:
        others["c4_streaming"] = streaming_bench(args, dev)

    cpu = None
    if args.cpu_baseline:
        cpu = cpu_baseline(layer, main_res, SPEC, args.cpu_reps)
        log(f"cpu baseline: {cpu}")

    line = {
        "metric": "MoE-layer tokens/sec + achieved HBM GB/s (decode), Mixtral-8x7B shape",
        "value": round(main_res["tokens_per_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": main_res["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(main_res["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "hbm_gbps": round(main_res["hbm_gbps"], 1),
        "step_roofline_frac": round(main_res["hbm_gbps"] / HBM_PEAK_GBPS, 4),
        "config": {"workload": f"mixtral8x7b_moe_layer_decode_T{args.tokens}", "hidden": SPEC.hidden,
                   "experts": SPEC.num_experts, "intermediate": SPEC.intermediate, "top_k": SPEC.top_k,
                   "rank": SPEC.rank, "gmap_p": SPEC.gmap_p, "tokens": args.tokens,
                   "active_experts": main_res["active_experts"], "step_bytes": int(main_res["step_bytes"]),
                   "expert_bytes": int(main_res["expert_bytes"]), "layer_copies": args.layers,
                   "expert_path": args.expert_path,
                   "graph": (f"one HIP graph of {args.layers} steps (one per layer copy), replayed"
                             if main_res["steps"] % args.layers == 0 else
                             f"one HIP graph of {main_res['steps']} steps cycling through the layer copies")},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "sweep": sweep,
        "gmap_density": density,
        "prefill": prefill,
        "packed4_backbones": packed4,
        "ns_compensation": ns_line,
    }
    line.update(others)
    print(json.dumps(line), flush=True)


def summary(r):
    out = {k: round(r[k], 4) for k in ("ms_per_step", "tokens_per_s", "hbm_gbps")}
    out["graph"] = r.get("graph", True)
    out["step_roofline_frac"] = round(r["hbm_gbps"] / HBM_PEAK_GBPS, 4)
    out["active_experts"] = r["active_experts"]
    out["step_bytes"] = int(r["step_bytes"])
    return out


def router_weight(spec, seed):
    """The router Linear's weight [E, H] (bf16 values), drawn so that its logits on the synthetic activations
    are N(0, router_std) as the config states: N(0, router_std^2 / E||x||^2) entries, E||x||^2 = H + the
    outlier channels' extra variance."""
    import numpy as np

    from tris_moe_amd import synthetic

    rng = np.random.default_rng(seed)
    ex2 = spec.hidden + spec.outlier_channels * (spec.outlier_scale ** 2 - 1.0)
    w = rng.standard_normal((spec.num_experts, spec.hidden), dtype=np.float32) * np.float32(spec.router_std / ex2 ** 0.5)
    return synthetic.bf16_round(w)


class LayerBench:
    """One synthetic layer of a config with `copies` HBM-resident copies, and the decode-step timing.  A step is
    the whole block, TrisSparseMoeBlock.forward: the router Linear on the bf16 activations, the bf16 -> fp16
    cast of the kernel input, and the grouped layer to the bf16 output (modeling_mixtral.py:539-608)."""

    def __init__(self, spec, layer, copies, dev, backbones=None, seed=0):
        import torch

        from tris_moe_amd import qlinear

        self.spec, self.layer, self.dev = spec, layer, dev
        self.expert_path = "auto"
        base_pl = {p: qlinear.payload_to_device(layer[p], dev) for p in PROJS}
        base_bb = backbones if backbones is not None else {p: torch.from_numpy(layer["backbones"][p]).to(dev)
                                                            for p in PROJS}
        self.base = (base_pl, base_bb)
        clone = lambda d: {k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in d.items()}
        self.copies = [({p: clone(base_pl[p]) for p in PROJS}, {k: (v.clone() if isinstance(v, torch.Tensor) else v)
                                                                 for k, v in base_bb.items()})
                       for _ in range(copies)]
        self.router_w = torch.from_numpy(router_weight(spec, seed + 77)).to(dev).to(torch.bfloat16)
        self.routers = [self.router_w.clone() for _ in range(copies)]
        self.shared = None
        if "shared_expert" in layer:
            gate = torch.from_numpy(layer["shared_expert_gate"]).to(dev).to(torch.bfloat16)
            self.shared = [tuple(torch.from_numpy(w).to(dev) for w in layer["shared_expert"]) + (gate.clone(),)
                           for _ in range(copies)]
        torch.cuda.synchronize()
        log(f"{spec.name}: {copies} layer copies resident")

    def copy_nbytes(self) -> int:
        """Device bytes of one layer copy (payloads, backbones, router, shared expert)."""
        import torch

        pl, bb = self.copies[0]
        n = sum(v.numel() * v.element_size() for p in PROJS for v in pl[p].values() if isinstance(v, torch.Tensor))
        n += sum(v.numel() * v.element_size() for v in bb.values() if isinstance(v, torch.Tensor))
        n += self.routers[0].numel() * 2
        if self.shared is not None:
            n += sum(w.numel() * w.element_size() for w in self.shared[0])
        return n

    def release(self):
        import torch

        self.copies = None
        self.shared = None
        self.routers = None
        torch.cuda.synchronize()
        torch.cuda.empty_cache()

    def inputs(self, tokens, seed):
        """The bf16 block input [T, H] and the router logits the block computes from it (fp32)."""
        import torch
        import torch.nn.functional as F

        from tris_moe_amd import synthetic

        inp = synthetic.make_inputs(self.spec, tokens, seed, self.layer["outlier_idx"])
        x = torch.from_numpy(inp["x"]).to(self.dev).to(torch.bfloat16)
        logits = F.linear(x, self.router_w).float()
        return x, logits

    def block(self, i, copies=None):
        """A TrisSparseMoeBlock over layer copy i's device tensors (no copies made)."""
        from tris_moe_amd import moe

        cps = self.copies if copies is None else copies
        pl, bb = cps[i % len(cps)]
        sh = self.shared[i % len(self.shared)] if self.shared is not None else None
        spec = self.spec
        blk = moe.TrisSparseMoeBlock(spec.hidden, spec.num_experts, spec.top_k, pl, bb, renormalize=spec.renormalize,
                                     shared_expert=sh[:3] if sh is not None else None,
                                     shared_expert_gate=sh[3] if sh is not None else None)
        blk.gate.weight.data = self.routers[i % len(self.routers)]
        return blk

    def step_bytes(self, logits, tokens, backbone_bytes=None):
        """Algorithmic bytes: active experts' compressed payload + backbones + layer input and output
        (+ the router weight, the shared expert's fp16 weights and its gate)."""
        import numpy as np

        from tris_moe_amd import moe, synthetic

        w, sel = moe.route_topk(logits, self.spec.top_k, self.spec.renormalize)
        active = sorted(set(sel.cpu().numpy().reshape(-1).tolist()))
        expert_bytes = sum(synthetic.payload_nbytes(self.layer[p], active) for p in PROJS)
        if backbone_bytes is None:
            backbone_bytes = sum(self.layer["backbones"][p].nbytes for p in PROJS)
        shared_bytes = sum(int(np.asarray(a).nbytes) for a in self.layer.get("shared_expert", ()))
        if "shared_expert_gate" in self.layer:
            shared_bytes += 2 * self.spec.hidden
        act_bytes = 2 * tokens * self.spec.hidden * 2 + 2 * self.spec.num_experts * self.spec.hidden
        return expert_bytes + backbone_bytes + act_bytes + shared_bytes, expert_bytes, active

    def measure(self, tokens, steps, warmup, seed, copies=None, backbone_bytes=None, graph=True):
        """Mean time of one block step at `tokens`: steps cycle through the layer copies; one graph holds one
        step per copy and is replayed ceil(steps / copies) times (graph=False: eager launches)."""
        import torch

        cps = self.copies if copies is None else copies
        x, logits = self.inputs(tokens, seed)
        x3 = x.view(1, tokens, self.spec.hidden)
        blocks = [self.block(i, cps) for i in range(len(cps))]
        for b in blocks:
            b.expert_path = self.expert_path

        def step(i):
            return blocks[i % len(blocks)].forward(x3)[0]

        for i in range(max(warmup, 1)):
            step(i)
        torch.cuda.synchronize()
        # exactly `steps` steps: one pass over the copies replayed steps / copies times, or, when the copies do
        # not divide the step count, one pass of `steps` steps cycling through them
        steps = max(1, steps)
        per_run = len(cps) if steps % len(cps) == 0 else steps
        reps = steps // per_run
        if graph:
            g = torch.cuda.CUDAGraph()
            try:
                with torch.cuda.graph(g):
                    for i in range(per_run):
                        step(i)
            except RuntimeError as exc:  # a path that cannot be captured: time it eagerly and say so
                log(f"{self.spec.name} T={tokens}: graph capture failed ({exc}); timing eager launches")
                torch.cuda.synchronize()
                return self.measure(tokens, steps, warmup, seed, copies, backbone_bytes, graph=False)
            g.replay()
            torch.cuda.synchronize()
            run = g.replay
        else:
            def run():
                for i in range(per_run):
                    step(i)
            run()
            torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            run()
        end.record()
        torch.cuda.synchronize()
        n = reps * per_run
        ms = start.elapsed_time(end) / n
        sb, eb, active = self.step_bytes(logits, tokens, backbone_bytes)
        return {"tokens": tokens, "steps": n, "ms_per_step": ms, "tokens_per_s": tokens / (ms / 1e3),
                "hbm_gbps": sb / (ms / 1e3) / 1e9, "step_bytes": sb, "expert_bytes": eb,
                "active_experts": len(active), "x16": x.to(torch.float16), "x": x, "logits": logits,
                "active": active, "graph": bool(graph)}


def config_bench(args, name, dev):
    """C0 (OLMoE, T = 16) or C3 (A3B with the fp16 shared expert, T = 1 / 32 / 1024) decode steps."""
    from tris_moe_amd import ext, synthetic
    from tris_moe_amd.configs import C0_OLMOE, C3_A3B

    spec = {"c0": C0_OLMOE, "c3": C3_A3B}[name]
    t0 = time.time()
    layer = synthetic.make_layer(spec, args.seed, ext.gr_encode)
    # enough copies that their footprint (C0 about 22 MB, C3 about 70 MB each) exceeds the 256 MB last-level cache
    copies = 16 if name == "c0" else 8
    lb = LayerBench(spec, layer, copies, dev, seed=args.seed)
    lb.expert_path = args.expert_path
    log(f"{spec.name}: layer generated in {time.time() - t0:.1f}s")
    out = {"workload": f"{spec.name}_moe_layer", "hidden": spec.hidden, "experts": spec.num_experts,
           "intermediate": spec.intermediate, "top_k": spec.top_k, "rank": spec.rank,
           "shared_expert_intermediate": spec.shared_expert_intermediate,
           "shared_expert_gate": "shared_expert_gate" in layer, "layer_copies": copies,
           "layer_copy_bytes": int(lb.copy_nbytes())}
    for tok in spec.tokens:
        r = lb.measure(tok, 64 if tok <= 64 else 16, 3, args.seed + tok)
        out[f"T{tok}"] = summary(r)
        log(f"{spec.name} T={tok}: {r['ms_per_step'] * 1e3:.1f} us/step, {r['tokens_per_s']:.0f} tok/s, "
            f"{r['hbm_gbps']:.0f} GB/s ({r['active_experts']} active experts)")
    lb.release()
    return out


def packed4_bench(args, lb):
    """The C1 decode step with every backbone 4-bit packed (group 128, as real checkpoints store SV)."""
    import numpy as np

    from tris_moe_amd import packing
    from tris_moe_amd.qlinear import PackedQuantMatrix4bit

    pk = {p: packing.pack_4bit(lb.layer["backbones"][p].astype(np.float32), 128) for p in PROJS}
    p4_bytes = sum(pk[p][k].nbytes for p in PROJS for k in ("qweight", "qzeros", "scales", "g_idx"))
    pcopies = [(pl, {p: PackedQuantMatrix4bit().set_from_payload(pk[p]).to(lb.dev) for p in PROJS})
               for pl, _ in lb.copies]
    out = {"backbone_bytes": int(p4_bytes), "group_size": 128}
    for tok in sorted({args.tokens, 1}):
        r = lb.measure(tok, max(args.steps // 2, 2 * args.layers), args.warmup, args.seed + tok, pcopies, p4_bytes)
        out[f"T{tok}"] = summary(r)
        log(f"packed4 backbones T={tok}: {r['ms_per_step'] * 1e3:.1f} us/step, {r['tokens_per_s']:.0f} tok/s")
    return out


def ns_bench(args, lb):
    """The C1 decode step with matrix-mode null-space compensation on every projection (rank 32 per expert)."""
    import numpy as np

    from tris_moe_amd import qlinear as ql
    from tris_moe_amd import synthetic

    spec = lb.spec
    rng = np.random.default_rng(args.seed)
    ranks = [32] * spec.num_experts
    ns_host = {"gate": synthetic.make_ns_payload(rng, spec.num_experts, spec.hidden, spec.intermediate, ranks),
               "up": synthetic.make_ns_payload(rng, spec.num_experts, spec.hidden, spec.intermediate, ranks),
               "down": synthetic.make_ns_payload(rng, spec.num_experts, spec.intermediate, spec.hidden, ranks)}
    ns_dev = {f"{p}_ns": ql.ns_payload_to_device(ns_host[p], lb.dev) for p in PROJS}
    ncopies = [(dict(pl, **ns_dev), bb) for pl, bb in lb.copies]
    out = {"rank_per_expert": 32}
    for tok in sorted({args.tokens, 1}):
        r = lb.measure(tok, max(args.steps // 2, 2 * args.layers), args.warmup, args.seed + tok, ncopies)
        out[f"T{tok}"] = {k: round(r[k], 3) for k in ("ms_per_step", "tokens_per_s")}
        log(f"ns compensation T={tok}: {r['ms_per_step'] * 1e3:.1f} us/step, {r['tokens_per_s']:.0f} tok/s")
    return out


def layer_flops_per_token(spec) -> int:
    """Algorithmic flops of one token through the layer: gate/up backbones, top_k x (gate/up expert GEMMs, down
    backbone, down expert GEMM)."""
    h, r, i, k = spec.hidden, spec.rank, spec.intermediate, spec.top_k
    return 2 * (2 * h * r) + k * (2 * (2 * r * i) + 2 * i * r + 2 * r * h)


def prefill_bench(args, lb):
    """C2: the same layer weights at --prefill tokens with N(0, 1) router logits,
    block steps over the layer copies replayed from a HIP graph; MFMA-bound, reported against the dense fp16
    MFMA peak."""
    from tris_moe_amd.configs import C2_MIXTRAL_PREFILL as SPEC2

    T = args.prefill
    steps = max(2 * len(lb.copies), 20)
    r = lb.measure(T, steps, 3, args.seed + T)
    ms = r["ms_per_step"]
    flops = layer_flops_per_token(SPEC2) * T
    tflops = flops / (ms / 1e3) / 1e12
    log(f"C2 prefill T={T}: {ms:.3f} ms/step, {T / (ms / 1e3):.0f} tok/s, {tflops:.1f} TFLOP/s")
    return {"workload": f"mixtral8x7b_moe_layer_prefill_T{T}", "tokens": T, "steps": r["steps"],
            "ms_per_step": round(ms, 4), "tokens_per_s": round(T / (ms / 1e3), 1),
            "graph": r["graph"], "tflops": round(tflops, 2), "mfma_peak_tflops": MFMA_FP16_PEAK_TFLOPS,
            "mfma_frac": round(tflops / MFMA_FP16_PEAK_TFLOPS, 4), "flops_per_token": layer_flops_per_token(SPEC2)}


# ------------------------------------------------------------------------------------------ dominant kernel
def gateup_kernel(lb, rows, active, hid_g, hid_u, eid, seg, prob):
    """The gate/up grouped GEMM the layer step runs at `rows` routed rows: returns (launch(copy index),
    kernel name, compressed bytes per launch (the routed experts' gate and up payloads with
    their GR streams, the two backbone outputs read, the fp16 output(s) written), kind)."""
    import torch

    from tris_moe_amd import ext, moe, synthetic

    spec, dev = lb.spec, lb.dev
    names = ("qweight1", "qweight2_sparse", "qweight2_sparse_prefix", "c_map", "g_idx", "col_pack3", "row_pack3")
    slots = int(eid.numel())
    tile_bound = rows // 4 + slots + 1
    weights = synthetic.payload_nbytes(lb.layer["gate"], active) + synthetic.payload_nbytes(lb.layer["up"], active)
    nblk = int(lb.layer["gate"]["q_gmap_gr_meta"].shape[1])
    decoded = []
    for pl, _ in lb.copies:
        pair = []
        for p in ("gate", "up"):
            buf = torch.empty((slots, nblk, 128), dtype=torch.int32, device=dev)
            pair.append(ext.compact3_tris_precomputed_grouped_block_gr_predecode(
                buf, eid, pl[p]["q_gmap_gr_words"], pl[p]["q_gmap_gr_offsets"], pl[p]["q_gmap_gr_meta"],
                spec.rank // 32, spec.intermediate))
        decoded.append(pair)
    if rows <= moe.FUSED_SWIGLU_MAX_ROWS:
        mlp = torch.empty((rows, spec.intermediate), dtype=torch.float16, device=dev)

        def launch(i):
            pl = lb.copies[i][0]
            ext.compact3_tris_precomputed_grouped_swiglu_forward_block_gr_predecoded(
                hid_g, hid_u, eid, seg, prob, tile_bound, decoded[i][0], *[pl["gate"][k] for k in names],
                decoded[i][1], *[pl["up"][k] for k in names], out=mlp)
        name = "grouped_mfma_kernel<2> (gate/up grouped GEMM + SwiGLU epilogue, predecoded bitmaps)"
        nbytes = weights + 2 * rows * spec.rank * 2 + rows * spec.intermediate * 2
        return launch, name, nbytes, "swiglu"
    g = torch.empty((rows, spec.intermediate), dtype=torch.float16, device=dev)
    u = torch.empty_like(g)

    def launch(i):
        pl = lb.copies[i][0]
        ext.compact3_tris_precomputed_grouped_dual_forward_block_gr_predecoded(
            hid_g, hid_u, eid, seg, prob, tile_bound, decoded[i][0], *[pl["gate"][k] for k in names],
            decoded[i][1], *[pl["up"][k] for k in names], True, out_a=g, out_b=u)
    name = "grouped_mfma_kernel<1> (gate and up grouped GEMMs, predecoded bitmaps)"
    nbytes = weights + 2 * rows * spec.rank * 2 + 2 * rows * spec.intermediate * 2
    return launch, name, nbytes, "dual"


def _dominant_setup(lb, x16, logits):
    from tris_moe_amd import ext

    spec = lb.spec
    route = ext.route_topk_grouped(logits, spec.top_k, spec.renormalize, 4)
    rows = int(x16.size(0)) * spec.top_k
    slots = min(spec.num_experts, rows)
    eid = route["expert_ids"][:slots]
    seg = route["segment_offsets"][: slots + 1]
    prob = route["problem_offsets"][: slots + 1]
    bb = lb.base[1]
    hid_g, hid_u = ext.backbone_linear_pair(x16, bb["gate"], bb["up"], row_index=route["grouped_token_indices"])
    active = sorted(set(route["selected_experts"].cpu().numpy().reshape(-1).tolist()))
    return gateup_kernel(lb, rows, active, hid_g, hid_u, eid, seg, prob)


def dominant_kernel_roofline(args, lb, main_res):
    """The gate/up grouped GEMM of the T-token step, one launch per layer copy replayed from a graph on its own
    stream and timed there with HIP events; achieved = compressed bytes / mean launch time."""
    import torch

    launch, kname, kbytes, kind = _dominant_setup(lb, main_res["x16"], main_res["logits"])
    kstream = torch.cuda.Stream(device=lb.dev)
    kstream.wait_stream(torch.cuda.current_stream())
    n = len(lb.copies)
    with torch.cuda.stream(kstream):
        for i in range(n):
            launch(i)
        gk = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gk, stream=kstream):
            for i in range(n):
                launch(i)
        gk.replay()
        kstream.synchronize()
        ks, ke = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ks.record(kstream)
        for _ in range(args.kernel_reps):
            gk.replay()
        ke.record(kstream)
        kstream.synchronize()
    kernel_s = ks.elapsed_time(ke) / 1e3 / (args.kernel_reps * n)
    achieved = kbytes / kernel_s / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": measured_traffic(args.tokens, kind),
            "kernel": kname, "kernel_us": round(kernel_s * 1e6, 2), "bytes_per_launch": int(kbytes),
            "bytes": "compressed: routed experts' gate+up payloads incl. GR words, "
                     "backbone outputs read, outputs written"}


def measured_traffic(tokens: int, kind: str):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    runs (scaled by a copy-kernel calibration), or None when no measurement matches this workload."""
    path = ROOT / "profiles" / f"grouped_mfma_{kind}_mixtral_decode_T{tokens}_traffic.json"
    try:
        return int(json.loads(path.read_text())["traffic_bytes"])
    except (OSError, ValueError, KeyError):
        return None


def profile_dominant_kernel(args, lb):
    """Eager launches of the dominant kernel at the bench workload, for hardware-counter runs."""
    import torch

    x, logits = lb.inputs(args.tokens, args.seed + args.tokens)
    launch, kname, nbytes, kind = _dominant_setup(lb, x.to(torch.float16), logits)
    for r in range(args.kernel_reps):
        launch(r % len(lb.copies))
    torch.cuda.synchronize()
    print(json.dumps({"kernel": kname, "kind": kind, "launches": args.kernel_reps, "bytes_per_launch": nbytes}))


# ---------------------------------------------------------------------------------------------------- C4
def streaming_bench(args, dev):
    """C4: a 32-layer Mixtral MoE stack at T = 8 (each layer's input the previous layer's output) with every
    layer's compressed payload and backbones streamed from pinned host memory into two device slots, the next
    layer's copy overlapping the current layer's kernels; against the same stack resident in HBM.  One
    synthetic layer per split-bitmap density is shared by all 32 layers' host blobs (the copies are real)."""
    import numpy as np
    import torch

    from tris_moe_amd import ext, moe, qlinear, streaming, synthetic
    from tris_moe_amd.configs import C4_DENSITIES, C4_STREAMING as SPEC

    T = SPEC.tokens[0]
    L = args.stream_layers
    results = {}
    for p in C4_DENSITIES:
        t0 = time.time()
        layer = synthetic.make_layer(SPEC, args.seed, ext.gr_encode, gmap_p=p)
        host = [{q: layer[q] for q in streaming.PROJECTIONS} for _ in range(L)]
        bbs = [layer["backbones"] for _ in range(L)]
        st = streaming.GroupedPayloadStreamer(host, dev, num_slots=2, backbones=bbs)
        log(f"C4 p={p}: layer generated and {L} pinned blobs of {st.layer_nbytes(0) / 1e6:.1f} MB packed in "
            f"{time.time() - t0:.1f}s")
        inp = synthetic.make_inputs(SPEC, T, args.seed + T, layer["outlier_idx"])
        x16 = torch.from_numpy(inp["x"]).to(dev).to(torch.bfloat16).to(torch.float16)
        rng = np.random.default_rng(args.seed)
        logits = [torch.from_numpy(rng.standard_normal((T, SPEC.num_experts)).astype(np.float32)).to(dev)
                  for _ in range(L)]

        def timed(fn, reps=3):
            fn()
            torch.cuda.synchronize()
            s_, e_ = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s_.record()
            for _ in range(reps):
                fn()
            e_.record()
            torch.cuda.synchronize()
            return s_.elapsed_time(e_) / reps / 1e3

        stream_s = timed(lambda: streaming.streamed_forward(st, x16, logits, SPEC.top_k, SPEC.renormalize,
                                                            SPEC.num_experts))
        layer_bytes = st.layer_nbytes(0)
        slot_bytes = int(2 * st.slot_bytes)
        del st
        # variant: backbones resident (L x 23 MB on the device), only the expert payloads streamed
        st_e = streaming.GroupedPayloadStreamer(host, dev, num_slots=2, backbones=None)
        bb_res = [{q: torch.from_numpy(layer["backbones"][q]).to(dev) for q in streaming.PROJECTIONS} for _ in range(L)]
        stream_e_s = timed(lambda: streaming.streamed_forward(st_e, x16, logits, SPEC.top_k, SPEC.renormalize,
                                                              SPEC.num_experts, backbones=bb_res))
        expert_bytes = st_e.layer_nbytes(0)
        del st_e
        # the same stack resident in HBM: L distinct device copies (so every layer reads HBM, not the cache)
        pl0 = {q: qlinear.payload_to_device(layer[q], dev) for q in streaming.PROJECTIONS}
        pls = [{q: {k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in pl0[q].items()}
                for q in streaming.PROJECTIONS} for _ in range(L)]

        def resident():
            x = x16
            for i in range(L):
                x = moe.grouped_moe_forward_from_logits(x, logits[i], SPEC.top_k, SPEC.renormalize, pls[i],
                                                        bb_res[i], SPEC.num_experts, torch.bfloat16).to(torch.float16)
        resident_s = timed(resident)
        results[f"p{p}"] = {
            "tokens_per_s": round(T / stream_s, 1), "ms_per_forward": round(stream_s * 1e3, 3),
            "resident_ms_per_forward": round(resident_s * 1e3, 3),
            "resident_tokens_per_s": round(T / resident_s, 1), "layer_bytes": int(layer_bytes),
            "h2d_gbps": round(L * layer_bytes / stream_s / 1e9, 2),
            "device_slot_bytes": slot_bytes, "resident_model_bytes": int(L * layer_bytes),
            "experts_only": {"tokens_per_s": round(T / stream_e_s, 1), "ms_per_forward": round(stream_e_s * 1e3, 3),
                             "layer_bytes": int(expert_bytes),
                             "h2d_gbps": round(L * expert_bytes / stream_e_s / 1e9, 2)}}
        log(f"C4 p={p}: streamed {stream_s * 1e3:.2f} ms / {L} layers ({T / stream_s:.0f} tok/s, "
            f"{L * layer_bytes / stream_s / 1e9:.1f} GB/s host-to-device), experts only {stream_e_s * 1e3:.2f} ms, "
            f"resident {resident_s * 1e3:.2f} ms")
        del bb_res, host, bbs, pl0, pls
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return {"workload": f"mixtral8x7b_moe_stack_{L}layers_T{T}_streamed", "layers": L, "tokens": T, "slots": 2,
            "device_budget": "two layer slots (the C4 budget as a parameter below the stack's payload)",
            "results": results}


# ------------------------------------------------------------------------------------------ CPU baseline
def cpu_baseline(layer, res, spec, reps):
    """The CPU oracle (the reference's CPU path restated: GR decode of every active expert's split bitmaps in
    C, exact fp16 dequant in numpy, fp32 GEMMs; the reference re-dequantises on every call,
    qlinear_cuda.py:4532-4547) on the same T-token layer step, every host core (the dequant spread over a
    thread pool, BLAS on all threads); one warm-up, then the median of `reps` repetitions."""
    try:
        import numpy as np

        import oracle
    except Exception as exc:  # oracle library not built
        return {"error": repr(exc)}
    nproc = os.cpu_count() or 1
    workers = max(1, min(nproc, 16))  # the box's CPU share for one GPU
    x = res["x16"].float().cpu().numpy().astype(np.float16)
    logits = res["logits"].cpu().numpy()
    w, sel = oracle.route_topk(logits, spec.top_k, spec.renormalize)
    payloads = {p: layer[p] for p in PROJS}
    active = sorted(set(sel.reshape(-1).tolist()))

    def one_step():
        caches = oracle.dequant_experts(payloads, active, workers)
        return oracle.moe_layer(x, w, sel, payloads, layer["backbones"], spec.num_experts, weight_caches=caches)

    one_step()  # warm-up
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        one_step()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    tokens = x.shape[0]
    return {"value": round(tokens / med, 3), "unit": "tokens/s", "cores": workers, "nproc": nproc, "kind": "port",
            "reps": reps, "median_s": round(med, 4), "min_s": round(min(times), 4),
            "sample": f"the full C1 layer step at T={tokens} ({len(active)} active experts): GR decode + exact fp16 "
                      f"dequant of every active expert + fp32 GEMMs; 1 warm-up + median of {reps} "
                      f"({sum(times):.1f}s timed)"}


if __name__ == "__main__":
    main()
