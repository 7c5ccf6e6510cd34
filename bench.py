#!/usr/bin/env python3
"""Benchmark of the TriS-MoE grouped expert path on one MI355X.

Workload: one Mixtral-8x7B-shaped MoE layer at
decode (hidden 4096, 8 experts, intermediate 14336, top-2, rank-512 fp16
backbones, binarised compact3 experts with a block-GR split bitmap at
p = 0.15).  A step is one full layer forward over one decode batch from the
router logits: fused softmax/top-k/route, gate/up backbone pair, GR predecode
of the routed experts' split bitmaps (gate, up, down in one launch, on a side
stream), MFMA grouped gate/up GEMM with the SwiGLU product, down backbone,
grouped down GEMM and the weighted scatter-add.  Synthetic seeded data; every step reads a different one of
--layers identical-content layer copies resident in HBM (so weights come from
HBM, not the 256 MB last-level cache), with each step captured in a HIP graph.

Prints ONE JSON line.  ``value`` is MoE-layer tokens/s; ``hbm_gbps`` the
layer's algorithmic bytes / step time; ``roofline`` is for the dominant
kernel, the MFMA gate/up grouped GEMM over predecoded bitmaps that the step runs at this batch
(grouped_mfma_kernel<1> for gate and up in separate workgroups, or grouped_mfma_kernel<2> with the
SwiGLU epilogue at <= 4 routed rows), timed live with HIP events on its own stream; ``cpu_baseline`` times the
CPU oracle (GR decode + exact fp16 dequant + fp32 GEMM) on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
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


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--tokens", type=int, default=16, help="decode batch of the reported line (1, 4 or 16)")
    ap.add_argument("--sweep", default="1,4", help="extra decode batches measured into 'sweep' ('' for none)")
    ap.add_argument("--layers", type=int, default=16, help="HBM-resident layer copies cycled through")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--cpu-baseline", type=int, default=1)
    ap.add_argument("--profile-kernel", action="store_true",
                    help="only run the dominant kernel eagerly --kernel-reps times (a target for rocprofv3 --pmc)")
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="only run a device-to-device copy of this many bytes 5 times (counter calibration)")
    ap.add_argument("--streaming", action="store_true",
                    help="only measure C4: 32 Mixtral layers at T=8 with whole-layer payloads streamed from pinned "
                         "host memory through two device slots, for p = 0.05, 0.15, 0.30 (one JSON line)")
    ap.add_argument("--stream-layers", type=int, default=32)
    ap.add_argument("--prefill", type=int, default=2048,
                    help="C2 prefill tokens measured into 'prefill' (0 for none)")
    ap.add_argument("--packed4", type=int, default=1,
                    help="also time the decode step with 4-bit packed backbones into 'packed4_backbones'")
    ap.add_argument("--ns", type=int, default=1,
                    help="also time the decode step with null-space compensation into 'ns_compensation'")
    ap.add_argument("--prefill-only", action="store_true",
                    help="measure only the C2 prefill step and print its JSON object")
    return ap.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main():
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU; --gpus must be 1 "
                          "(sharding across GPUs is designed, not built)"}))
        sys.exit(2)
    import numpy as np
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
    from tris_moe_amd import ext, moe, qlinear, synthetic
    from tris_moe_amd.configs import C1_MIXTRAL_DECODE as SPEC

    tris_moe_amd.load_library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.streaming:
        streaming_bench(args, dev)
        return
    t0 = time.time()
    layer = synthetic.make_layer(SPEC, args.seed, ext.gr_encode)
    log(f"synthetic layer generated in {time.time() - t0:.1f}s")
    projs = ("gate", "up", "down")
    base_payloads = {p: qlinear.payload_to_device(layer[p], dev) for p in projs}
    base_backbones = {p: torch.from_numpy(layer["backbones"][p]).to(dev) for p in projs}

    def clone_payload(pl):
        return {k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in pl.items()}

    copies = [({p: clone_payload(base_payloads[p]) for p in projs}, {p: v.clone() for p, v in base_backbones.items()})
              for _ in range(args.layers)]
    torch.cuda.synchronize()
    log(f"{args.layers} layer copies resident")

    def measure(tokens: int, steps: int, warmup: int, cps=None, backbone_bytes=None):
        cps = copies if cps is None else cps
        inp = synthetic.make_inputs(SPEC, tokens, args.seed + tokens, layer["outlier_idx"])
        x16 = torch.from_numpy(inp["x"]).to(dev).to(torch.bfloat16).to(torch.float16)
        logits = torch.from_numpy(inp["router_logits"]).to(dev)

        def step(i):
            pl, bb = cps[i % len(cps)]
            return moe.grouped_moe_forward_from_logits(x16, logits, SPEC.top_k, SPEC.renormalize, pl, bb,
                                                       SPEC.num_experts, torch.bfloat16)

        for i in range(max(warmup, 1)):
            step(i)
        torch.cuda.synchronize()
        graphs = []
        for i in range(len(cps)):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                step(i)
            graphs.append(g)
        for g in graphs:
            g.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for s in range(steps):
            graphs[s % len(graphs)].replay()
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / steps
        # algorithmic bytes of the step (actual routing of this batch)
        w, sel = moe.route_topk(logits, SPEC.top_k, SPEC.renormalize)
        active = sorted(set(sel.cpu().numpy().reshape(-1).tolist()))
        expert_bytes = sum(synthetic.payload_nbytes(layer[p], active) for p in projs)
        if backbone_bytes is None:
            backbone_bytes = sum(layer["backbones"][p].nbytes for p in projs)
        act_bytes = 2 * tokens * SPEC.hidden * 2
        step_bytes = expert_bytes + backbone_bytes + act_bytes
        return {"tokens": tokens, "ms_per_step": ms, "tokens_per_s": tokens / (ms / 1e3),
                "hbm_gbps": step_bytes / (ms / 1e3) / 1e9, "step_bytes": step_bytes, "expert_bytes": expert_bytes,
                "active_experts": len(active), "x16": x16, "logits": logits, "active": active}

    if args.profile_kernel:
        profile_dominant_kernel(args, layer, base_payloads, base_backbones, SPEC, dev)
        return
    if args.prefill_only:
        print(json.dumps(prefill_bench(args, layer, copies, dev)), flush=True)
        return
    main_res = measure(args.tokens, args.steps, args.warmup)
    log(f"T={args.tokens}: {main_res['ms_per_step'] * 1e3:.1f} us/step, {main_res['tokens_per_s']:.0f} tok/s, "
        f"{main_res['hbm_gbps']:.0f} GB/s")
    sweep = {}
    for tok in [int(t) for t in args.sweep.split(",") if t.strip()]:
        if tok == args.tokens:
            continue
        r = measure(tok, max(args.steps // 2, 10), args.warmup)
        sweep[f"T{tok}"] = {k: round(r[k], 3) for k in ("ms_per_step", "tokens_per_s", "hbm_gbps")}
        sweep[f"T{tok}"]["active_experts"] = r["active_experts"]
        log(f"T={tok}: {r['ms_per_step'] * 1e3:.1f} us/step, {r['tokens_per_s']:.0f} tok/s, {r['hbm_gbps']:.0f} GB/s")

    # ---- the same step with 4-bit packed backbones (group 128, as real checkpoints store SV)
    packed4 = None
    if args.packed4:
        from tris_moe_amd import packing
        from tris_moe_amd.qlinear import PackedQuantMatrix4bit

        pk = {p: packing.pack_4bit(layer["backbones"][p].astype(np.float32), 128) for p in projs}
        p4_bytes = sum(pk[p][k].nbytes for p in projs for k in ("qweight", "qzeros", "scales", "g_idx"))
        pcopies = [(pl, {p: PackedQuantMatrix4bit().set_from_payload(pk[p]).to(dev) for p in projs})
                   for pl, _ in copies]
        packed4 = {"backbone_bytes": int(p4_bytes), "group_size": 128}
        for tok in sorted({args.tokens, 1}):
            r = measure(tok, max(args.steps // 2, 10), args.warmup, pcopies, p4_bytes)
            packed4[f"T{tok}"] = {k: round(r[k], 3) for k in ("ms_per_step", "tokens_per_s", "hbm_gbps")}
            log(f"packed4 backbones T={tok}: {r['ms_per_step'] * 1e3:.1f} us/step, {r['tokens_per_s']:.0f} tok/s")
        del pcopies

    # ---- the same step with matrix-mode null-space compensation on every projection (rank 32 per expert)
    ns_line = None
    if args.ns:
        from tris_moe_amd import qlinear as ql

        rng = np.random.default_rng(args.seed)
        ranks = [32] * SPEC.num_experts
        ns_host = {"gate": synthetic.make_ns_payload(rng, SPEC.num_experts, SPEC.hidden, SPEC.intermediate, ranks),
                   "up": synthetic.make_ns_payload(rng, SPEC.num_experts, SPEC.hidden, SPEC.intermediate, ranks),
                   "down": synthetic.make_ns_payload(rng, SPEC.num_experts, SPEC.intermediate, SPEC.hidden, ranks)}
        ns_dev = {f"{p}_ns": ql.ns_payload_to_device(ns_host[p], dev) for p in projs}
        ncopies = [(dict(pl, **ns_dev), bb) for pl, bb in copies]
        ns_line = {"rank_per_expert": 32}
        for tok in sorted({args.tokens, 1}):
            r = measure(tok, max(args.steps // 2, 10), args.warmup, ncopies)
            ns_line[f"T{tok}"] = {k: round(r[k], 3) for k in ("ms_per_step", "tokens_per_s")}
            log(f"ns compensation T={tok}: {r['ms_per_step'] * 1e3:.1f} us/step, {r['tokens_per_s']:.0f} tok/s")
        del ncopies

    # ---- dominant kernel: the MFMA gate/up grouped GEMM over predecoded split bitmaps that the step runs,
    # one launch per layer copy, replayed from a graph on its own stream and timed there with HIP events
    x16, logits = main_res["x16"], main_res["logits"]
    w, sel = moe.route_topk(logits, SPEC.top_k, SPEC.renormalize)
    route = ext.build_grouped_route_device(sel, SPEC.num_experts, 4)
    rows = int(sel.numel())
    slots = min(SPEC.num_experts, rows)
    eid = route["expert_ids"][:slots]
    seg = route["segment_offsets"][: slots + 1]
    prob = route["problem_offsets"][: slots + 1]
    hid_g = ext.backbone_linear(x16, base_backbones["gate"], row_index=route["grouped_token_indices"])
    hid_u = ext.backbone_linear(x16, base_backbones["up"], row_index=route["grouped_token_indices"])
    nblk = int(layer["gate"]["q_gmap_gr_meta"].shape[1])
    decoded = []
    for pl, _ in copies:
        pair = []
        for p in ("gate", "up"):
            buf = torch.empty((slots, nblk, 128), dtype=torch.int32, device=dev)
            pair.append(ext.compact3_tris_precomputed_grouped_block_gr_predecode(
                buf, eid, pl[p]["q_gmap_gr_words"], pl[p]["q_gmap_gr_offsets"], pl[p]["q_gmap_gr_meta"],
                SPEC.rank // 32, SPEC.intermediate))
        decoded.append(pair)

    active = main_res["active"]
    launch, kname, kbytes, kind = gateup_kernel(ext, moe, synthetic, layer, rows, active, SPEC, hid_g, hid_u, eid,
                                                seg, prob, dev)

    def dual(i):
        launch(copies[i][0], decoded[i][0], decoded[i][1])

    kstream = torch.cuda.Stream(device=dev)
    kstream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(kstream):
        for i in range(len(copies)):
            dual(i)
        gk = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gk, stream=kstream):
            for i in range(len(copies)):
                dual(i)
        gk.replay()
        kstream.synchronize()
        ks, ke = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ks.record(kstream)
        for _ in range(args.kernel_reps):
            gk.replay()
        ke.record(kstream)
        kstream.synchronize()
    kernel_s = ks.elapsed_time(ke) / 1e3 / (args.kernel_reps * len(copies))
    achieved = kbytes / kernel_s / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": measured_traffic(args.tokens, kind),
                "kernel": kname, "kernel_us": round(kernel_s * 1e6, 2), "bytes_per_launch": int(kbytes)}
    log(f"gate/up grouped GEMM ({kind}): {kernel_s * 1e6:.1f} us/launch, {achieved:.0f} GB/s algorithmic")

    prefill = prefill_bench(args, layer, copies, dev) if args.prefill > 0 else None

    cpu = None
    if args.cpu_baseline:
        cpu = cpu_baseline(layer, main_res, SPEC)
        log(f"cpu baseline: {cpu}")

    line = {
        "metric": "MoE-layer tokens/sec + achieved HBM GB/s (decode), Mixtral-8x7B shape",
        "value": round(main_res["tokens_per_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(main_res["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "hbm_gbps": round(main_res["hbm_gbps"], 1),
        "config": {"workload": f"mixtral8x7b_moe_layer_decode_T{args.tokens}", "hidden": SPEC.hidden,
                   "experts": SPEC.num_experts, "intermediate": SPEC.intermediate, "top_k": SPEC.top_k,
                   "rank": SPEC.rank, "gmap_p": SPEC.gmap_p, "tokens": args.tokens,
                   "active_experts": main_res["active_experts"], "step_bytes": int(main_res["step_bytes"]),
                   "layer_copies": args.layers, "graph": True},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "sweep": sweep,
        "prefill": prefill,
        "packed4_backbones": packed4,
        "ns_compensation": ns_line,
    }
    print(json.dumps(line), flush=True)


def layer_flops_per_token(spec) -> int:
    """Algorithmic flops of one token through the layer: gate/up backbones, top_k x (gate/up expert GEMMs, down
    backbone, down expert GEMM)."""
    h, r, i, k = spec.hidden, spec.rank, spec.intermediate, spec.top_k
    return 2 * (2 * h * r) + k * (2 * (2 * r * i) + 2 * i * r + 2 * r * h)


def prefill_bench(args, layer, copies, dev):
    """C2: the same layer weights at --prefill tokens with N(0, 1) router logits,
    one full layer step (eager launches) per layer copy in turn; MFMA-bound, reported against the dense
    fp16 MFMA peak."""
    import torch

    from tris_moe_amd import moe, synthetic
    from tris_moe_amd.configs import C2_MIXTRAL_PREFILL as SPEC2

    T = args.prefill
    inp = synthetic.make_inputs(SPEC2, T, args.seed + T, layer["outlier_idx"])
    x16 = torch.from_numpy(inp["x"]).to(dev).to(torch.bfloat16).to(torch.float16)
    logits = torch.from_numpy(inp["router_logits"]).to(dev)

    def step(i):
        pl, bb = copies[i % len(copies)]
        return moe.grouped_moe_forward_from_logits(x16, logits, SPEC2.top_k, SPEC2.renormalize, pl, bb,
                                                   SPEC2.num_experts, torch.bfloat16)

    for i in range(3):
        step(i)
    torch.cuda.synchronize()
    steps = max(2 * len(copies), 20)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        step(i)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    flops = layer_flops_per_token(SPEC2) * T
    tflops = flops / (ms / 1e3) / 1e12
    log(f"prefill T={T}: {ms:.3f} ms/step, {T / (ms / 1e3):.0f} tok/s, {tflops:.1f} TFLOP/s")
    return {"workload": f"mixtral8x7b_moe_layer_prefill_T{T}", "tokens": T, "steps": steps,
            "ms_per_step": round(ms, 4), "tokens_per_s": round(T / (ms / 1e3), 1),
            "tflops": round(tflops, 2), "mfma_peak_tflops": MFMA_FP16_PEAK_TFLOPS,
            "mfma_frac": round(tflops / MFMA_FP16_PEAK_TFLOPS, 4), "flops_per_token": layer_flops_per_token(SPEC2)}


def gateup_kernel(ext, moe, synthetic, layer, rows, active, spec, hid_g, hid_u, eid, seg, prob, dev):
    """The gate/up grouped GEMM the layer step runs at `rows` routed rows: returns (launch(payloads,
    decoded_gate, decoded_up), kernel name, algorithmic bytes per launch).  Bytes: the routed experts'
    payloads with predecoded bitmaps, the two backbone outputs read, the fp16 output(s) written."""
    import torch

    names = ("qweight1", "qweight2_sparse", "qweight2_sparse_prefix", "c_map", "g_idx", "col_pack3", "row_pack3")
    slots = int(eid.numel())
    tile_bound = rows // 4 + slots + 1
    weights = synthetic.predecoded_nbytes(layer["gate"], active) + synthetic.predecoded_nbytes(layer["up"], active)
    if rows <= moe.FUSED_SWIGLU_MAX_ROWS:
        mlp = torch.empty((rows, spec.intermediate), dtype=torch.float16, device=dev)

        def launch(pl, dg, du):
            ext.compact3_tris_precomputed_grouped_swiglu_forward_block_gr_predecoded(
                hid_g, hid_u, eid, seg, prob, tile_bound, dg, *[pl["gate"][k] for k in names], du,
                *[pl["up"][k] for k in names], out=mlp)
        name = "grouped_mfma_kernel<2> (gate/up grouped GEMM + SwiGLU epilogue, predecoded bitmaps)"
        nbytes = weights + 2 * rows * spec.rank * 2 + rows * spec.intermediate * 2
        return launch, name, nbytes, "swiglu"
    g = torch.empty((rows, spec.intermediate), dtype=torch.float16, device=dev)
    u = torch.empty_like(g)

    def launch(pl, dg, du):
        ext.compact3_tris_precomputed_grouped_dual_forward_block_gr_predecoded(
            hid_g, hid_u, eid, seg, prob, tile_bound, dg, *[pl["gate"][k] for k in names], du,
            *[pl["up"][k] for k in names], True, out_a=g, out_b=u)
    name = "grouped_mfma_kernel<1> (gate and up grouped GEMMs, predecoded bitmaps)"
    nbytes = weights + 2 * rows * spec.rank * 2 + 2 * rows * spec.intermediate * 2
    return launch, name, nbytes, "dual"


def measured_traffic(tokens: int, kind: str):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    runs (scaled by a copy-kernel calibration), or None when no measurement matches this workload."""
    path = ROOT / "profiles" / f"grouped_mfma_{kind}_mixtral_decode_T{tokens}_traffic.json"
    try:
        return int(json.loads(path.read_text())["traffic_bytes"])
    except (OSError, ValueError, KeyError):
        return None


def profile_dominant_kernel(args, layer, payloads, backbones, spec, dev):
    """Eager launches of the dominant kernel at the bench workload, for hardware-counter runs."""
    import torch

    from tris_moe_amd import ext, moe, synthetic

    inp = synthetic.make_inputs(spec, args.tokens, args.seed + args.tokens, layer["outlier_idx"])
    x16 = torch.from_numpy(inp["x"]).to(dev).to(torch.bfloat16).to(torch.float16)
    logits = torch.from_numpy(inp["router_logits"]).to(dev)
    route = ext.route_topk_grouped(logits, spec.top_k, spec.renormalize, 4)
    rows = args.tokens * spec.top_k
    slots = min(spec.num_experts, rows)
    eid = route["expert_ids"][:slots]
    seg = route["segment_offsets"][: slots + 1]
    prob = route["problem_offsets"][: slots + 1]
    hid_g, hid_u = ext.backbone_linear_pair(x16, backbones["gate"], backbones["up"],
                                            row_index=route["grouped_token_indices"])
    nblk = int(layer["gate"]["q_gmap_gr_meta"].shape[1])
    dec = []
    for p in ("gate", "up"):
        buf = torch.empty((slots, nblk, 128), dtype=torch.int32, device=dev)
        dec.append(ext.compact3_tris_precomputed_grouped_block_gr_predecode(
            buf, eid, payloads[p]["q_gmap_gr_words"], payloads[p]["q_gmap_gr_offsets"],
            payloads[p]["q_gmap_gr_meta"], spec.rank // 32, spec.intermediate))
    active = sorted(set(route["selected_experts"].cpu().numpy().reshape(-1).tolist()))
    launch, kname, nbytes, kind = gateup_kernel(ext, moe, synthetic, layer, rows, active, spec, hid_g, hid_u, eid,
                                                seg, prob, dev)
    for _ in range(args.kernel_reps):
        launch(payloads, dec[0], dec[1])
    torch.cuda.synchronize()
    print(json.dumps({"kernel": kname, "kind": kind, "launches": args.kernel_reps, "bytes_per_launch": nbytes}))


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
        # variant: backbones resident (L x 23 MB on the device), only the expert payloads streamed
        st_e = streaming.GroupedPayloadStreamer(host, dev, num_slots=2, backbones=None)
        bb_res = [{q: torch.from_numpy(layer["backbones"][q]).to(dev) for q in streaming.PROJECTIONS} for _ in range(L)]
        stream_e_s = timed(lambda: streaming.streamed_forward(st_e, x16, logits, SPEC.top_k, SPEC.renormalize,
                                                              SPEC.num_experts, backbones=bb_res))
        expert_bytes = st_e.layer_nbytes(0)
        # the same stack resident in HBM: L distinct device copies (so every layer reads HBM, not the cache)
        pl0 = {q: qlinear.payload_to_device(layer[q], dev) for q in streaming.PROJECTIONS}
        bb0 = {q: torch.from_numpy(layer["backbones"][q]).to(dev) for q in streaming.PROJECTIONS}
        pls = [{q: {k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in pl0[q].items()}
                for q in streaming.PROJECTIONS} for _ in range(L)]
        bbs_dev = [{q: v.clone() for q, v in bb0.items()} for _ in range(L)]

        def resident():
            x = x16
            for i in range(L):
                x = moe.grouped_moe_forward_from_logits(x, logits[i], SPEC.top_k, SPEC.renormalize, pls[i],
                                                        bbs_dev[i], SPEC.num_experts, torch.bfloat16).to(torch.float16)
        resident_s = timed(resident)
        layer_bytes = st.layer_nbytes(0)
        results[f"p{p}"] = {
            "tokens_per_s": round(T / stream_s, 1), "ms_per_forward": round(stream_s * 1e3, 3),
            "resident_ms_per_forward": round(resident_s * 1e3, 3), "layer_bytes": int(layer_bytes),
            "h2d_gbps": round(L * layer_bytes / stream_s / 1e9, 2),
            "device_slot_bytes": int(2 * st.slot_bytes), "resident_model_bytes": int(L * layer_bytes),
            "experts_only": {"tokens_per_s": round(T / stream_e_s, 1), "ms_per_forward": round(stream_e_s * 1e3, 3),
                             "layer_bytes": int(expert_bytes),
                             "h2d_gbps": round(L * expert_bytes / stream_e_s / 1e9, 2)}}
        log(f"C4 p={p}: streamed {stream_s * 1e3:.2f} ms / {L} layers ({T / stream_s:.0f} tok/s, "
            f"{L * layer_bytes / stream_s / 1e9:.1f} GB/s host-to-device), experts only {stream_e_s * 1e3:.2f} ms, "
            f"resident {resident_s * 1e3:.2f} ms")
        del st, st_e, bb_res, host, bbs, pl0, bb0, pls, bbs_dev
        torch.cuda.synchronize()
    print(json.dumps({"metric": "C4 MoE-stack tokens/sec with whole-layer payload streaming (pinned host -> 2 "
                      "device slots), Mixtral-8x7B shape", "unit": "tokens/s", "n_gpus": 1,
                      "config": {"workload": f"mixtral8x7b_moe_stack_{L}layers_T{T}_streamed", "layers": L,
                                 "tokens": T, "slots": 2, "data": "synthetic"},
                      "results": results}), flush=True)


def cpu_baseline(layer, res, spec):
    """Time the CPU oracle (restated reference CPU path) on one full layer step: GR decode of every
    active expert's bitmaps (C), exact fp16 dequant (numpy), fp32 GEMMs; BLAS limited to one thread."""
    import numpy as np

    try:
        import oracle
        from threadpoolctl import threadpool_limits
    except Exception as exc:  # oracle library not built
        return {"error": repr(exc)}
    x = res["x16"].float().cpu().numpy().astype(np.float16)
    logits = res["logits"].cpu().numpy()
    w, sel = oracle.route_topk(logits, spec.top_k, spec.renormalize)
    payloads = {p: layer[p] for p in ("gate", "up", "down")}
    with threadpool_limits(limits=1):
        t0 = time.perf_counter()
        oracle.moe_layer(x, w, sel, payloads, layer["backbones"], spec.num_experts)
        dt = time.perf_counter() - t0
    tokens = x.shape[0]
    return {"value": round(tokens / dt, 3), "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"1 full layer step at T={tokens} ({res['active_experts']} active experts): GR decode + "
                      f"exact fp16 dequant of every active expert + fp32 GEMMs, {dt:.2f}s"}


if __name__ == "__main__":
    main()
