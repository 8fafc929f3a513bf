#!/usr/bin/env python3
"""Benchmark of the MI355X FP8 block-scaled MoE path (one JSON line).

Headline workload (made of config-2 layers): steady
batch-1 decode through 42 independent MoE layers (H=4096, I=1536, 288 routed
experts, top-8, one shared expert, FP32 router; 229 GB of E4M3 banks
resident in HBM), one BF16 token per step with a residual add, a fresh
seeded input every step.  One step (42 x 3 launches + the input draw) is
captured once as a HIP graph and replayed; `value` = microseconds per MoE
layer = step time / 42.  The dominant kernel (top-k prologue, routed
gate/up/SwiGLU, shared down) is the `roofline` entry, timed with
HIP events on its stream against the HBM roofline.

Also reported: the grouped prefill configs 4 (256 tokens, near-uniform) and 5 (2,048 tokens, Zipf
router bias) as routes/s with HBM and FP8-MFMA roofline fractions, a parity
sample against the CPU oracle, and the CPU oracle's own decode time on the
host cores (the reference has no CPU FP8 path; MLX is not installable).
"""

from __future__ import annotations

import argparse
import importlib
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path
from types import SimpleNamespace

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
PEAK_FP8_TFLOPS = 5000.0   # dense FP8 MFMA
SEED = 20260901


def parse():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=512)
    p.add_argument("--warmup", type=int, default=16)
    p.add_argument("--layers", type=int, default=42)
    p.add_argument("--kernel-steps", type=int, default=8, help="stage-graph replays (x8) for per-launch timing")
    p.add_argument("--prefill-iters", type=int, default=10)
    p.add_argument("--cpu-reps", type=int, default=5,
                   help="timed calls per config of the CPU comparator (median, after 2 warm-ups)")
    p.add_argument("--parity-layers", type=int, default=3)
    p.add_argument("--no-prefill", action="store_true")
    p.add_argument("--prefill-only", action="store_true",
                   help="one synthetic layer, configs 4 and 5 prefill only (for profiling the grouped GEMM)")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--ref-layers", type=int, default=8,
                   help="layers of the reference-shape leg (H=4096, I=2048); 0 skips it")
    p.add_argument("--layout", default="rows",
                   help="expert-bank layout: rows (the reference's row-major layout, the library's default), "
                        "tiled (16-row groups) or a row-group exponent 1..7")
    p.add_argument("--json-out", type=str, default="")
    p.add_argument("--traffic-run", action="store_true", help="short eager program for rocprofv3 --pmc passes")
    p.add_argument("--summarize-traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                   help="print the counter summary of two --pmc runs of --traffic-run")
    p.add_argument("--summarize-prefill", nargs=4, metavar=("TRACE_CSV", "FETCH_CSV", "WRITE_CSV", "BENCH_JSON"),
                   help="print the per-kernel summary of --prefill-only runs: a --kernel-trace run, two --pmc runs "
                        "and the JSON line of the traced run")
    return p.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def decode_layer_bytes(H, I, Is, E, k):
    """Algorithmic bytes of one decode layer: every weight byte touched once."""
    sr, sh, srs = math.ceil(I / 128), math.ceil(H / 128), math.ceil(Is / 128)
    router = E * H * 4 + E * 4
    gate_up = k * (2 * I * H + 2 * sr * sh * 4)
    down = k * (H * I + sh * sr * 4)
    shared = 3 * Is * H + (2 * srs * sh + sh * srs) * 4
    return {"router": router, "routed_gate_up": gate_up, "routed_down": down, "shared": shared,
            "activations": 2 * H * 2, "total": router + gate_up + down + shared + 2 * H * 2}


def step_launch_bytes(H, I, Is, E, k):
    """Algorithmic bytes of the three decode launches (each weight byte once,
    activations read / written once, the residual read once)."""
    sr, sh, srs = math.ceil(I / 128), math.ceil(H / 128), math.ceil(Is / 128)
    router_shared = E * H * 4 + (2 * Is * H + 2 * srs * sh * 4) + H * 2 + E * 4 + Is * 2
    gate_up = k * (2 * I * H + 2 * sr * sh * 4) + (Is * H + sh * srs * 4) + H * 2 + E * 4 * 2 + k * I * 2 + Is * 2 + H * 2
    down = k * (H * I + sh * sr * 4) + k * I * 2 + H * 2 + H * 2 + H * 2
    return {"router_shared": router_shared, "gate_up": gate_up, "down": down}


def main():
    args = parse()
    if args.summarize_traffic:
        summarize_traffic(*args.summarize_traffic)
        return
    if args.summarize_prefill:
        summarize_prefill(*args.summarize_prefill)
        return
    if args.gpus != 1:
        print(f"bench.py measures one MI355X; --gpus {args.gpus} is not supported on this single-GPU build "
              "(the multi-GPU sharding is described, not run)", file=sys.stderr)
        sys.exit(2)
    if args.traffic_run:
        traffic_run(args)
        return
    import numpy as np
    import torch

    pkg = importlib.import_module("glm53-flash-mlx_amd")
    syn = importlib.import_module("glm53-flash-mlx_amd.synthetic")
    N = importlib.import_module("glm53-flash-mlx_amd._native")
    packed = importlib.import_module("glm53-flash-mlx_amd.packed")

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = syn.layer_config()
    H, I, E, k = cfg.hidden_size, cfg.moe_intermediate_size, cfg.n_routed_experts, cfg.num_experts_per_tok
    Is = I * cfg.n_shared_experts
    L = 1 if args.prefill_only else args.layers

    # ------------------------------------------------------------ weights ---
    t0 = time.perf_counter()
    layers = []
    layout = int(args.layout) if args.layout.isdigit() else args.layout
    for layer in range(L):
        bank, shared, gate = syn.synth_layer(cfg, SEED, layer, dev, layout=layout)
        plan = packed.DecodePlan(H, I, Is, E, k, cfg.swiglu_limit)
        bank.code_flags()
        layers.append(SimpleNamespace(bank=bank, shared=shared, gate=gate, plan=plan))
    torch.cuda.synchronize()
    gen_s = time.perf_counter() - t0
    resident = sum(l.bank.nbytes for l in layers) + L * (3 * Is * H + E * H * 4)
    log(f"generated {L} layers, {resident / 1e9:.1f} GB resident, in {gen_s:.1f} s")

    if args.prefill_only:
        line = json.dumps({"prefill": bench_prefill(args, layers[0], cfg, dev, torch, np, pkg, syn),
                           "bank_layout": layers[0].bank.layout})
        print(line, flush=True)
        if args.json_out:
            Path(args.json_out).write_text(line + "\n")
        return

    # ------------------------------------------------------- decode graph ---
    x = torch.empty(H, dtype=torch.bfloat16, device=dev)
    counter = torch.zeros(1, dtype=torch.int32, device=dev)
    lib = N.lib()

    def step():
        N.check(lib.glm53_synth_step_input(N.ptr(x), H, SEED, 1.0, N.ptr(counter), N.stream_handle(dev)))
        for l in layers:
            l.plan.step(l.bank, l.shared, l.gate, x, x, x, N.STAGE_ALL, dev)

    def time_steps():
        for _ in range(2):
            step()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        torch.cuda.synchronize()
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        wall0 = time.perf_counter()
        start.record()
        for _ in range(args.steps):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / args.steps, time.perf_counter() - wall0

    ms_step, wall = time_steps()
    us_layer = ms_step * 1000.0 / L
    finite = bool(torch.isfinite(x.float()).all().item())
    log(f"decode: {ms_step:.3f} ms/step, {us_layer:.2f} us/layer (wall {wall:.2f} s, finite={finite})")

    bytes_layer = decode_layer_bytes(H, I, Is, E, k)
    layer_gbs = bytes_layer["total"] / (us_layer * 1e-6) / 1e9

    # ------------------------------------------- per-launch HIP-event timing --
    # Per-launch durations: a graph holds one launch kind for all L layers back
    # to back (each layer's own weights, so no launch is served from L2 /
    # MALL), replayed between two HIP events on the launch stream.  Event
    # pairs around single eager launches would time host enqueue latency and
    # the events' own cache flushes instead.
    def run_stage(mask):
        def run():
            for l in layers:
                l.plan.step(l.bank, l.shared, l.gate, x, x, x, mask, dev)
        return run

    stage_us = {}
    for name, mask in (("router", N.STAGE_ROUTER), ("gate_up", N.STAGE_GATE_UP), ("down", N.STAGE_DOWN)):
        stage_us[name] = time_graph(run_stage(mask), args.kernel_steps * 8, torch) / L
    router_us, gate_up_us, down_us = stage_us["router"], stage_us["gate_up"], stage_us["down"]
    probe = read_probe(lib, N, layers[-1].bank, dev, torch)
    copy = copy_probe(dev, torch)
    launch_bytes = step_launch_bytes(H, I, Is, E, k)
    gu_bytes = launch_bytes["gate_up"]
    gu_gbs = gu_bytes / (gate_up_us * 1e-6) / 1e9
    down_bytes = launch_bytes["down"]
    log(f"launches: router+shared {router_us:.2f} us, gate/up {gate_up_us:.2f} us ({gu_gbs:.0f} GB/s), "
        f"down {down_us:.2f} us ({down_bytes / (down_us * 1e-6) / 1e9:.0f} GB/s)")

    errors = [l.plan.error_flag() for l in layers]  # synchronous; after every timed replay
    if any(errors):
        raise RuntimeError(f"decode error flags after the timed replays: {errors}")

    # -------------------------------------------------------------- parity ---
    parity = parity_sample(args, layers, cfg, dev, torch, np)

    # ------------------------------------------------------ config-1 linear ---
    linear = bench_linear(dev, torch, pkg, syn)
    log(f"config-1 linear: {linear['us_per_linear']:.2f} us per GEMV in a graph")

    # ------------------------------------------------------------- prefill ---
    prefill = {}
    if not args.no_prefill:
        prefill = bench_prefill(args, layers[0], cfg, dev, torch, np, pkg, syn)

    # --------------------------------------------------------- CPU baseline ---
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args, layers, cfg, dev, torch, np, syn)
        linear["cpu_us"] = {"value": cpu["configs"]["1"], "kind": cpu["kind"], "cores": cpu["cores"]}
        for name, key in (("config4_256_tokens", "4"), ("config5_2048_tokens_zipf", "5")):
            if name in prefill:
                prefill[name]["cpu_us"] = {"value": cpu["configs"][key], "kind": cpu["kind"], "cores": cpu["cores"]}

    # ------------------------------------------------ reference shape leg ---
    layout_name = layers[0].bank.layout
    ref_shape = None
    if args.ref_layers > 0:
        del layers  # frees the config-2 stack (229 GB) before the I = 2048 layers are made
        torch.cuda.empty_cache()
        ref_shape = bench_reference_shape(args, layout, dev, torch, pkg, syn, N, packed)

    result = {
        "metric": "µs per MoE layer @ batch-1 decode (HBM GB/s %peak); prefill routes/s (%FP8 MFMA)",
        "value": round(us_layer, 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "e4m3xbf16->f32",
        "data": "synthetic (seeded N(0,0.02) weights quantised per 128x128 block, N(0,1) bf16 tokens)",
        "config": {
            "workload": f"BASELINE config 3: steady batch-1 decode, {L} independent config-2 MoE layers "
                        f"(H={H}, I={I}, {E} experts top-{k} + 1 shared, FP32 router, swiglu_limit=10), "
                        "BF16 residual, fresh seeded token per step, HIP-graph replay",
            "layers": L, "hidden": H, "intermediate": I, "experts": E, "top_k": k, "shared_experts": 1,
            "resident_bytes": resident, "parallelism": "single GPU",
            "bank_layout": layout_name,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "step_gate_up_kernel<16,4,3> (top-k, 8 routed gate/up rows with SwiGLU, shared down rows)",
            "achieved": round(gu_gbs, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(gu_gbs / PEAK_HBM_GBS, 4),
            "traffic": load_traffic("step_gate_up_kernel"),
            "traffic_source": "profiles/decode_traffic_pmc.md (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; calibrated)",
            "bytes_per_launch": gu_bytes,
            "avg_launch_us": round(gate_up_us, 3),
        },
        "decode": {
            "us_per_layer": round(us_layer, 3),
            "tokens_per_s": round(1000.0 / ms_step, 1),
            "layer_bytes": bytes_layer["total"],
            "layer_GBps": round(layer_gbs, 1),
            "layer_hbm_frac": round(layer_gbs / PEAK_HBM_GBS, 4),
            "launch_us": {"router_shared": round(router_us, 3), "gate_up": round(gate_up_us, 3),
                          "down_reduce": round(down_us, 3)},
            "launch_bytes": launch_bytes,
            "launch_GBps": {"router_shared": round(launch_bytes["router_shared"] / (router_us * 1e-6) / 1e9, 1),
                            "gate_up": round(gu_gbs, 1),
                            "down_reduce": round(down_bytes / (down_us * 1e-6) / 1e9, 1)},
            "launch_note": "stage-only graphs of one launch kind; kernel durations in profiles/",
            "achievable_read_GBps": probe,
            "copy_GBps": copy,
            "error_flags_clear": True,
            "weights_generated_s": round(gen_s, 1),
            "final_state_finite": finite,
        },
        "linear_config1": linear,
        "prefill": prefill,
        "parity": parity,
        "cpu_baseline": cpu,
        "reference_shape": ref_shape,
    }
    line = json.dumps(result)
    print(line, flush=True)
    if args.json_out:
        Path(args.json_out).write_text(line + "\n")


def time_graph(fn, reps, torch):
    """Mean microseconds per replay of a graph holding fn's launches."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        g.replay()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) * 1000.0 / reps


def bench_linear(dev, torch, pkg, syn, copies=24, reps=20):
    """y = block_fp8_linear(x bf16 [1,4096], W [4096,4096],
    s [32,32]) (fp8.py:254-299).  One graph replays the GEMV over `copies`
    distinct weight matrices (403 MB, more than the 256 MB last-level
    cache), so each launch streams its weights from HBM; the per-GEMV time
    includes the graph's kernel-to-kernel gaps."""
    K = N = 4096
    lins = []
    for i in range(copies):
        lin = pkg.BlockFP8Linear(K, N, device=dev)
        syn.fill_fp8(lin.weight, lin.weight_scale_inv, syn.key(91, i), 0.02)
        lins.append(lin)
    x = syn.normal_bf16((1, K), syn.key(91, "x"), device=dev)
    out = [None] * copies

    def run():
        for i, lin in enumerate(lins):
            out[i] = lin(x)

    us = time_graph(run, reps, torch) / copies
    nbytes = K * N + 4 * (K // 128) * (N // 128) + 2 * K + 2 * N
    finite = bool(torch.isfinite(out[-1].float()).all().item())
    del lins
    return {"us_per_linear": round(us, 3), "bytes": nbytes, "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
            "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4), "finite": finite,
            "note": f"graph of {copies} GEMVs over distinct weights; kernel time in profiles/"}


def read_probe(lib, N, bank, dev, torch):
    """Achievable streaming-read rate: a read-only kernel over regions of the
    size of one gate/up launch (and 4 GiB), taken from a resident bank."""
    out = {}
    blocks = 4096
    sink = torch.empty(4 * blocks, dtype=torch.int32, device=dev)
    base = bank.gate_up_weight
    span = base.numel()
    for label, size in (("113MB", 113309696 // 256 * 256), ("1GiB", 1 << 30), ("4GiB", min(4 << 30, span))):
        regions = max(1, min(16, span // size))

        def run(size=size, regions=regions):
            for r in range(regions):
                N.check(lib.glm53_probe_read(N.ctypes.c_void_p(base.data_ptr() + r * size), size, N.ptr(sink), blocks,
                                             N.stream_handle(dev)))
        us = time_graph(run, 4, torch) / regions
        out[label] = round(size / (us * 1e-6) / 1e9, 1)
    return out


def copy_probe(dev, torch):
    """STREAM-like device copy: 1 GiB read + 1 GiB written per copy, rate
    counting both (graph of 4 copies between distinct buffers)."""
    n = 1 << 30
    src = [torch.empty(n, dtype=torch.uint8, device=dev) for _ in range(2)]
    dst = [torch.empty(n, dtype=torch.uint8, device=dev) for _ in range(2)]

    def run():
        for i in range(4):
            dst[i % 2].copy_(src[(i + 1) % 2])

    us = time_graph(run, 4, torch) / 4
    del src, dst
    return round(2 * n / (us * 1e-6) / 1e9, 1)


def host_layer_subset(layer, ids, torch, np):
    idx = torch.as_tensor(np.asarray(ids, dtype=np.int64), device=layer.bank.gate_up_weight.device)
    b = layer.bank
    gate_up, down = b.reference_weights(idx)  # the oracle reads the reference row-major layout
    bank = SimpleNamespace(
        gate_up_weight=gate_up.cpu().numpy(),
        gate_up_scale_inv=b.gate_up_scale_inv.index_select(0, idx).cpu().numpy(),
        down_weight=down.cpu().numpy(),
        down_scale_inv=b.down_scale_inv.index_select(0, idx).cpu().numpy(),
        intermediate_size=b.intermediate_size)
    s = layer.shared
    shared = SimpleNamespace(gate=(s.gate_proj.weight.cpu().numpy(), s.gate_proj.weight_scale_inv.cpu().numpy()),
                             up=(s.up_proj.weight.cpu().numpy(), s.up_proj.weight_scale_inv.cpu().numpy()),
                             down=(s.down_proj.weight.cpu().numpy(), s.down_proj.weight_scale_inv.cpu().numpy()))
    return bank, shared


def bits(t, torch, np):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def parity_sample(args, layers, cfg, dev, torch, np):
    """One eager step; the first `parity_layers` layers are checked against the
    CPU oracle on the device's own expert selection."""
    from oracle import oracle as O

    syn = importlib.import_module("glm53-flash-mlx_amd.synthetic")
    x = syn.normal_bf16((cfg.hidden_size,), syn.key(SEED, "parity"), device=dev)
    worst = {"cosine": 1.0, "max_abs_rel": 0.0, "bit_exact_fraction": 1.0}
    router_mismatch = 0
    for l in layers[:args.parity_layers]:
        ids, scores = l.gate(x.reshape(1, -1))
        out = torch.empty_like(x)
        l.plan.step(l.bank, l.shared, l.gate, x, None, out, 7, dev)
        xb = bits(x, torch, np)
        ids_o, _ = O.router(xb[None], l.gate.weight.cpu().numpy(), l.gate.e_score_correction_bias.cpu().numpy())
        router_mismatch += int(set(ids_o[0].tolist()) != set(ids.cpu().numpy()[0].tolist()))
        hb, hs = host_layer_subset(l, ids.cpu().numpy()[0], torch, np)
        want = O.decode_moe(xb, hb, np.arange(8), scores.cpu().numpy()[0], cfg.swiglu_limit, hs)
        st = O.compare(bits(out, torch, np), want)
        worst["cosine"] = min(worst["cosine"], st["cosine"])
        worst["max_abs_rel"] = max(worst["max_abs_rel"], st["max_abs_rel"])
        worst["bit_exact_fraction"] = min(worst["bit_exact_fraction"], st["bit_exact_fraction"])
        x = (x.float() + out.float()).to(torch.bfloat16)
    worst["layers_checked"] = args.parity_layers
    worst["router_set_mismatches"] = router_mismatch
    worst["gates"] = "cosine >= 0.9999 and max_abs_rel <= 2e-2 vs CPU oracle (Direct semantics)"
    worst["pass"] = worst["cosine"] >= 0.9999 and worst["max_abs_rel"] <= 2e-2
    return {k: (round(v, 7) if isinstance(v, float) else v) for k, v in worst.items()}


def bench_prefill(args, layer, cfg, dev, torch, np, pkg, syn):
    H, I, E, k = cfg.hidden_size, cfg.moe_intermediate_size, cfg.n_routed_experts, cfg.num_experts_per_tok
    Is = I
    out = {}
    zipf_gate = pkg.Float32Gate(layer.gate.weight, syn.zipf_bias(E).to(dev), top_k=k)
    for name, tokens, gate in (("config4_256_tokens", 256, layer.gate), ("config5_2048_tokens_zipf", 2048, zipf_gate)):
        moe = pkg.SortedGroupedFP8MoE(layer.bank, cfg, gate, layer.shared)
        x = syn.normal_bf16((1, tokens, H), syn.key(SEED, name), device=dev)
        ids, _ = gate(x.reshape(tokens, H))
        counts = torch.bincount(ids.reshape(-1).long(), minlength=E).cpu().numpy()
        for _ in range(2):
            moe(x)
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(args.prefill_iters):
            y = moe(x)
        e.record()
        torch.cuda.synchronize()
        us = s.elapsed_time(e) * 1000.0 / args.prefill_iters
        routes = tokens * k
        touched = int((counts > 0).sum())
        expert_bytes = 3 * I * H + (2 * math.ceil(I / 128) * (H // 128) + (H // 128) * math.ceil(I / 128)) * 4
        weight_bytes = touched * expert_bytes + 3 * Is * H + E * H * 4
        act_bytes = 2 * tokens * H * 2
        flops = 2 * routes * 3 * I * H + 2 * tokens * 3 * Is * H
        gbs = (weight_bytes + act_bytes) / (us * 1e-6) / 1e9
        tflops = flops / (us * 1e-6) / 1e12
        out[name] = {
            "tokens": tokens, "routes": routes, "us": round(us, 1), "routes_per_s": round(routes / (us * 1e-6), 1),
            "tokens_per_s": round(tokens / (us * 1e-6), 1), "touched_experts": touched,
            "max_expert_share": round(float(counts.max()) / routes, 4),
            "experts_under_10_routes": int((counts < 10).sum()),
            "algorithmic_bytes": weight_bytes + act_bytes, "GBps": round(gbs, 1),
            "hbm_frac": round(gbs / PEAK_HBM_GBS, 4), "algorithmic_tflops": round(tflops, 1),
            "mfma_fp8_frac": round(tflops / PEAK_FP8_TFLOPS, 4),
            "binding_roofline": "hbm" if (weight_bytes + act_bytes) / (PEAK_HBM_GBS * 1e9) > flops / (PEAK_FP8_TFLOPS * 1e12) else "mfma",
            "finite": bool(torch.isfinite(y.float()).all().item()),
        }
        log(f"prefill {name}: {us:.1f} us, {gbs:.0f} GB/s, {tflops:.1f} TFLOP/s")
    return out


def bench_reference_shape(args, layout, dev, torch, pkg, syn, N, packed):
    """The reference's own measured shape (the real checkpoint: H=4096,
    I=2048, 288 experts top-8, one shared expert of I=2048) on `ref_layers`
    synthetic layers.  Decode: one step (input draw + 3 launches per layer)
    captured as a graph and replayed, as the headline; and, as the
    reference times its operator (probe_fused_packed_gate_up_swiglu_decode.py
    :396-411: gate, routed MoE and shared expert of one layer, then a host
    synchronisation), the median wall time of single host-synchronised
    eager layer calls.  Prefill: SortedGroupedFP8MoE at 256 tokens, routed
    near-uniformly and onto 51 experts (the count of the reference's
    layer-3 run, m3ultra512-grouped-fp8-layer3-20260828.json:149-152),
    event-timed and host-synchronised."""
    cfg = syn.layer_config(intermediate=2048)
    H, I, E, k = cfg.hidden_size, cfg.moe_intermediate_size, cfg.n_routed_experts, cfg.num_experts_per_tok
    L = args.ref_layers
    t0 = time.perf_counter()
    layers = []
    for layer in range(L):
        bank, shared, gate = syn.synth_layer(cfg, SEED + 1, layer, dev, layout=layout)
        layers.append(SimpleNamespace(bank=bank, shared=shared, gate=gate,
                                      plan=packed.DecodePlan(H, I, I, E, k, cfg.swiglu_limit)))
    torch.cuda.synchronize()
    log(f"reference shape: generated {L} layers (H={H}, I={I}) in {time.perf_counter() - t0:.1f} s")

    x = torch.empty(H, dtype=torch.bfloat16, device=dev)
    counter = torch.zeros(1, dtype=torch.int32, device=dev)
    lib = N.lib()

    def step():
        N.check(lib.glm53_synth_step_input(N.ptr(x), H, SEED + 1, 1.0, N.ptr(counter), N.stream_handle(dev)))
        for l in layers:
            l.plan.step(l.bank, l.shared, l.gate, x, x, x, N.STAGE_ALL, dev)

    reps = max(16, args.steps // 2)
    us_layer = time_graph(step, reps, torch) / L
    nbytes = decode_layer_bytes(H, I, I, E, k)["total"]
    gbs = nbytes / (us_layer * 1e-6) / 1e9

    # single host-synchronised layer calls, as the reference's operator timing
    xs = [syn.normal_bf16((H,), syn.key(SEED + 1, "eager", i), device=dev) for i in range(4 * L)]
    out = torch.empty_like(xs[0])
    wall = []
    for i, xi in enumerate(xs):
        l = layers[i % L]
        t = time.perf_counter()
        l.plan.step(l.bank, l.shared, l.gate, xi, None, out, N.STAGE_ALL, dev)
        torch.cuda.synchronize()
        if i >= L:  # the first pass over the layers is the warm-up
            wall.append((time.perf_counter() - t) * 1e6)
    errors = [l.plan.error_flag() for l in layers]
    if any(errors):
        raise RuntimeError(f"reference-shape decode error flags: {errors}")
    log(f"reference shape decode: {us_layer:.2f} us/layer in a graph ({gbs:.0f} GB/s), "
        f"{statistics.median(wall):.1f} us per host-synchronised call")

    tokens = 256
    l0 = layers[0]
    keep = torch.randperm(E, generator=torch.Generator().manual_seed(SEED))[:51]
    bias51 = torch.full((E,), -1.0, dtype=torch.float32)
    bias51[keep] = 0.0
    prefill = {}
    for name, gate in (("near_uniform", l0.gate),
                       ("51_experts", pkg.Float32Gate(l0.gate.weight, bias51.to(dev), top_k=k))):
        moe = pkg.SortedGroupedFP8MoE(l0.bank, cfg, gate, l0.shared)
        xp = syn.normal_bf16((1, tokens, H), syn.key(SEED + 1, "prefill", name), device=dev)
        ids, _ = gate(xp.reshape(tokens, H))
        counts = torch.bincount(ids.reshape(-1).long(), minlength=E).cpu()
        for _ in range(2):
            moe(xp)
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(args.prefill_iters):
            y = moe(xp)
        e.record()
        torch.cuda.synchronize()
        us = s.elapsed_time(e) * 1000.0 / args.prefill_iters
        synced = []
        for _ in range(5):
            t = time.perf_counter()
            y = moe(xp)
            torch.cuda.synchronize()
            synced.append((time.perf_counter() - t) * 1e6)
        touched = int((counts > 0).sum())
        prefill[name] = {"us": round(us, 1), "host_synchronised_us": round(statistics.median(synced), 1),
                         "touched_experts": touched, "max_expert_routes": int(counts.max()),
                         "routes_per_expert_mean": round(tokens * k / touched, 2),
                         "finite": bool(torch.isfinite(y.float()).all().item())}
        log(f"reference shape prefill {name}: {us:.1f} us ({touched} experts)")
    return {
        "shape": {"hidden": H, "intermediate": I, "shared_intermediate": I, "experts": E, "top_k": k,
                  "layers": L, "bank_layout": l0.bank.layout},
        "decode_us_per_layer": round(us_layer, 3),
        "decode_GBps": round(gbs, 1),
        "decode_hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
        "decode_layer_bytes": nbytes,
        "decode_host_synchronised_us": round(statistics.median(wall), 1),
        "prefill_256_tokens": prefill,
        "reference_m3_ultra": {
            "decode_layer_ms": 1.0629, "prefill_256_tokens_ms": 22.0797,
            "source": "bench-results/m3ultra512-fused-packed-gate-up-swiglu-decode-20260901.json "
                      "(operator.3.with_shared_expert.fused.median_ms: router + routed + shared of real layer 3, "
                      "host-synchronised) and m3ultra512-grouped-fp8-layer3-20260828.json (grouped_seconds median "
                      "at 256 tokens, 51 experts touched)"},
        "note": "context only, not vs_baseline: other hardware, real checkpoint weights vs synthetic ones",
    }


def cpu_baseline(args, layers, cfg, dev, torch, np, syn):
    """The CPU comparator on the host cores: oracle/cpu_direct.py, the
    reference's Direct path (fp8.py:343-400 with the FP32 router of
    patch.py:131-142) in C with FP32 accumulation, OpenMP threads and AVX2
    FMA -- the role the task gives to MLX's CPU stream -- on the inputs the
    GPU legs run: BASELINE config 1 (one [1, 4096] x [4096, 4096] linear,
    bench_linear's first matrix), config 2 (one batch-1 decode layer: layer
    0 of the stack, router included; config 3's layers are 42 such), config
    4 (256 tokens) and config 5 (2,048 tokens, Zipf router bias) on layer
    0.  Each is the median of `cpu_reps` calls after 2 warm-ups
    (scripts/probe_grouped_fp8_moe.py:46-60 of the reference), with the bank
    already in host memory (the reference layout, copied once)."""
    from oracle import cpu_direct as C

    H, I, E, k = cfg.hidden_size, cfg.moe_intermediate_size, cfg.n_routed_experts, cfg.num_experts_per_tok
    l0 = layers[0]
    gu, dw = l0.bank.reference_weights()
    bank = SimpleNamespace(gate_up_weight=gu.cpu().numpy(), gate_up_scale_inv=l0.bank.gate_up_scale_inv.cpu().numpy(),
                           down_weight=dw.cpu().numpy(), down_scale_inv=l0.bank.down_scale_inv.cpu().numpy(),
                           intermediate_size=I)
    del gu, dw
    s = l0.shared
    shared = SimpleNamespace(gate=(s.gate_proj.weight.cpu().numpy(), s.gate_proj.weight_scale_inv.cpu().numpy()),
                             up=(s.up_proj.weight.cpu().numpy(), s.up_proj.weight_scale_inv.cpu().numpy()),
                             down=(s.down_proj.weight.cpu().numpy(), s.down_proj.weight_scale_inv.cpu().numpy()))
    rw = l0.gate.weight.cpu().numpy()
    biases = {"4": l0.gate.e_score_correction_bias.cpu().numpy(), "5": syn.zipf_bias(E).numpy()}
    limit = cfg.swiglu_limit

    def timed(fn):
        for _ in range(2):
            fn()
        samples = []
        for _ in range(args.cpu_reps):
            t0 = time.perf_counter()
            fn()
            samples.append(time.perf_counter() - t0)
        return statistics.median(samples) * 1e6, sum(samples)

    lin_w = torch.empty((4096, 4096), dtype=torch.uint8, device=dev)
    lin_s = torch.empty((32, 32), dtype=torch.float32, device=dev)
    syn.fill_fp8(lin_w, lin_s, syn.key(91, 0), 0.02)
    lin_w, lin_s = lin_w.cpu().numpy(), lin_s.cpu().numpy()
    x_lin = bits(syn.normal_bf16((1, 4096), syn.key(91, "x"), device=dev), torch, np)
    x_dec = bits(syn.normal_bf16((H,), syn.key(SEED, "cpu", 0), device=dev), torch, np)[None]
    xs = {"4": bits(syn.normal_bf16((256, H), syn.key(SEED, "config4_256_tokens"), device=dev), torch, np),
          "5": bits(syn.normal_bf16((2048, H), syn.key(SEED, "config5_2048_tokens_zipf"), device=dev), torch, np)}

    def moe(x, bias):
        ids, sc = C.router(x, rw, bias, top_k=k)
        return C.direct_moe(x, bank, ids, sc, limit, shared)

    out, work = {}, 0.0
    out["1"], w = timed(lambda: C.linear(x_lin, lin_w, lin_s))
    work += w
    out["2"], w = timed(lambda: moe(x_dec, biases["4"]))
    work += w
    for key in ("4", "5"):
        out[key], w = timed(lambda key=key: moe(xs[key], biases[key]))
        work += w
    cores = C.num_threads()
    return {"value": round(out["2"], 1), "unit": "us/layer", "cores": cores, "kind": "port",
            "configs": {key: round(v, 1) for key, v in out.items()},
            "sample": f"the reference's Direct path restated in C (oracle/glm53_cpu_direct.c: FP32 accumulation, "
                      f"OpenMP x {cores} threads, AVX2 FMA) at BASELINE config 2 (value: one batch-1 decode layer, "
                      f"router + 8 routed + shared, layer 0 of the stack; config 3 = 42 such layers), and in "
                      f"'configs' (us per call) also config 1 (one 4096 x 4096 linear), 4 (256 tokens) and 5 "
                      f"(2,048 tokens, Zipf bias); median of {args.cpu_reps} calls after 2 warm-ups each "
                      f"({work:.1f} s of timed CPU work), bank in host memory; CPU {cpu_model()}"}


def traffic_run(args):
    """Short eager program for `rocprofv3 --pmc` passes: each decode launch on
    4 layers (4 times), the read probe over 113,309,696 B and a 64 MiB torch
    device copy, whose counter readings calibrate FETCH_SIZE / WRITE_SIZE."""
    import torch

    syn = importlib.import_module("glm53-flash-mlx_amd.synthetic")
    N = importlib.import_module("glm53-flash-mlx_amd._native")
    packed = importlib.import_module("glm53-flash-mlx_amd.packed")
    dev = torch.device("cuda:0")
    cfg = syn.layer_config()
    H, I, E, k = cfg.hidden_size, cfg.moe_intermediate_size, cfg.n_routed_experts, cfg.num_experts_per_tok
    layers = []
    for layer in range(4):
        bank, shared, gate = syn.synth_layer(cfg, SEED, layer, dev)
        bank.code_flags()
        layers.append(SimpleNamespace(bank=bank, shared=shared, gate=gate,
                                      plan=packed.DecodePlan(H, I, I, E, k, cfg.swiglu_limit)))
    x = syn.normal_bf16((H,), syn.key(SEED, "traffic"), device=dev)
    torch.cuda.synchronize()
    for _ in range(4):
        for l in layers:
            for mask in (N.STAGE_ROUTER, N.STAGE_GATE_UP, N.STAGE_DOWN):
                l.plan.step(l.bank, l.shared, l.gate, x, None, x, mask, dev)
    lib = N.lib()
    sink = torch.empty(4 * 4096, dtype=torch.int32, device=dev)
    probe_bytes = 113309696 // 256 * 256
    for r in range(4):
        N.check(lib.glm53_probe_read(N.ctypes.c_void_p(layers[r].bank.gate_up_weight.data_ptr()), probe_bytes,
                                     N.ptr(sink), 4096, N.stream_handle(dev)))
    src = torch.empty(64 << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"traffic run done: probe {probe_bytes} B, copy {64 << 20} B")


def summarize_traffic(fetch_csv, write_csv):
    """Per-kernel mean FETCH_SIZE / WRITE_SIZE (KiB per dispatch) from two
    rocprofv3 counter-collection CSVs, calibrated against the read probe
    (fetch) and the 64 MiB device copy (write); prints a markdown summary
    whose last line is the JSON that bench.py reads back."""
    import csv

    def load(path, counter):
        rows = {}
        for row in csv.DictReader(open(path)):
            if row.get("Counter_Name") != counter:
                continue
            name = row["Kernel_Name"]
            rows.setdefault(name, []).append(float(row["Counter_Value"]))
        return {n: (statistics.mean(v), len(v), sum(v)) for n, v in rows.items()}

    fetch, write = load(fetch_csv, "FETCH_SIZE"), load(write_csv, "WRITE_SIZE")

    def pick(table, key):
        hits = [n for n in table if key in n]
        return hits[0] if hits else None

    # totals over the calibration dispatches: the runtime may split one copy
    # into several dispatches, so calibrate on sums (4 probes, 4 copies)
    probe_bytes = 113309696 // 256 * 256
    copy_bytes = 64 << 20
    probe_k = pick(fetch, "probe_read_kernel")
    copy_kw = pick(write, "copyBuffer") or pick(write, "elementwise_kernel")
    fetch_scale = 4 * probe_bytes / (fetch[probe_k][2] * 1024.0)
    write_scale = 4 * copy_bytes / (write[copy_kw][2] * 1024.0)
    keys = ("step_router_shared_kernel", "step_gate_up_kernel", "step_down_kernel", "probe_read_kernel")
    print("| kernel | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | fetched B (calibrated) | written B (calibrated) |")
    print("|---|---|---|---|---|---|")
    out = {}
    for name in sorted(set(fetch) | set(write)):
        f = fetch.get(name, (float("nan"), 0, 0.0))
        w = write.get(name, (float("nan"), 0, 0.0))
        fb, wb = f[0] * 1024.0 * fetch_scale, w[0] * 1024.0 * write_scale
        print(f"| {name[:90]} | {f[1]} | {f[0]:.1f} | {w[0]:.1f} | {fb:.0f} | {wb:.0f} |")
        for key in keys:
            if key in name:
                out[key] = {"fetch_bytes": round(fb), "write_bytes": round(wb), "traffic_bytes": round(fb + wb)}
    print()
    print(f"calibration: 4 read probes of {probe_bytes} B -> FETCH_SIZE x {fetch_scale:.4f}; "
          f"4 device copies of {copy_bytes} B ({copy_kw[:60]}, {write[copy_kw][1]} dispatches) "
          f"-> WRITE_SIZE x {write_scale:.4f}")
    print()
    print("traffic_json: " + json.dumps({"fetch_scale": fetch_scale, "write_scale": write_scale, "kernels": out}))


def _prefill_calls(rows, order_key):
    """Dispatch rows of a --prefill-only run cut into MoE calls: a call runs
    from a many-token router launch to the reduction that ends it, and counts
    when it holds a grouped GEMM (the gate call bench_prefill makes before
    each config has none).  The first half of the calls is config 4, the
    second config 5."""
    rows = sorted(rows, key=order_key)
    calls, cur = [], None
    for r in rows:
        if "router_tile_kernel" in r["Kernel_Name"]:
            cur = []
            calls.append(cur)
        if cur is not None:
            cur.append(r)
            if "reduce_kernel" in r["Kernel_Name"] and "glm53::" in r["Kernel_Name"]:
                cur = None  # the call's last launch: the restore or Direct-order reduction
    calls = [c for c in calls if any("grouped_gemm" in r["Kernel_Name"] for r in c)]
    half = len(calls) // 2
    return {"4": calls[:half], "5": calls[half:]}


def _prefill_label(name, seen):
    """Short kernel label; repeated kernels of one call get their position."""
    short = name.replace("(anonymous namespace)::", "").split("(")[0].replace("void ", "").replace("glm53::", "")
    seen[short] = seen.get(short, 0) + 1
    return short if seen[short] == 1 else f"{short} #{seen[short]}"


def summarize_prefill(trace_csv, fetch_csv, write_csv, bench_json):
    """Per-kernel mean duration (kernel trace) and calibrated HBM bytes
    (FETCH_SIZE x the read-probe factor of the decode traffic summary,
    WRITE_SIZE 1:1) of one grouped prefill call at configs 4 and 5, with
    each GEMM's fetched bytes against its unique weight bytes."""
    import csv

    bench = json.loads(Path(bench_json).read_text())["prefill"]
    fetch_scale = 1.0
    for line in (ROOT / "profiles" / "decode_traffic_pmc.md").read_text().splitlines():
        if line.startswith("traffic_json: "):
            fetch_scale = json.loads(line[len("traffic_json: "):])["fetch_scale"]
    trace = _prefill_calls(list(csv.DictReader(open(trace_csv))), lambda r: int(r["Start_Timestamp"]))

    def counters(path, counter):
        rows = [r for r in csv.DictReader(open(path)) if r["Counter_Name"] == counter]
        return _prefill_calls(rows, lambda r: int(r["Dispatch_Id"]))

    fetch, write = counters(fetch_csv, "FETCH_SIZE"), counters(write_csv, "WRITE_SIZE")

    def per_kernel(calls, value):
        acc = {}
        for call in calls:
            seen = {}
            for r in call:
                acc.setdefault(_prefill_label(r["Kernel_Name"], seen), []).append(value(r))
        return {k: statistics.mean(v) for k, v in acc.items()}

    H, I = 4096, 1536
    unique = {"grouped_gemm_kernel<1,": 2 * I * H, "grouped_gemm_kernel<0,": I * H,
              "grouped_gemm_wide_kernel<1>": 2 * I * H, "grouped_gemm_wide_kernel<0>": I * H}
    print("| config | kernel | us | fetched MB | written MB | unique weight MB | fetched / unique |")
    print("|---|---|---|---|---|---|---|")
    out = {}
    for cfg, name in (("4", "config4_256_tokens"), ("5", "config5_2048_tokens_zipf")):
        us = per_kernel(trace[cfg], lambda r: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
        fb = per_kernel(fetch[cfg], lambda r: float(r["Counter_Value"]) * 1024.0 * fetch_scale)
        wb = per_kernel(write[cfg], lambda r: float(r["Counter_Value"]) * 1024.0)
        touched = bench[name]["touched_experts"]
        for k in us:
            u = next((b for key, b in unique.items() if k.startswith(key)), None)
            uw = (touched + 1) * u if u else None  # touched routed experts + the shared expert
            ratio = f"{fb[k] / uw:.2f}" if uw and k in fb else ""
            print(f"| {cfg} | {k} | {us[k]:.1f} | {fb.get(k, float('nan')) / 1e6:.1f} | "
                  f"{wb.get(k, float('nan')) / 1e6:.1f} | {uw / 1e6 if uw else '':{'.1f' if uw else ''}} | {ratio} |")
            out.setdefault(cfg, {})[k] = {"us": round(us[k], 2), "fetch_bytes": round(fb.get(k, 0)),
                                          "write_bytes": round(wb.get(k, 0))}
        print(f"| {cfg} | whole call (HIP events, traced run) | {bench[name]['us']:.1f} | | | | |")
    print()
    print(f"calls: {len(trace['4'])} + {len(trace['5'])} traced, {len(fetch['4'])} + {len(fetch['5'])} counted; "
          f"FETCH_SIZE x {fetch_scale:.4f}, WRITE_SIZE x 1; touched experts: config 4 "
          f"{bench['config4_256_tokens']['touched_experts']}, config 5 {bench['config5_2048_tokens_zipf']['touched_experts']}")
    print()
    print("prefill_json: " + json.dumps(out))


def load_traffic(kernel_key):
    """HBM bytes per launch for `kernel_key` from the committed counter
    summary, or None when no summary is present."""
    path = ROOT / "profiles" / "decode_traffic_pmc.md"
    try:
        for line in path.read_text().splitlines():
            if line.startswith("traffic_json: "):
                entry = json.loads(line[len("traffic_json: "):])["kernels"].get(kernel_key)
                return None if entry is None else entry["traffic_bytes"]
    except (OSError, ValueError, KeyError):
        return None
    return None


def cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


if __name__ == "__main__":
    main()
