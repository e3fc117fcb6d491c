#!/usr/bin/env python3
"""Benchmark of the MI355X fused-MoE operator (one expert-parallel rank, 32 of 256
experts) on one GPU.

    python bench.py [--steps K] [--warmup W] [--config IDX] [--gpus 1]

A step is one call of ``kernel(...)`` (route -> dispatch -> GEMM1+SwiGLU -> GEMM2 ->
combine) over one batch of seeded synthetic inputs already resident in HBM.  Weights
and activations rotate over copies so that a step does not find its weights in the
256 MB MALL (Infinity Cache): by default as many copies as put at least twice the
MALL's bytes between two uses of one copy (the algorithmic bytes of a call, from its
routing, times the other copies), and at least 4; ``--rotate N`` fixes the count.  The
copy count and that reuse distance are reported in the line.

The headline (``value``) is configs[1] of BASELINE.json (decode, T=64): W untimed
warmup steps, then exactly K timed steps between two ``torch.cuda.synchronize()``.
It is measured first, right after its inputs are generated on the GPU: each config's
CPU baseline leaves the GPU idle for seconds, after which a few warmup calls do not
bring the clocks back up (measured after another config's CPU baseline, the headline
read ~5% slower, in its per-call HIP events too).  Without ``--config``, every one of
the five configs is measured the same way (K steps after W warmup; the other configs
warm up for at least 20 steps and 20 ms of calls, so the GPU reaches steady clocks) and
reported in ``per_config``, in config order: latency, effective TFLOP/s, the fraction of the
whole call's roofline, the roofline of the dominant kernel measured with HIP events
that the runtime stamps at that kernel's own start and end on the library's stream
(the library's stage profiler, hipExtLaunchKernelGGL), and the CPU baseline (the reference's CPU-shaped path,
moe.cu:137-240, restated in torch-CPU) timed on this host on a bounded sample.

Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(REPO, "flash-infer-bench-starter-kit_amd")

METRIC = "fused-MoE latency (us) + eff. TFLOPS vs T; % HBM / FP8-MFMA roofline"
HEADLINE_CONFIG = 1
HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
BF16_PEAK_TFLOPS = 2500.0
MIN_CONFIG_WARMUP = 20
MIN_CONFIG_WARMUP_MS = 20.0
MALL_BYTES = 256 << 20           # MI355X Infinity Cache
MIN_ROTATE = 4


def _load(name: str, path: str):
    import importlib.util
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--config", type=int, default=None,
                    help="measure only this index of BASELINE.json configs (it becomes the headline)")
    ap.add_argument("--rotate", type=int, default=0,
                    help="input copies cycled over steps (0: enough for a reuse distance of "
                         "twice the MALL, at least 4)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="skip the HIP-graph replay timing")
    ap.add_argument("--no-quantizer", action="store_true", help="skip the quantizer leg")
    ap.add_argument("--cpu-budget-s", type=float, default=8.0,
                    help="CPU-baseline time budget per config (seconds)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run K device-to-device copies of MIB MiB (calibrates "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE against known bytes)")
    return ap.parse_args()


def copy_calibration(mib: int, steps: int) -> int:
    import torch
    n = mib * (1 << 20)
    src = torch.randint(0, 255, (n,), dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "steps": steps}))
    return 0


def traffic_from_profiles(workload: str, kernel: str):
    """HBM bytes per dispatch of `kernel` measured by rocprofv3 --pmc, committed as
    profiles/<kernel>_<workload>_traffic.txt ('hbm_bytes_per_dispatch: N')."""
    p = os.path.join(REPO, "profiles", f"{kernel}_{workload}_traffic.txt")
    if not os.path.exists(p):
        return None
    for line in open(p):
        if line.startswith("hbm_bytes_per_dispatch:"):
            return float(line.split(":", 1)[1])
    return None


def kernel_work(stage: str, T: int, n_a: int, e_a: int, touched: int) -> dict:
    """Algorithmic bytes and flops of one launch of a stage's kernel (never padded
    rows): the per-unit figures times the units the launch processes."""
    return {
        "gemm1": dict(bytes=e_a * (4096 * 7168 + 32 * 56 * 4) + touched * (7168 + 56 * 4) + n_a * 2048 * 2,
                      flops=n_a * 2 * 7168 * 4096, peak_tflops=FP8_PEAK_TFLOPS),
        # GEMM2 runs fp16 MFMA (streaming) or two FP8 MFMAs per product (prefill hi/lo):
        # either way its MFMA ceiling on the algorithmic flops is the 16-bit rate
        "gemm2": dict(bytes=e_a * (7168 * 2048 + 56 * 16 * 4) + n_a * 2048 * 2 + n_a * 7168 * 2,
                      flops=n_a * 2 * 2048 * 7168, peak_tflops=BF16_PEAK_TFLOPS),
        "combine": dict(bytes=n_a * 7168 * 2 + T * 7168 * 2 + T * 8 * 4 + n_a * 4, flops=0,
                        peak_tflops=FP8_PEAK_TFLOPS),
        "route": dict(bytes=T * 256 * 4 + 512 + T * 8 * 8, flops=0, peak_tflops=FP8_PEAK_TFLOPS),
        "dispatch": dict(bytes=T * 8 * 8 * 2 + n_a * 8, flops=0, peak_tflops=FP8_PEAK_TFLOPS),
    }[stage]


def roofline_of(stage: str, us: float, work: dict, workload: str) -> dict:
    dur_s = us * 1e-6
    ridge = work["peak_tflops"] * 1e12 / (HBM_PEAK_GBS * 1e9)
    intensity = work["flops"] / max(1, work["bytes"])
    if intensity > ridge:
        ach = work["flops"] / dur_s / 1e12
        roof = dict(bound="mfma", achieved=ach, peak=work["peak_tflops"], unit="TFLOP/s",
                    frac=ach / work["peak_tflops"])
    else:
        ach = work["bytes"] / dur_s / 1e9
        roof = dict(bound="hbm", achieved=ach, peak=HBM_PEAK_GBS, unit="GB/s", frac=ach / HBM_PEAK_GBS)
    roof.update(kernel=stage, algorithmic_bytes=work["bytes"], algorithmic_flops=work["flops"],
                kernel_us=us, traffic=traffic_from_profiles(workload, stage))
    return roof


def cpu_baseline(o, wl, base: dict, cfg, budget_s: float) -> dict:
    """reference_cpu_forward (moe.cu's control flow: fp32 dequant of all 32 experts in
    every call, routing, per-expert loop) on the host cores, 1 warmup + timed calls
    until the budget runs out (at most 5); median."""
    import numpy as np
    import torch
    ncores = len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)
    host = {kk: (v.detach().cpu() if isinstance(v, torch.Tensor) else v) for kk, v in base.items()}
    out_cpu = torch.empty_like(host["output"])
    cargs = wl.as_args({**host, "output": out_cpu})
    times = []
    tb = time.perf_counter()
    while True:
        c0 = time.perf_counter()
        o.reference_cpu_forward(*cargs)
        times.append(time.perf_counter() - c0)
        if len(times) >= 2 and (time.perf_counter() - tb + times[-1] > budget_s or len(times) >= 6):
            break
    timed = times[1:]
    del host, cargs
    return dict(value=float(np.median(timed)) * 1e3, unit="ms/call", cores=torch.get_num_threads(),
                kind="port",
                sample=f"{len(timed)} timed full calls of {cfg.name} (T={cfg.T}) after 1 warmup; "
                       f"fp32 dequant of all 32 experts inside each call as in moe.cu:164-176")


def measure_config(idx: int, a, k, wl, o, steps: int, warmup: int, quantizer: bool,
                   warm_ms: float = 0.0) -> dict:
    import numpy as np
    import torch

    cfg = wl.CONFIGS[idx]
    dev = torch.device("cuda:0")
    log(f"[bench] config {idx} {cfg.name} T={cfg.T}: generating inputs")
    base = wl.make_inputs(cfg, device=dev)
    T = cfg.T
    ws = torch.empty(k.workspace_bytes(T), dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()

    ids, _ = k.route(base["routing_logits"], base["routing_bias"], cfg.routed_scaling_factor)
    ids = ids.cpu()
    work = wl.algorithmic_work(ids, cfg.local_expert_offset, T)
    le = ids.to(torch.int64) - cfg.local_expert_offset
    touched = int(((le >= 0) & (le < 32)).any(dim=1).sum())
    n_a, e_a = work["N_a"], work["E_a"]

    # input copies: between two uses of one copy, the other copies' calls touch at least
    # twice the MALL's bytes (unless --rotate fixes the count)
    ncopies = a.rotate if a.rotate > 0 else \
        max(MIN_ROTATE, 1 + -(-2 * MALL_BYTES // max(1, work["bytes"])))
    copies = [base]
    for _ in range(ncopies - 1):
        copies.append({kk: (v.clone() if isinstance(v, torch.Tensor) else v) for kk, v in base.items()})
    arglists = [wl.as_args(c) for c in copies]
    rotation = {"copies": ncopies, "bytes_per_call": work["bytes"],
                "reuse_distance_bytes": (ncopies - 1) * work["bytes"], "mall_bytes": MALL_BYTES}
    log(f"[bench] config {idx}: {ncopies} input copies, reuse distance "
        f"{rotation['reuse_distance_bytes'] / 2**20:.0f} MiB")
    torch.cuda.synchronize()

    for i in range(warmup):
        k.forward(*arglists[i % len(arglists)], workspace=ws)
    torch.cuda.synchronize()
    # configs other than the headline: more warmup calls until warm_ms have passed
    w0, extra = time.perf_counter(), 0
    while (time.perf_counter() - w0) * 1e3 < warm_ms:
        for i in range(10):
            k.forward(*arglists[i % len(arglists)], workspace=ws)
        torch.cuda.synchronize()
        extra += 10
    warmup += extra

    # timed region: exactly `steps` calls back to back, synchronised on both sides
    stream = torch.cuda.current_stream(dev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        k.forward(*arglists[i % len(arglists)], workspace=ws)
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / steps
    log(f"[bench] config {idx}: {ms_per_step * 1e3:.1f} us per call")

    # per-call distribution: a second pass with events around each call (the event
    # packets themselves add a few microseconds per call, so this is not the value)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    for i in range(steps):
        starts[i].record(stream)
        k.forward(*arglists[i % len(arglists)], workspace=ws)
        ends[i].record(stream)
    torch.cuda.synchronize()
    ev_us = np.array([s.elapsed_time(e) * 1e3 for s, e in zip(starts, ends)])

    # per-stage kernel durations: the library times each kernel with a pair of HIP events
    # stamped at the kernel's start and end (launch gaps excluded), summed per stage
    k.profile_begin(steps)
    for i in range(steps):
        k.forward(*arglists[i % len(arglists)], workspace=ws, flags=k.FLAG_PROFILE)
    torch.cuda.synchronize()
    n_prof, stage_ms = k.profile_read()
    k.profile_end()
    stages_us = {name: ms * 1e3 for name, ms in zip(k.STAGES, stage_ms)}

    # HIP-graph replay: the forward only launches kernels on the caller's stream, so a
    # caller can capture a call and replay it (one graph per input copy, replayed
    # round-robin); reported beside the eager latency, which stays the value
    graph_us = None
    if not a.no_graph:
        side = torch.cuda.Stream(dev)
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            for al in arglists:
                k.forward(*al, workspace=ws)
        stream.wait_stream(side)
        torch.cuda.synchronize()
        graphs = []
        for al in arglists:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                k.forward(*al, workspace=ws)
            graphs.append(g)
        for i in range(warmup):
            graphs[i % len(graphs)].replay()
        torch.cuda.synchronize()
        g0 = time.perf_counter()
        for i in range(steps):
            graphs[i % len(graphs)].replay()
        torch.cuda.synchronize()
        graph_us = (time.perf_counter() - g0) * 1e6 / steps
        del graphs

    # the step before the operator: blockwise FP8 quantizer of bf16 activations
    # [T, 7168] (algorithmic bytes: read 2 B, write 1 B per element, 4 B per scale)
    quant = None
    if quantizer:
        xq = [torch.randn(T, 7168, device=dev).to(torch.bfloat16) for _ in range(2)]
        qo = torch.empty(T, 7168, dtype=torch.float8_e4m3fn, device=dev)
        qs = torch.empty(56, T, dtype=torch.float32, device=dev)
        for i in range(warmup):
            k.quantize_fp8_blockwise(xq[i % 2], qo, qs)
        qe0, qe1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        qe0.record(stream)
        for i in range(steps):
            k.quantize_fp8_blockwise(xq[i % 2], qo, qs)
        qe1.record(stream)
        torch.cuda.synchronize()
        q_us = qe0.elapsed_time(qe1) * 1e3 / steps
        q_bytes = T * 7168 * 3 + T * 56 * 4
        quant = dict(us=round(q_us, 3), bytes=q_bytes, gbs=q_bytes / (q_us * 1e-6) / 1e9,
                     hbm_frac=q_bytes / (q_us * 1e-6) / (HBM_PEAK_GBS * 1e9),
                     input="bf16 [T, 7168] -> e4m3 + fp32 [56, T]")
        del xq

    # roofline of the dominant kernel (algorithmic bytes / flops, never padded rows)
    lay = k.workspace_layout(T)
    dom = max(("gemm1", "gemm2", "combine", "route", "dispatch"), key=lambda s: stages_us[s])
    roof = roofline_of(dom, stages_us[dom], kernel_work(dom, T, n_a, e_a, touched), cfg.name)

    lat_us = ms_per_step * 1e3
    eff_tflops = work["flops"] / (lat_us * 1e-6) / 1e12
    floor_us = max(work["bytes"] / (HBM_PEAK_GBS * 1e9),
                   (n_a * 2 * 7168 * 4096) / (FP8_PEAK_TFLOPS * 1e12)
                   + (n_a * 2 * 2048 * 7168) / (BF16_PEAK_TFLOPS * 1e12)) * 1e6
    cpu = None
    if not a.no_cpu_baseline:
        log(f"[bench] config {idx}: CPU baseline (budget {a.cpu_budget_s}s)")
        cpu = cpu_baseline(o, wl, base, cfg, a.cpu_budget_s)
    res = {
        "config_index": idx,
        "workload": cfg.name,
        "T": T,
        "local_expert_offset": cfg.local_expert_offset,
        "hot_local_experts": list(cfg.hot_local_experts),
        "value": round(lat_us, 3),
        "unit": "us",
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 6),
        "dtype": {0: "fp8_e4m3 GEMM1 + fp16 GEMM2 (W2 widened exactly), fp32 accumulate",
                  1: "fp8_e4m3 GEMM1 + fp8 hi/lo GEMM2 (two FP8 MFMAs per product), fp32 accumulate",
                  2: "fp8_e4m3 GEMM1 (fp16 C, converted to fp8 hi/lo) + fp8 hi/lo GEMM2, "
                     "fp32 accumulate"}[lay.intermediate_format],
        "plan": {"tile_m": lay.tile_m, "dispatch_in_gemm1": bool(lay.dispatch_in_gemm1),
                 "combine_in_gemm2": bool(lay.combine_in_gemm2)},
        "latency_us": {"mean_wall": round(lat_us, 3), "median_event": float(np.median(ev_us)),
                       "p10_event": float(np.percentile(ev_us, 10)),
                       "p90_event": float(np.percentile(ev_us, 90)),
                       "graph_replay_wall": None if graph_us is None else round(graph_us, 3)},
        "eff_tflops": eff_tflops,
        "fp8_peak_frac": eff_tflops / FP8_PEAK_TFLOPS,
        "work": {"N_a": n_a, "E_a": e_a, "tokens_touched": touched, "flops": work["flops"],
                 "bytes": work["bytes"]},
        "roofline_floor_us": floor_us,
        "frac_of_floor": floor_us / lat_us,
        "hbm_frac_whole_call": work["bytes"] / (lat_us * 1e-6) / (HBM_PEAK_GBS * 1e9),
        "stages_us": stages_us,
        "profiled_calls": n_prof,
        "rotation": rotation,
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    if quant is not None:
        res["quantizer"] = quant
    del arglists, copies, base, ws
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res


def main() -> int:
    a = parse()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only (one expert-parallel rank's share); "
              f"--gpus {a.gpus} is not supported in this build.", file=sys.stderr)
        return 2
    if a.copy_calibration:
        return copy_calibration(a.copy_calibration, a.steps)

    import torch

    k = _load("moe_mi355_kernel", os.path.join(PKG, "kernel.py"))
    wl = _load("moe_mi355_workloads", os.path.join(PKG, "workloads.py"))
    k._build_extension()  # fail loudly before any timing if the library is missing
    o = None if a.no_cpu_baseline else _load("moe_oracle", os.path.join(REPO, "oracle", "moe_oracle.py"))
    torch.cuda.set_device(torch.device("cuda:0"))

    head_idx = HEADLINE_CONFIG if a.config is None else a.config
    # the headline first (see the module docstring), then the others in config order
    order = [a.config] if a.config is not None else \
        [head_idx] + [i for i in range(len(wl.CONFIGS)) if i != head_idx]
    results = {}
    for idx in order:
        head = idx == head_idx
        results[idx] = measure_config(idx, a, k, wl, o, a.steps,
                                      a.warmup if head else max(a.warmup, MIN_CONFIG_WARMUP),
                                      quantizer=(head and not a.no_quantizer),
                                      warm_ms=0.0 if head else MIN_CONFIG_WARMUP_MS)
    h = results[head_idx]
    line = {
        "metric": METRIC,
        "value": h["value"],
        "unit": "us",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": h["ms_per_step"],
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": h["dtype"],
        "data": "synthetic (seeded N(0,1) logits/hidden, N(0,0.02) weights, block-quantised)",
        "config": {"workload": h["workload"], "T": h["T"],
                   "local_expert_offset": h["local_expert_offset"],
                   "routed_scaling_factor": wl.CONFIGS[head_idx].routed_scaling_factor,
                   "hot_local_experts": h["hot_local_experts"],
                   "rotate_copies": h["rotation"]["copies"],
                   "reuse_distance_bytes": h["rotation"]["reuse_distance_bytes"],
                   "parallelism": "ep-rank (32 of 256 experts) on 1 GPU"},
        "latency_us": h["latency_us"],
        "eff_tflops": h["eff_tflops"],
        "work": h["work"],
        "roofline_floor_us": h["roofline_floor_us"],
        "frac_of_floor": h["frac_of_floor"],
        "hbm_frac_whole_call": h["hbm_frac_whole_call"],
        "stages_us": h["stages_us"],
        "profiled_calls": h["profiled_calls"],
        "roofline": h["roofline"],
        "cpu_baseline": h["cpu_baseline"],
        "quantizer": h.get("quantizer"),
        "per_config": [results[i] for i in sorted(results)],
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
