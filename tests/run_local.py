#!/usr/bin/env python3
"""Local workload runner: every workload through the operator's DPS entry point, with a
status, GPU latency, the CPU reference's latency, the speedup and the numerical error
against the fp32 oracle -- what the reference's scripts/run_local.py (lines 30-98)
reports per workload through the flashinfer-bench harness, which is not available here.

    python tests/run_local.py                      # the five BASELINE configs
    python tests/run_local.py --configs 0,1        # some of them
    python tests/run_local.py --workload w.safetensors [--workload ...]

Workload files (safetensors) hold the kernel's ten inputs under their argument names:
routing_logits fp32 [T,256], routing_bias bf16 [256], hidden_states float8_e4m3fn
[T,7168], hidden_states_scale fp32 [56,T], gemm1_weights float8_e4m3fn [32,4096,7168],
gemm1_weights_scale fp32 [32,32,56], gemm2_weights float8_e4m3fn [32,7168,2048],
gemm2_weights_scale fp32 [32,56,16], local_expert_offset int64 scalar and
routed_scaling_factor fp32 scalar (``save_workload`` writes one).

Status per workload: PASSED when every checked output element satisfies
|gpu - ref| <= 1e-2 + 1e-2 |ref| against the oracle's fp32 result (all tokens up to
T = 64, a seeded sample of tokens beyond) and the output is finite;
INCORRECT_NUMERICAL otherwise; RUNTIME_ERROR when the call raises.  Timing: W warmup
calls, then `trials` runs of `iterations` calls between HIP events on the current
stream (inputs rotate over 4 copies so the 256 MB MALL cannot hold the weights); the
latency is the median over trials.  The CPU reference is the oracle's
reference_cpu_forward (moe.cu's control flow) on this host's cores.
This runner is test infrastructure: it uses the oracle as the checker.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
sys.path.insert(0, HERE)

DEFINITION = "moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048"
ATOL = 1e-2
RTOL = 1e-2
ARG_NAMES = ("routing_logits", "routing_bias", "hidden_states", "hidden_states_scale",
             "gemm1_weights", "gemm1_weights_scale", "gemm2_weights", "gemm2_weights_scale",
             "local_expert_offset", "routed_scaling_factor")


def check_output(got, ref) -> dict:
    """Error statistics of a bf16 output against the fp32 reference rows, and the
    status they imply."""
    import torch
    got = got.float()
    err = (got - ref).abs()
    finite = bool(torch.isfinite(got).all())
    bound = ATOL + RTOL * ref.abs()
    within = err <= bound
    rel = err / ref.abs().clamp_min(1e-6)
    stats = dict(max_abs_error=float(err.max()) if err.numel() else 0.0,
                 max_rel_error=float(rel.max()) if rel.numel() else 0.0,
                 frac_within=float(within.float().mean()) if within.numel() else 1.0,
                 checked_elements=int(err.numel()))
    stats["status"] = "PASSED" if finite and bool(within.all()) else "INCORRECT_NUMERICAL"
    return stats


def format_result(name: str, r: dict) -> str:
    """One line per workload, in the layout of the reference's print_results."""
    line = f"  Workload {name}: {r['status']}"
    if r.get("latency_ms") is not None:
        line += f" | {r['latency_ms']:.3f} ms"
    if r.get("reference_latency_ms") is not None:
        line += f" | ref {r['reference_latency_ms']:.1f} ms"
    if r.get("speedup_factor") is not None:
        line += f" | {r['speedup_factor']:.2f}x speedup"
    if r.get("max_abs_error") is not None:
        line += f" | abs_err={r['max_abs_error']:.2e}, rel_err={r['max_rel_error']:.2e}"
    if r.get("error"):
        line += f" | {r['error']}"
    return line


def print_results(results: dict) -> None:
    for def_name, traces in results.items():
        print(f"\n{def_name}:")
        for name, r in traces.items():
            print(format_result(name, r))


def save_workload(path: str, inputs: dict) -> None:
    """Write a workload file of the layout run_local reads (host copies of `inputs`)."""
    import torch
    from safetensors.torch import save_file
    d = {k: inputs[k].detach().cpu().contiguous() for k in ARG_NAMES[:8]}
    d["local_expert_offset"] = torch.tensor(int(inputs["local_expert_offset"]), dtype=torch.int64)
    d["routed_scaling_factor"] = torch.tensor(float(inputs["routed_scaling_factor"]), dtype=torch.float32)
    save_file(d, path)


def load_workload(path: str, device) -> dict:
    import torch
    from safetensors.torch import load_file
    f = load_file(path)
    missing = [k for k in ARG_NAMES if k not in f]
    if missing:
        raise ValueError(f"{path}: missing {missing}")
    d = {k: f[k].to(device) for k in ARG_NAMES[:8]}
    d["local_expert_offset"] = int(f["local_expert_offset"].item())
    d["routed_scaling_factor"] = float(f["routed_scaling_factor"].item())
    T = d["routing_logits"].shape[0]
    d["output"] = torch.empty(T, 7168, dtype=torch.bfloat16, device=device)
    return d


def run_workload(d: dict, *, warmup: int = 3, iterations: int = 100, trials: int = 5,
                 check_tokens: int = 32, cpu_runs: int = 1, tamper=None) -> dict:
    """Run one workload; `tamper` (tests only) edits the output before it is checked."""
    import numpy as np
    import torch
    from conftest import oracle, pkg
    k = pkg("kernel")
    wl = pkg("workloads")
    o = oracle()
    T = d["routing_logits"].shape[0]
    res = dict(T=T, local_expert_offset=int(d["local_expert_offset"]))
    try:
        out = torch.full_like(d["output"], float("nan"))
        k.kernel(*wl.as_args({**d, "output": out}))
        torch.cuda.synchronize()
    except Exception as e:        # the harness reports a failing solution the same way
        res.update(status="RUNTIME_ERROR", error=f"{type(e).__name__}: {e}")
        return res
    if tamper is not None:
        tamper(out)
    toks = list(range(T)) if T <= 64 else sorted(
        np.random.default_rng(T).choice(T, min(T, check_tokens), replace=False).tolist())
    ids, w = o.route(d["routing_logits"], d["routing_bias"], d["routed_scaling_factor"])
    ref = o.expert_forward(d["hidden_states"], d["hidden_states_scale"], d["gemm1_weights"],
                           d["gemm1_weights_scale"], d["gemm2_weights"], d["gemm2_weights_scale"],
                           ids, w, d["local_expert_offset"], tokens=toks)
    got = out[torch.as_tensor(toks, device=out.device)].cpu()
    res.update(check_output(got, ref))
    res["checked_tokens"] = len(toks)

    copies = [d] + [{kk: (v.clone() if isinstance(v, torch.Tensor) else v) for kk, v in d.items()}
                    for _ in range(3)]
    arglists = [wl.as_args(c) for c in copies]
    stream = torch.cuda.current_stream()
    for i in range(warmup):
        k.kernel(*arglists[i % 4])
    per_trial = []
    for _ in range(trials):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(iterations):
            k.kernel(*arglists[i % 4])
        e1.record(stream)
        torch.cuda.synchronize()
        per_trial.append(e0.elapsed_time(e1) / iterations)
    res["latency_ms"] = float(np.median(per_trial))
    del copies, arglists

    if cpu_runs > 0:
        torch.set_num_threads(len(os.sched_getaffinity(0)))
        host = {kk: (v.cpu() if isinstance(v, torch.Tensor) else v) for kk, v in d.items()}
        hout = torch.empty(T, 7168, dtype=torch.bfloat16)
        times = []
        for _ in range(cpu_runs):
            t0 = time.perf_counter()
            o.reference_cpu_forward(*[host[n] for n in ARG_NAMES], hout)
            times.append((time.perf_counter() - t0) * 1e3)
        res["reference_latency_ms"] = float(np.median(times))
        res["reference_cores"] = torch.get_num_threads()
        res["speedup_factor"] = res["reference_latency_ms"] / res["latency_ms"]
    return res


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--configs", default="0,1,2,3,4", help="BASELINE config indices ('' for none)")
    ap.add_argument("--workload", action="append", default=[], help="safetensors workload file")
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--iterations", type=int, default=100)
    ap.add_argument("--trials", type=int, default=5)
    ap.add_argument("--check-tokens", type=int, default=32)
    ap.add_argument("--cpu-runs", type=int, default=1, help="timed CPU-reference calls (0: none)")
    ap.add_argument("--json", default=None, help="also write the results here")
    a = ap.parse_args()

    import torch
    from conftest import pkg
    wl = pkg("workloads")
    dev = torch.device("cuda:0")
    results = {DEFINITION: {}}
    jobs = [(wl.CONFIGS[int(i)].name, ("config", int(i))) for i in a.configs.split(",") if i.strip()]
    jobs += [(os.path.basename(p), ("file", p)) for p in a.workload]
    for name, (kind, what) in jobs:
        print(f"[run_local] {name}", file=sys.stderr, flush=True)
        d = wl.make_inputs(wl.CONFIGS[what], device=dev) if kind == "config" else load_workload(what, dev)
        results[DEFINITION][name] = run_workload(d, warmup=a.warmup, iterations=a.iterations,
                                                 trials=a.trials, check_tokens=a.check_tokens,
                                                 cpu_runs=a.cpu_runs)
        del d
        torch.cuda.empty_cache()
    print_results(results)
    if a.json:
        with open(a.json, "w") as f:
            json.dump(results, f, indent=1)
    ok = all(r["status"] == "PASSED" for r in results[DEFINITION].values())
    return 0 if ok else 1


if __name__ == "__main__":
    sys.exit(main())
