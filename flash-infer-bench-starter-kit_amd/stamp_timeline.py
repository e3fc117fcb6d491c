"""Timeline of one decode call (T <= 64) from in-kernel stamps, in microseconds.

The library built with ``-DMOE_MI355_STAMPS`` (``python build.py --stamps``, which this
script runs when ``libmoe_mi355_stamps.so`` is missing or stale) has its decode kernels
write the device's constant 100 MHz clock at every workgroup's start and end: the route,
the GEMM1 with the dispatch folded in (also when its items start, after the dispatch),
the GEMM2 (streaming, or with the combine folded in) and the combine.  The script runs
one BASELINE config on cuda:0 with its inputs rotating over ``--copies`` copies, in
bursts of calls issued back to back; after each burst it reads the stamps, which then
hold the burst's last call (a call in the steady state of a stream of calls).  It prints
the median over ``--samples`` bursts, relative to the call's first workgroup start (the
route kernel's, or at T <= 8 the GEMM1's, which routes the tokens itself), of
each kernel's first and last workgroup start, the median and last workgroup end, and
the gap from the previous kernel's last end to the next kernel's first start.

Usage: python stamp_timeline.py --config 0 [--samples 60] [--copies 8] [--burst 6]
       [--markdown]
"""
from __future__ import annotations

import argparse
import ctypes
import importlib.util
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SLOTS = 8192          # kStampSlots (csrc/stamps.h)
CLOCK_US = 0.01       # one tick of the 100 MHz constant clock


def _load(name, path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod          # dataclasses look their module up there
    spec.loader.exec_module(mod)
    return mod


# kernel, stamps per workgroup, reader suffix
TABLES = [("route", 2, "route"), ("gemm1", 3, "gemm1"), ("gemm2", 2, "gemm2"),
          ("gemm2+combine", 2, "gemm2_combine"), ("combine", 2, "combine")]


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--config", type=int, default=0)
    ap.add_argument("--samples", type=int, default=60)
    ap.add_argument("--copies", type=int, default=8)
    ap.add_argument("--burst", type=int, default=6)
    ap.add_argument("--markdown", action="store_true")
    a = ap.parse_args()

    import torch
    if not torch.cuda.is_available():
        print("stamp_timeline.py needs a GPU", file=sys.stderr)
        return 2
    build = _load("moe_mi355_build", os.path.join(HERE, "build.py"))
    lib_path = build.ensure_built(stamps=True)
    k = _load("moe_mi355_kernel", os.path.join(HERE, "kernel.py"))
    k._LIB_PATH = lib_path
    wl = _load("moe_mi355_workloads", os.path.join(HERE, "workloads.py"))
    cfg = wl.CONFIGS[a.config]
    if cfg.T > 64:
        print("the stamps cover the decode chain (T <= 64) only", file=sys.stderr)
        return 2

    d = wl.make_inputs(cfg, device="cuda")
    copies = [d] + [{n: (v.clone() if isinstance(v, torch.Tensor) else v) for n, v in d.items()}
                    for _ in range(a.copies - 1)]
    ws = torch.empty(k.workspace_bytes(cfg.T), dtype=torch.uint8, device="cuda")
    k.forward(*wl.as_args(d), workspace=ws)
    torch.cuda.synchronize()
    lib = ctypes.CDLL(lib_path)
    buf = np.zeros(SLOTS, dtype=np.uint64)
    readers = {}
    for name, _, suffix in TABLES:
        f = getattr(lib, f"moe_mi355_stamps_{suffix}")
        f.restype, f.argtypes = ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]
        readers[name] = f

    def read(name):
        if readers[name](buf.ctypes.data_as(ctypes.c_void_p), 0) != 0:
            raise RuntimeError(f"reading the {name} stamps failed")
        return buf.astype(np.int64)

    for i in range(20):
        k.forward(*wl.as_args(copies[i % len(copies)]), workspace=ws)
    torch.cuda.synchronize()
    rows = {}
    for smp in range(a.samples):
        for name in readers:
            if readers[name](None, 1) != 0:
                raise RuntimeError("resetting the stamps failed")
        for i in range(a.burst):
            k.forward(*wl.as_args(copies[(smp * a.burst + i) % len(copies)]), workspace=ws)
        torch.cuda.synchronize()
        t = {name: read(name).copy() for name in readers}
        starts = [t[name][:(SLOTS // per) * per].reshape(-1, per)[:, 0] for name, per, _ in TABLES]
        t0 = min(x[x > 0].min() for x in starts if (x > 0).any())
        prev_end = None
        for name, per, _ in TABLES:
            m = t[name][:(SLOTS // per) * per].reshape(-1, per)
            m = m[m[:, 0] > 0]
            if len(m) == 0:
                continue
            us = (m - t0) * CLOCK_US
            ends = us[:, per - 1]
            vals = {"workgroups": float(len(m)), "first start": us[:, 0].min(),
                    "last start": us[:, 0].max(), "median end": float(np.median(ends)),
                    "last end": ends.max()}
            if per == 3:
                vals["median items start"] = float(np.median(us[:, 1]))
            vals["gap before"] = us[:, 0].min() - prev_end if prev_end is not None else 0.0
            prev_end = ends.max()
            for key, v in vals.items():
                rows.setdefault((name, key), []).append(v)

    cols = ["workgroups", "first start", "median items start", "last start", "median end",
            "last end", "gap before"]
    title = f"config {a.config} (T = {cfg.T}, offset {cfg.local_expert_offset}), {a.samples} samples"
    if a.markdown:
        print(f"Timeline of one call, {title} (µs from the call's first workgroup start, medians):\n")
        print("| kernel | " + " | ".join(cols) + " |")
        print("|---" * (len(cols) + 1) + "|")
    else:
        print(title)
    for name, _, _ in TABLES:
        if (name, "workgroups") not in rows:
            continue
        cells = []
        for c in cols:
            v = rows.get((name, c))
            cells.append("" if v is None else (f"{np.median(v):.0f}" if c == "workgroups" else f"{np.median(v):.2f}"))
        if a.markdown:
            print(f"| {name} | " + " | ".join(cells) + " |")
        else:
            print(f"  {name:14s} " + "  ".join(f"{c}={x}" for c, x in zip(cols, cells) if x))
    return 0


if __name__ == "__main__":
    sys.exit(main())
