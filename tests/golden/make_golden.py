"""Write the committed golden fixtures of the fused-MoE path (run on a CPU).

The reference ships no golden vectors for this path, and its own implementation cannot
run here (CUDA/CUTLASS only), so these fixtures are the CPU oracle's answers, frozen
after the oracle was pinned against independent library routines and closed forms.
They guard both sides: the CPU tests check the oracle still reproduces them, and the
GPU tests check the HIP path against them without recomputing anything.

Fixtures (numpy .npz, no pickles):
  routing.npz   routing inputs (logits fp32, bias bf16 bits, factor) and the expected
                top-8 ids and weight bits; cases: all-equal logits, half-integer ties,
                hot bias, large logits, a duplicated maximum, plain random
  dispatch.npz  expert offsets, permutation, weights, inverse map and row tiles for
                one routing at local offsets 0 / 64 / 224 and tile heights 16 / 64
  forward.npz   a 6-token end-to-end case: crafted logits that route tokens to local
                experts {5, 9, 20} (one token to none); hidden states and scales
                stored; expert weights regenerated from a seed (they are 1.4 GB) with
                a checksum to detect generator drift; expected fp32 accumulator

Usage:  python tests/golden/make_golden.py      (rewrites the three files)
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from conftest import oracle, pkg  # noqa: E402

E_GLOBAL, TOP_K = 256, 8
FORWARD_SEED = 20261201
FORWARD_EXPERTS = (5, 9, 20)


def routing_cases():
    """(name, logits [T,256] fp32, bias bf16 [256], factor) tuples."""
    rng = np.random.default_rng(7)
    zb = torch.zeros(E_GLOBAL, dtype=torch.bfloat16)
    rb = (torch.from_numpy(rng.standard_normal(E_GLOBAL).astype(np.float32)) * 0.1).to(torch.bfloat16)
    cases = [("equal", np.zeros((4, E_GLOBAL), np.float32), zb, 2.5)]
    lg = (np.round(rng.standard_normal((48, E_GLOBAL)) * 2) / 2).astype(np.float32)
    cases.append(("half_int_ties", lg, zb, 2.5))
    hot = torch.zeros(E_GLOBAL)
    hot[[3, 11, 19, 27, 200]] = 3.0
    cases.append(("hot_bias", rng.standard_normal((24, E_GLOBAL)).astype(np.float32),
                  hot.to(torch.bfloat16), 1.0))
    cases.append(("large", (rng.standard_normal((16, E_GLOBAL)) * 60).astype(np.float32), rb, 2.5))
    dup = np.zeros((4, E_GLOBAL), np.float32)
    dup[:, 40] = dup[:, 41] = 2.0
    dup[:, 64] = 2.5
    cases.append(("dup_max", dup, zb, 2.5))
    cases.append(("random", rng.standard_normal((48, E_GLOBAL)).astype(np.float32), rb, 2.5))
    return cases


def make_routing(o) -> dict:
    out = {}
    names = []
    for i, (name, lg, b, f) in enumerate(routing_cases()):
        ids, w = o.route(lg, b, f)
        names.append(name)
        out[f"c{i}_logits"] = lg
        out[f"c{i}_bias_bits"] = b.view(torch.int16).numpy().view(np.uint16)
        out[f"c{i}_factor"] = np.float64(f)
        out[f"c{i}_ids"] = ids
        out[f"c{i}_w_bits"] = w.view(np.uint32)
    out["names"] = np.array(names)
    return out


def make_dispatch(o) -> dict:
    rng = np.random.default_rng(11)
    T = 150
    lg = rng.standard_normal((T, E_GLOBAL)).astype(np.float32)
    b = torch.zeros(E_GLOBAL)
    b[[70, 75, 230]] = 1.5  # crowd a few experts so some get more than one tile
    ids, w = o.route(lg, b.to(torch.bfloat16), 2.5)
    out = dict(ids=ids, w_bits=w.view(np.uint32))
    for off in (0, 64, 224):
        for tm in (16, 64):
            r = o.dispatch(ids, w, off, tm)
            key = f"o{off}_m{tm}"
            out[f"{key}_exp_off"] = r["exp_off"]
            out[f"{key}_sorted_tok"] = r["sorted_tok"]
            out[f"{key}_sorted_w_bits"] = r["sorted_w"].view(np.uint32)
            out[f"{key}_inv"] = r["inv"]
            out[f"{key}_tiles"] = r["tiles"]
    return out


def forward_activations(wl):
    """Crafted logits: every token's group 0 (local experts 0..31 at offset 0) holds only
    the strong experts listed per token; the last token has none."""
    rng = np.random.default_rng(FORWARD_SEED)
    T = 6
    lg = (rng.standard_normal((T, E_GLOBAL)) * 0.5).astype(np.float32)
    lg[:, :32] = -8.0
    strong = {0: (5, 9), 1: (5, 9), 2: (9, 20), 3: (5, 20), 4: (5, 9, 20), 5: ()}
    for t, es in strong.items():
        for j, e in enumerate(es):
            lg[t, e] = 3.0 - 0.25 * j
    g = torch.Generator().manual_seed(FORWARD_SEED)
    x = torch.randn(T, wl.H, generator=g).to(torch.bfloat16)
    hs, hs_scale = wl.quantize_rows_128(x)
    bias = torch.zeros(E_GLOBAL, dtype=torch.bfloat16)
    return lg, bias, hs, hs_scale


def forward_weights(wl):
    cfg = wl.Config("golden_forward", 6, 0, seed=FORWARD_SEED)
    return wl.make_weights(cfg, device="cpu", experts=FORWARD_EXPERTS)


def weight_checksum(wts: dict) -> np.ndarray:
    """Sum of the e4m3 bytes and of the scales of each generated expert."""
    sums = []
    for e in FORWARD_EXPERTS:
        sums.append(int(wts["gemm1_weights"][e].view(torch.uint8).to(torch.int64).sum()))
        sums.append(int(wts["gemm2_weights"][e].view(torch.uint8).to(torch.int64).sum()))
    return np.array(sums, dtype=np.int64)


def make_forward(o, wl) -> dict:
    lg, bias, hs, hs_scale = forward_activations(wl)
    wts = forward_weights(wl)
    ids, w = o.route(lg, bias, 2.5)
    acc = o.expert_forward(hs, hs_scale, wts["gemm1_weights"], wts["gemm1_weights_scale"],
                           wts["gemm2_weights"], wts["gemm2_weights_scale"], ids, w, 0)
    return dict(logits=lg, bias_bits=bias.view(torch.int16).numpy().view(np.uint16),
                factor=np.float64(2.5), local_expert_offset=np.int64(0),
                hidden_states=hs.view(torch.uint8).numpy(), hidden_states_scale=hs_scale.numpy(),
                seed=np.int64(FORWARD_SEED), experts=np.array(FORWARD_EXPERTS, np.int32),
                weight_checksum=weight_checksum(wts), ids=ids, w_bits=w.view(np.uint32),
                acc=acc.numpy())


def main() -> None:
    o = oracle()
    wl = pkg("workloads")
    np.savez_compressed(os.path.join(HERE, "routing.npz"), **make_routing(o))
    np.savez_compressed(os.path.join(HERE, "dispatch.npz"), **make_dispatch(o))
    np.savez_compressed(os.path.join(HERE, "forward.npz"), **make_forward(o, wl))
    for f in ("routing.npz", "dispatch.npz", "forward.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
