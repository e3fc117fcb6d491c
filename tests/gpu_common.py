"""Shared helpers of the GPU tests: seeded inputs generated on the device (cached per
config for the session) and the output tolerance check."""
import functools
import sys

import numpy as np
import torch

from conftest import oracle, pkg

# Output tolerance against the fp32 CPU oracle (bf16 output): |gpu - ref| <= ATOL + RTOL |ref|
ATOL = 1e-2
RTOL = 1e-2


def note(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@functools.lru_cache(maxsize=None)
def config_inputs(idx: int) -> dict:
    wl = pkg("workloads")
    cfg = wl.CONFIGS[idx]
    note(f"[gpu] generating inputs for config {idx} ({cfg.name}, T={cfg.T})")
    d = wl.make_inputs(cfg, device="cuda")
    torch.cuda.synchronize()
    return d


def first_tokens(d0: dict, T: int) -> dict:
    """The first T tokens of a config's inputs (same weights)."""
    d = dict(d0)
    d["routing_logits"] = d0["routing_logits"][:T].contiguous()
    d["hidden_states"] = d0["hidden_states"][:T].contiguous()
    d["hidden_states_scale"] = d0["hidden_states_scale"][:, :T].contiguous()
    d["output"] = torch.empty(T, d0["output"].shape[1], dtype=torch.bfloat16, device="cuda")
    return d


def run_forward(d: dict, flags: int = 0, **kw) -> torch.Tensor:
    """One forward call on a NaN-filled output: through the DPS entry `kernel`, or
    through `forward` when call flags are given."""
    k = pkg("kernel")
    wl = pkg("workloads")
    out = torch.full_like(d["output"], float("nan"))
    args = wl.as_args({**d, "output": out, **kw})
    if flags:
        k.forward(*args, flags=flags)
    else:
        k.kernel(*args)
    torch.cuda.synchronize()
    return out


def compare_to_oracle(d: dict, out: torch.Tensor, tokens) -> dict:
    """fp32 oracle on `tokens` vs the GPU bf16 output rows; returns error stats."""
    o = oracle()
    ids, w = o.route(d["routing_logits"], d["routing_bias"], d["routed_scaling_factor"])
    acc = o.expert_forward(d["hidden_states"], d["hidden_states_scale"], d["gemm1_weights"],
                           d["gemm1_weights_scale"], d["gemm2_weights"], d["gemm2_weights_scale"],
                           ids, w, d["local_expert_offset"], tokens=tokens)
    got = out[torch.as_tensor(tokens, device=out.device)].float().cpu()
    err = (got - acc).abs()
    bound = ATOL + RTOL * acc.abs()
    stats = dict(max_abs=float(err.max()), p99_abs=float(torch.quantile(err.flatten()[:1_000_000], 0.99)),
                 mean_abs=float(err.mean()), frac_within=float((err <= bound).float().mean()),
                 max_ref=float(acc.abs().max()), n=int(err.numel()))
    return stats
