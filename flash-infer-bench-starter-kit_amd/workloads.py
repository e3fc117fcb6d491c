"""Seeded synthetic workloads of the five benchmark configurations.

Shapes and distributions (DeepSeek-V3 local-rank MoE, 32 of 256 experts):
  routing_logits  fp32 N(0,1)               [T, 256]
  routing_bias    bf16 N(0,0.1)             [256]   (+3.0 on 4 local experts for "skew")
  hidden_states   bf16 N(0,1) -> e4m3 with per-token per-128-column scale amax/448,
                  scales stored block-major [56, T]
  gemm1_weights   N(0,0.02) -> e4m3 per 128x128 block, scale amax/448  [32,4096,7168] + [32,32,56]
  gemm2_weights   same scheme                                           [32,7168,2048] + [32,56,16]
  routed_scaling_factor 2.5
Weights are regenerated from the seed on every use, never stored.  Each expert's
weights come from their own generator (seed, expert), so one expert can be rebuilt
alone.  Generation runs on whatever device is given (the GPU box generates there).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Iterable, Optional

import torch

H, I, E_GLOBAL, E_LOCAL, BLK = 7168, 2048, 256, 32, 128
FP8_MAX = 448.0


@dataclass(frozen=True)
class Config:
    name: str
    T: int
    local_expert_offset: int = 0
    hot_local_experts: tuple = field(default_factory=tuple)
    routed_scaling_factor: float = 2.5
    seed: int = 0


CONFIGS = [
    Config("decode_t8", 8, 0, seed=20260000),
    Config("decode_t64", 64, 0, seed=20260001),
    Config("prefill_t1024_off64", 1024, 64, seed=20260002),
    Config("prefill_t8192", 8192, 0, seed=20260003),
    Config("skew_t4096", 4096, 0, hot_local_experts=(3, 11, 19, 27), seed=20260004),
]


def _gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def quantize_rows_128(x: torch.Tensor):
    """[T, H] float -> (e4m3 [T, H], fp32 scales [H/128, T]) with per-(row, 128) amax/448."""
    T = x.shape[0]
    xf = x.float().view(T, H // BLK, BLK)
    amax = xf.abs().amax(dim=2)
    scale = torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))
    q = (xf / scale[:, :, None]).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q.view(T, H), scale.t().contiguous()


def quantize_blocks_128(w: torch.Tensor):
    """[R, C] float -> (e4m3 [R, C], fp32 [R/128, C/128]) with per 128x128 block amax/448."""
    R, C = w.shape
    b = w.float().view(R // BLK, BLK, C // BLK, BLK)
    amax = b.abs().amax(dim=(1, 3))
    scale = torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))
    q = (b / scale[:, None, :, None]).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q.view(R, C), scale


def _draw_routing(cfg: Config, g: torch.Generator, device, T: int):
    logits = torch.randn(T, E_GLOBAL, generator=g, device=device, dtype=torch.float32)
    bias = (torch.randn(E_GLOBAL, generator=g, device=device, dtype=torch.float32) * 0.1)
    for le in cfg.hot_local_experts:
        bias[cfg.local_expert_offset + le] += 3.0
    return logits, bias.to(torch.bfloat16)


def make_routing_inputs(cfg: Config, device="cpu", T: Optional[int] = None):
    """The config's (logits fp32 [T, 256], bias bf16 [256]) alone: the same values as
    make_activations, without drawing and quantising the hidden states."""
    T = cfg.T if T is None else T
    return _draw_routing(cfg, _gen(device, cfg.seed), device, T)


def make_activations(cfg: Config, device="cpu", T: Optional[int] = None) -> dict:
    """Logits, bias and quantised hidden states of a config (T may be overridden)."""
    T = cfg.T if T is None else T
    g = _gen(device, cfg.seed)
    logits, bias = _draw_routing(cfg, g, device, T)
    x = torch.randn(T, H, generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)
    hs, hs_scale = quantize_rows_128(x)
    return dict(routing_logits=logits, routing_bias=bias, hidden_states=hs,
                hidden_states_scale=hs_scale)


def make_weights(cfg: Config, device="cpu", experts: Optional[Iterable[int]] = None) -> dict:
    """Block-quantised expert weights.  ``experts`` limits which local experts get
    random values (the others are zero bytes with scale 1) -- enough for a check
    that only touches those experts and much cheaper on a CPU."""
    todo = set(range(E_LOCAL) if experts is None else experts)
    w1 = torch.zeros(E_LOCAL, 2 * I, H, dtype=torch.float8_e4m3fn, device=device)
    s1 = torch.ones(E_LOCAL, 2 * I // BLK, H // BLK, dtype=torch.float32, device=device)
    w2 = torch.zeros(E_LOCAL, H, I, dtype=torch.float8_e4m3fn, device=device)
    s2 = torch.ones(E_LOCAL, H // BLK, I // BLK, dtype=torch.float32, device=device)
    for e in sorted(todo):
        g = _gen(device, cfg.seed * 1000 + 17 + e)
        a = torch.randn(2 * I, H, generator=g, device=device, dtype=torch.float32) * 0.02
        w1[e], s1[e] = quantize_blocks_128(a)
        del a
        b = torch.randn(H, I, generator=g, device=device, dtype=torch.float32) * 0.02
        w2[e], s2[e] = quantize_blocks_128(b)
        del b
    return dict(gemm1_weights=w1, gemm1_weights_scale=s1, gemm2_weights=w2,
                gemm2_weights_scale=s2)


def make_inputs(cfg: Config, device="cpu", T: Optional[int] = None,
                experts: Optional[Iterable[int]] = None) -> dict:
    """All kernel arguments of a config, output included (zeros)."""
    d = make_activations(cfg, device, T)
    d.update(make_weights(cfg, device, experts))
    T = d["routing_logits"].shape[0]
    d["local_expert_offset"] = cfg.local_expert_offset
    d["routed_scaling_factor"] = cfg.routed_scaling_factor
    d["output"] = torch.zeros(T, H, dtype=torch.bfloat16, device=device)
    return d


ARG_ORDER = ("routing_logits", "routing_bias", "hidden_states", "hidden_states_scale",
             "gemm1_weights", "gemm1_weights_scale", "gemm2_weights", "gemm2_weights_scale",
             "local_expert_offset", "routed_scaling_factor", "output")


def as_args(d: dict) -> list:
    return [d[k] for k in ARG_ORDER]


def algorithmic_work(ids, offset: int, T: int) -> dict:
    """N_a, E_a, FLOPs and HBM bytes of one call from the actual routing ids."""
    ids = torch.as_tensor(ids).to(torch.int64)
    le = ids - offset
    local = (le >= 0) & (le < E_LOCAL)
    n_a = int(local.sum())
    e_a = int(torch.unique(le[local]).numel())
    flops = n_a * (2 * H * 2 * I + 2 * I * H)
    w_bytes = e_a * (2 * I * H + (2 * I // BLK) * (H // BLK) * 4 + H * I + (H // BLK) * (I // BLK) * 4)
    act_bytes = T * (E_GLOBAL * 4 + H + (H // BLK) * 4 + H * 2) + E_GLOBAL * 2
    return dict(N_a=n_a, E_a=e_a, flops=flops, bytes=w_bytes + act_bytes,
                gemm1_bytes=e_a * (2 * I * H + (2 * I // BLK) * (H // BLK) * 4) + T * (H + (H // BLK) * 4) + n_a * I * 2,
                gemm2_bytes=e_a * (H * I + (H // BLK) * (I // BLK) * 4) + n_a * I * 2 + n_a * H * 4)
