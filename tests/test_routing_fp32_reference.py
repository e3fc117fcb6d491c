"""The canonical routing against the reference's literal fp32 op sequence (CPU only).

The operator routes with a canonical sigmoid (binary64, one rounding to fp32) so that
host and device agree bit for bit.  The reference's routing is moe.cu:178-206: fp32
``at::sigmoid``, ``+ bias``, ``topk(2)`` per group, ``sum``, ``topk(4)`` of the group
scores, ``masked_fill(-inf)``, ``topk(8)``, and weights ``s * M / (sum(s * M) + 1e-20)
* factor``.  Two correct implementations of that sequence may only disagree where the
scores they compare are within rounding of each other.  This test runs the literal
sequence (torch's own fp32 sigmoid, topk and masked_fill) on every token of the five
benchmark configs and on the routing tie fixtures, and checks that each token where the
two disagree is such a near-tie:

* a different expert set: the canonical 4th and 5th group scores, or the 8th and 9th
  pruned expert scores, lie within kNearTieUlp ulp of each other;
* the same set in a different order: two adjacent selected scores lie within
  kNearTieUlp ulp;
* the same set: the weights agree to kWeightRtol (one fp32 sigmoid ulp plus the order
  of an 8-term sum).

The counts are printed (``pytest -s``) so they can be quoted; exact ties in the
fixtures are near-ties of gap 0.
"""
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN_DIR, oracle, pkg

kNearTieUlp = 2
kWeightRtol = 2e-6


def _ulps(a: float, b: float) -> float:
    """|a - b| in units of the fp32 spacing at the larger magnitude."""
    m = max(abs(a), abs(b))
    return abs(a - b) / float(np.spacing(np.float32(m))) if m > 0 else 0.0


def literal_fp32_route(logits: np.ndarray, bias_bf16: torch.Tensor, factor: float):
    """moe.cu:178-206 step by step in torch fp32 (its library calls, its order)."""
    lg = torch.from_numpy(np.ascontiguousarray(logits, dtype=np.float32))
    T = lg.shape[0]
    s = torch.sigmoid(lg)                                   # moe.cu:183
    sb = s + bias_bf16.float().reshape(-1)                  # moe.cu:184
    top2 = sb.view(T, 8, 32).topk(2, dim=2).values          # moe.cu:186-187
    gs = top2.sum(2)                                        # moe.cu:188
    gidx = gs.topk(4, dim=1).indices                        # moe.cu:190
    gmask = torch.zeros_like(gs).scatter_(1, gidx, 1.0)     # moe.cu:191-192
    smask = gmask.unsqueeze(2).expand(T, 8, 32).reshape(T, 256)
    pruned = sb.masked_fill(smask == 0, float("-inf"))      # moe.cu:198-199
    idx = pruned.topk(8, dim=1).indices                     # moe.cu:200
    M = torch.zeros_like(s).scatter_(1, idx, 1.0)           # moe.cu:202-203
    w = s * M
    wsum = w.sum(1, keepdim=True) + 1e-20                   # moe.cu:204-205
    w = (w / wsum) * float(factor)                          # moe.cu:206
    return idx.numpy().astype(np.int32), w.gather(1, idx).numpy()


def canonical_scores(logits: np.ndarray, bias_bf16: torch.Tensor):
    """s + bias with the canonical sigmoid, and the group scores (top-2 sums, fp32)."""
    lg = torch.from_numpy(np.ascontiguousarray(logits, dtype=np.float32))
    s = torch.sigmoid(lg.double()).float()
    sb = (s + bias_bf16.float().reshape(-1)).numpy()
    srt = -np.sort(-sb.reshape(-1, 8, 32), axis=2)
    gs = (srt[:, :, 0] + srt[:, :, 1]).astype(np.float32)
    return sb, gs


def compare(logits, bias_bf16, factor, literal_logits=None) -> dict:
    """Canonical route vs the literal fp32 sequence on the same inputs (or, to plant a
    disagreement, on literal_logits)."""
    o = oracle()
    ids_c, w_c = o.route(logits, bias_bf16, factor)
    ids_l, w_l = literal_fp32_route(logits if literal_logits is None else literal_logits,
                                    bias_bf16, factor)
    sb, gs = canonical_scores(logits, bias_bf16)
    T = ids_c.shape[0]
    set_diff, order_diff, far = [], [], []
    max_rel = 0.0
    for t in range(T):
        same_set = set(ids_c[t].tolist()) == set(ids_l[t].tolist())
        if not same_set:
            g = np.sort(gs[t])[::-1]
            kept = np.argsort(-gs[t], kind="stable")[:4]
            pr = np.concatenate([sb[t, 32 * k:32 * k + 32] for k in kept])
            v = np.sort(pr)[::-1]
            gap = min(_ulps(g[3], g[4]), _ulps(v[7], v[8]))
            set_diff.append((t, gap))
            if gap > kNearTieUlp:
                far.append((t, gap))
            continue
        if not np.array_equal(ids_c[t], ids_l[t]):
            sel = sb[t, ids_c[t]]
            gap = min(_ulps(sel[j], sel[j + 1]) for j in range(7))
            order_diff.append((t, gap))
            if gap > kNearTieUlp:
                far.append((t, gap))
        lw = dict(zip(ids_l[t].tolist(), w_l[t].tolist()))
        for j in range(8):
            ref = lw[int(ids_c[t, j])]
            max_rel = max(max_rel, abs(float(w_c[t, j]) - ref) / max(abs(ref), 1e-30))
    return dict(T=T, set_diff=len(set_diff), order_diff=len(order_diff), far=far,
                max_gap_ulp=max([g for _, g in set_diff + order_diff], default=0.0),
                weight_max_rel=max_rel)


def _report(name, r):
    print(f"[fp32-route] {name}: T={r['T']} set differs {r['set_diff']}, order differs "
          f"{r['order_diff']}, largest boundary gap {r['max_gap_ulp']:.1f} ulp, "
          f"weight max rel {r['weight_max_rel']:.2e}")


@pytest.mark.parametrize("ci", range(5))
def test_literal_fp32_route_differs_only_at_near_ties(ci):
    wl = pkg("workloads")
    cfg = wl.CONFIGS[ci]
    lg, bias = wl.make_routing_inputs(cfg)
    r = compare(lg.numpy(), bias, cfg.routed_scaling_factor)
    _report(cfg.name, r)
    assert not r["far"], f"disagreements away from a near-tie: {r['far'][:5]}"
    assert r["weight_max_rel"] <= kWeightRtol


def test_literal_fp32_route_on_tie_fixtures():
    g = np.load(os.path.join(GOLDEN_DIR, "routing.npz"))
    for i, name in enumerate(g["names"]):
        bias = torch.from_numpy(g[f"c{i}_bias_bits"].view(np.int16)).view(torch.bfloat16)
        r = compare(g[f"c{i}_logits"], bias, float(g[f"c{i}_factor"]))
        _report(str(name), r)
        assert not r["far"], f"{name}: disagreements away from a near-tie: {r['far'][:5]}"
        assert r["weight_max_rel"] <= kWeightRtol


def test_near_tie_check_catches_a_real_disagreement():
    """A planted difference far from any tie (the literal path fed logits in which the
    top expert of token 0 drops out of its top-8) must be reported: the check is not
    vacuous."""
    wl = pkg("workloads")
    lg, bias = wl.make_routing_inputs(wl.CONFIGS[1])
    lg = lg.numpy()
    ids_c, _ = oracle().route(lg, bias, 2.5)
    shifted = lg.copy()
    shifted[0, int(ids_c[0, 0])] -= 8.0
    r = compare(lg, bias, 2.5, literal_logits=shifted)
    assert r["set_diff"] == 1 and [t for t, _ in r["far"]] == [0]
