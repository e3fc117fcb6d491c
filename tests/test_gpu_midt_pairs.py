"""The GEMM pairs of mid-size T on a light and a heavy routing (T = 1024).

Between T = 200 and 1344 the default GEMM1 (variant 8, token-sharing, three workgroups
per CU) decides on the device, from the call's tile count, whether three or two
workgroups per CU work: two when the items (64-row tiles x 32) fall in (768, 1024], where
both take two rounds, three otherwise.  The light routing of config 2 (707 rows) lands
in that window, the heavy one (eight hot local experts, every token routed to them) far
above it, so both paths run.  Every pair that can run at this T -- the default, the
two-per-CU token-sharing GEMM1 (7/5), both token-sharing GEMM1s with the token-sharing
GEMM2 (8/7, 7/7), the prefill pair (4/5) and the 32-row streaming GEMM1 with the
conversion (2/5) -- must match the fp32 oracle on sampled tokens."""
import numpy as np
import pytest
import torch

from conftest import pkg
from gpu_common import compare_to_oracle, config_inputs, note

pytestmark = pytest.mark.gpu

PAIRS = [(8, 5), (7, 5), (8, 7), (7, 7), (4, 5), (2, 5)]


def _inputs(routing):
    wl = pkg("workloads")
    d = dict(config_inputs(2))                        # T = 1024, offset 64, its weights
    if routing == "heavy":
        cfg = wl.Config("heavy_t1024", 1024, 64, hot_local_experts=(0, 4, 8, 12, 16, 20, 24, 28),
                        seed=20264444)
        d.update(wl.make_activations(cfg, device="cuda"))
        d["output"] = torch.empty(1024, 7168, dtype=torch.bfloat16, device="cuda")
    return d


def _items(d, flags):
    """Work items of the token-sharing GEMM1 for this routing: 64-row tiles x 32."""
    k = pkg("kernel")
    wl = pkg("workloads")
    T = d["routing_logits"].shape[0]
    lay = k.workspace_layout(T, flags)
    ws = torch.empty(lay.total, dtype=torch.uint8, device="cuda")
    out = torch.empty_like(d["output"])
    k.forward(*wl.as_args({**d, "output": out}), workspace=ws, flags=flags)
    torch.cuda.synchronize()
    return 32 * int(ws[lay.meta + 33 * 4:lay.meta + 34 * 4].view(torch.int32).item()), out


@pytest.mark.parametrize("routing", ["light", "heavy"])
def test_every_pair_matches_oracle_at_t1024(routing):
    k = pkg("kernel")
    d = _inputs(routing)
    assert k.workspace_layout(1024).tile_m == 64          # the default is the token-sharing GEMM1
    items, default_out = _items(d, 0)
    note(f"[gpu] T=1024 {routing} routing: {items} token-sharing items")
    if routing == "light":
        assert 768 < items <= 1024                        # two workgroups per CU work
    else:
        assert items > 1024                               # all three per CU work
    toks = sorted(np.random.default_rng(1024).choice(1024, 24, replace=False).tolist())
    forced = {}
    for g1, g2 in PAIRS:
        _, out = _items(d, k.plan_flags(g1, g2))
        forced[(g1, g2)] = out
        st = compare_to_oracle(d, out, toks)
        note(f"[gpu] T=1024 {routing} pair {g1}/{g2}: {st}")
        assert st["frac_within"] == 1.0, (g1, g2, st)
    # the default plan is pair 8/5, whichever number of workgroups per CU it ran
    assert torch.equal(default_out.view(torch.int16), forced[(8, 5)].view(torch.int16))
    # variants 7 and 8 compute every item the same way: only the workgroup differs
    assert torch.equal(forced[(7, 5)].view(torch.int16), forced[(8, 5)].view(torch.int16))
    assert torch.equal(forced[(7, 7)].view(torch.int16), forced[(8, 7)].view(torch.int16))
