"""HIP graph capture of the forward pass (runs on the MI355X box).

The forward issues only kernel launches on the caller's stream (no allocation, no
memset, no host synchronisation), so a caller can capture one call into a graph and
replay it, the way decode loops remove per-call launch cost.  Each replay here runs
after eager work on the same buffers and a device synchronisation, and must match
the eager result bit for bit; one replay runs on inputs rewritten in place after
capture, to show the graph recomputes rather than replaying stale results.
"""
import pytest
import torch

from conftest import pkg
from gpu_common import config_inputs, first_tokens, note

pytestmark = pytest.mark.gpu


def _eager(k, wl, d, ws):
    out = torch.full_like(d["output"], float("nan"))
    k.forward(*wl.as_args({**d, "output": out}), workspace=ws)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("idx", [0, 1, 2, 3, 4])
def test_graph_replay_matches_eager(idx):
    k = pkg("kernel")
    wl = pkg("workloads")
    d0 = config_inputs(idx)
    T = d0["routing_logits"].shape[0]
    note(f"[gpu] graph capture config {idx} T={T}")
    # private copies of the inputs the test rewrites
    d = {key: (v.clone() if isinstance(v, torch.Tensor) else v) for key, v in d0.items()}
    ws = torch.empty(k.workspace_bytes(T), dtype=torch.uint8, device="cuda")
    ref = _eager(k, wl, d, ws)

    out = torch.full_like(d["output"], float("nan"))
    args = wl.as_args({**d, "output": out})
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):          # warm-up on the capture stream
        k.forward(*args, workspace=ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        k.forward(*args, workspace=ws)
    torch.cuda.synchronize()

    for rep in range(3):
        # eager work on the same output and workspace between replays
        out.fill_(float("nan"))
        _eager(k, wl, d, ws)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"replay {rep}"

    # new routing logits and hidden rows written into the captured buffers
    gen = torch.Generator(device="cuda").manual_seed(1000 + idx)
    d["routing_logits"].copy_(torch.randn(d["routing_logits"].shape, generator=gen, device="cuda"))
    d["hidden_states"].view(torch.uint8).copy_(torch.roll(d0["hidden_states"].view(torch.uint8), 1, dims=0))
    d["hidden_states_scale"].copy_(torch.roll(d0["hidden_states_scale"], 1, dims=1))
    ref2 = _eager(k, wl, d, ws)
    out.fill_(float("nan"))
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref2.view(torch.int16))
    assert not torch.equal(ref2.view(torch.int16), ref.view(torch.int16))
    note(f"[gpu] graph config {idx}: 4 replays bit-identical to eager")


@pytest.mark.parametrize("T", [4, 8, 16])
def test_graph_replay_after_c_beyond_fp16(T):
    """A captured call whose inputs first send C beyond the fp16 range (hidden-state
    scales 2^10 times larger), then, rewritten in place, keep it inside: each replay
    matches the eager call on the same inputs bit for bit.  At T <= 8 no route kernel
    clears the C-range flag word, so the second replay finds the word the first one set
    and must still take the usual path; T = 16 runs the route kernel's plan."""
    k = pkg("kernel")
    wl = pkg("workloads")
    d = first_tokens(config_inputs(1), T)
    d["hidden_states_scale"] = d["hidden_states_scale"].clone()     # rewritten in place below
    normal_scale = d["hidden_states_scale"].clone()
    d["hidden_states_scale"].mul_(1024.0)
    ws = torch.empty(k.workspace_bytes(T), dtype=torch.uint8, device="cuda")
    note(f"[gpu] graph capture with C beyond fp16, T={T}")
    ref_wide = _eager(k, wl, d, ws)
    out = torch.full_like(d["output"], float("nan"))
    args = wl.as_args({**d, "output": out})
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        k.forward(*args, workspace=ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        k.forward(*args, workspace=ws)
    torch.cuda.synchronize()
    for rep in range(2):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref_wide.view(torch.int16)), f"wide replay {rep}"
    d["hidden_states_scale"].copy_(normal_scale)
    torch.cuda.synchronize()
    for rep in range(2):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        ref = _eager(k, wl, d, torch.empty_like(ws))
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"normal replay {rep}"
    assert not torch.equal(ref.view(torch.int16), ref_wide.view(torch.int16))
    note(f"[gpu] graph T={T}: wide then normal replays bit-identical to eager")
