"""The forward without a workspace argument (moe_mi355_forward_noalloc): it runs on the
library's own per-GPU scratch array and allocates nothing.  Its results must be
bit-identical to moe_mi355_forward's on the same inputs, also on a second call with a
smaller T (the array keeps the previous call's contents, which must not leak into
the next call), and it must reject token counts beyond its maximum."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import pkg

MAX_T = 256          # MOE_MI355_NOALLOC_MAX_TOKENS


def _args(k, d, out):
    return k.MoeArgs(
        routing_logits=d["routing_logits"].data_ptr(),
        routing_bias=d["routing_bias"].data_ptr(),
        hidden_states=d["hidden_states"].data_ptr(),
        hidden_states_scale=d["hidden_states_scale"].data_ptr(),
        gemm1_weights=d["gemm1_weights"].data_ptr(),
        gemm1_weights_scale=d["gemm1_weights_scale"].data_ptr(),
        gemm2_weights=d["gemm2_weights"].data_ptr(),
        gemm2_weights_scale=d["gemm2_weights_scale"].data_ptr(),
        local_expert_offset=int(d["local_expert_offset"]),
        routed_scaling_factor=float(d["routed_scaling_factor"]),
        output=out.data_ptr(), T=int(d["routing_logits"].shape[0]), flags=0,
        workspace=None, workspace_bytes=0)


def test_noalloc_rejects_sizes_beyond_its_maximum():
    """Checked before any device work, so this runs without a GPU."""
    k = pkg("kernel")
    L = k._build_extension()
    a = k.MoeArgs()
    a.T = MAX_T + 1
    rc = L.moe_mi355_forward_noalloc(ctypes.byref(a), None)
    assert rc == -9
    assert "MOE_MI355_NOALLOC_MAX_TOKENS" in L.moe_mi355_strerror(rc).decode()
    a.T = 1 << 20
    assert L.moe_mi355_forward_noalloc(ctypes.byref(a), None) == -9
    a.T = -1
    assert L.moe_mi355_forward_noalloc(ctypes.byref(a), None) == -2
    a.T = 0
    assert L.moe_mi355_forward_noalloc(ctypes.byref(a), None) == 0
    assert L.moe_mi355_forward_noalloc(None, None) == -1
    # the array holds the workspace of the largest call it accepts
    assert L.moe_mi355_noalloc_scratch_bytes() >= k.workspace_bytes(MAX_T)
    assert L.moe_mi355_noalloc_scratch_bytes() <= 64 << 20


@pytest.mark.gpu
def test_noalloc_matches_forward_on_consecutive_calls():
    """T = 256 (the maximum), then smaller calls on the same array (37 tokens with
    another expert offset, then 5, then 3, where GEMM1 routes the tokens itself and no
    kernel clears the C-range flag word): each output is bit-identical to
    moe_mi355_forward's with a fresh workspace, and the call allocates no memory
    through torch."""
    from gpu_common import config_inputs, first_tokens, note
    k = pkg("kernel")
    wl = pkg("workloads")
    L = k._build_extension()
    dev = torch.device("cuda:0")
    full = config_inputs(3)
    for T, offset in ((MAX_T, 0), (37, 64), (5, 0), (3, 32)):
        d = first_tokens(full, T)
        d["local_expert_offset"] = offset
        note(f"[gpu] noalloc T={T} offset={offset}")
        ref = torch.full_like(d["output"], float("nan"))
        k.forward(*wl.as_args({**d, "output": ref}))
        out = torch.full_like(d["output"], float("nan"))
        a = _args(k, d, out)
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated(dev)
        with torch.cuda.device(dev):
            rc = L.moe_mi355_forward_noalloc(
                ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
        assert rc == 0, L.moe_mi355_strerror(rc).decode()
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated(dev) == before
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"T={T}"
        assert bool(torch.isfinite(out.float()).all())
        note(f"[gpu] noalloc T={T} bit-identical, max |out| {float(out.float().abs().max()):.3g}")


@pytest.mark.gpu
@pytest.mark.parametrize("T", [3, 8, MAX_T])
def test_noalloc_under_graph_capture(T):
    """After one eager call on the device (which looks up the array's address and the
    launch grid), noalloc calls can be captured into a HIP graph: each replay, run
    after eager forward calls on the same output and a device synchronisation, is
    bit-identical to moe_mi355_forward with a fresh workspace; and a warm eager call
    leaves the device's free memory (hipMemGetInfo) unchanged."""
    from gpu_common import config_inputs, first_tokens, note
    k = pkg("kernel")
    wl = pkg("workloads")
    L = k._build_extension()
    dev = torch.device("cuda:0")
    d = first_tokens(config_inputs(1 if T <= 64 else 3), T)
    ref = torch.full_like(d["output"], float("nan"))
    k.forward(*wl.as_args({**d, "output": ref}))
    out = torch.full_like(d["output"], float("nan"))
    a = _args(k, d, out)
    side = torch.cuda.Stream(dev)

    def call(stream):
        return L.moe_mi355_forward_noalloc(ctypes.byref(a), ctypes.c_void_p(stream.cuda_stream))

    note(f"[gpu] noalloc graph capture T={T}")
    side.wait_stream(torch.cuda.current_stream(dev))
    assert call(side) == 0                 # the warm call, on the capture stream
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info(dev)[0]
    assert call(side) == 0
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info(dev)[0] == free0
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        rc = call(side)
    assert rc == 0, L.moe_mi355_strerror(rc).decode()
    torch.cuda.synchronize()
    for rep in range(3):
        out.fill_(float("nan"))
        other = torch.full_like(out, float("nan"))
        k.forward(*wl.as_args({**d, "output": other}))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"replay {rep}"
    note(f"[gpu] noalloc graph T={T}: 3 replays bit-identical")
