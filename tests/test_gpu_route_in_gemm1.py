"""GEMM1 with the routing and the dispatch folded in (GEMM1 variant 9, the plan for
T <= 8; from T = 5 in workgroups of 8 waves, one token per wave, then two groups of four
taking items): every
workgroup routes the call's tokens from the logits itself, then runs the
folded dispatch and its streaming items; the route launch goes away.  Its output must
be bit-identical to the pair it replaces (GEMM1 variant 5 after the route kernel, with
GEMM2 variant 6), its workspace must hold the same routing and dispatch, and, with no
route kernel to clear the C-range flag word on this path, GEMM2 checks a set word against
C's group exponents: whatever the workspace's flag words held before, the output is the
route-kernel pair's bit for bit."""
import numpy as np
import pytest
import torch

from conftest import oracle, pkg
from gpu_common import compare_to_oracle, config_inputs, first_tokens, note, run_forward

pytestmark = pytest.mark.gpu

C_FLAG = 35      # meta word of the C-range flag (kCWideFlag = 32 + 3)


def _bits(t):
    return t.view(torch.int16)


def _call(d, flags, ws):
    """Output of one forward call on workspace ws (NaN-filled output beforehand)."""
    k = pkg("kernel")
    wl = pkg("workloads")
    out = torch.full_like(d["output"], float("nan"))
    k.forward(*wl.as_args({**d, "output": out}), workspace=ws, flags=flags)
    torch.cuda.synchronize()
    return out


def _meta(ws, lay):
    return ws[lay.meta:lay.meta + 64 * 4].view(torch.int32)


@pytest.mark.parametrize("T,cfg,offset", [(1, 0, 0), (1, 3, 32), (2, 1, 0), (3, 3, 0), (3, 0, 96),
                                          (4, 0, 0), (4, 1, 224), (4, 3, 64), (5, 0, 0), (6, 3, 32),
                                          (7, 1, 0), (8, 0, 0), (8, 3, 224)])
def test_matches_the_route_kernel_pair_bit_for_bit(T, cfg, offset):
    k = pkg("kernel")
    d = first_tokens(config_inputs(cfg), T)
    d["local_expert_offset"] = offset
    assert k.workspace_layout(T).dispatch_in_gemm1 == 1
    note(f"[gpu] route in GEMM1 T={T} config={cfg} offset={offset}")
    folded = run_forward(d, flags=k.plan_flags(9, 6))
    assert torch.equal(_bits(folded), _bits(run_forward(d, flags=k.plan_flags(5, 6))))
    assert torch.equal(_bits(run_forward(d)), _bits(folded))       # the default plan
    st = compare_to_oracle(d, folded, list(range(T)))
    note(f"[gpu] T={T} offset={offset} stats {st}")
    assert st["frac_within"] == 1.0, st


@pytest.mark.parametrize("T,offset", [(3, 0), (4, 64), (7, 32), (8, 0)])
def test_workspace_routing_and_dispatch_are_bit_exact(T, offset):
    """The routing ids and weights the last workgroup writes, and the dispatch, equal
    the oracle's bit for bit (the separate route kernel's are pinned the same way)."""
    k = pkg("kernel")
    wl = pkg("workloads")
    d = first_tokens(config_inputs(3), T)
    d["local_expert_offset"] = offset
    flags = k.plan_flags(9, 6)
    lay = k.workspace_layout(T, flags)
    ws = torch.zeros(lay.total, dtype=torch.uint8, device="cuda")
    note(f"[gpu] route in GEMM1 workspace T={T} offset={offset}")
    _call(d, flags, ws)

    def arr(off, n, dt):
        return ws[off:off + n * 4].view(dt).cpu().numpy()

    o = oracle()
    rids, rw = o.route(d["routing_logits"], d["routing_bias"], d["routed_scaling_factor"])
    assert np.array_equal(arr(lay.topk_ids, T * 8, torch.int32).reshape(T, 8), rids)
    assert np.array_equal(arr(lay.topk_weights, T * 8, torch.float32).reshape(T, 8).view(np.uint32),
                          np.asarray(rw, np.float32).view(np.uint32))
    r = o.dispatch(rids, rw, offset, lay.tile_m)
    meta = arr(lay.meta, 34, torch.int32)
    assert np.array_equal(meta[:33], r["exp_off"])
    nt = r["tiles"].shape[0]
    assert meta[33] == nt
    assert np.array_equal(arr(lay.tiles, nt * 4, torch.int32).reshape(nt, 4), r["tiles"])
    na = int(r["exp_off"][-1])
    assert np.array_equal(arr(lay.sorted_tokens, na, torch.int32), r["sorted_tok"])
    assert np.array_equal(arr(lay.inverse_rows, T * 8, torch.int32).reshape(T, 8), r["inv"])


@pytest.mark.parametrize("T", [4, 8])
def test_c_beyond_fp16_takes_the_rare_path(T):
    """Hidden-state scales 2^10 times larger: C leaves the fp16 range, GEMM1 sets the
    C-range flag word, GEMM2 finds nonzero group exponents and takes its rare path, and
    the output is the route-kernel pair's bit for bit.  A normal call on the same
    workspace afterwards finds the word still set (nothing cleared it), finds every
    exponent 0, clears the word, and matches too.  T = 4 runs the 4-wave form, T = 8 the
    8-wave one."""
    k = pkg("kernel")
    d = dict(first_tokens(config_inputs(1), T))
    d["hidden_states_scale"] = d["hidden_states_scale"] * 1024.0
    flags = k.plan_flags(9, 6)
    lay = k.workspace_layout(T, flags)
    ws = torch.zeros(lay.total, dtype=torch.uint8, device="cuda")
    note(f"[gpu] route in GEMM1, C beyond fp16, T={T}")
    wide = _call(d, flags, ws)
    assert int(_meta(ws, lay)[C_FLAG]) == 1
    assert torch.equal(_bits(wide), _bits(run_forward(d, flags=k.plan_flags(5, 6))))
    d2 = first_tokens(config_inputs(1), T)
    normal = _call(d2, flags, ws)
    assert int(_meta(ws, lay)[C_FLAG]) == 0
    assert torch.equal(_bits(normal), _bits(run_forward(d2, flags=k.plan_flags(5, 6))))


@pytest.mark.parametrize("T", [4, 8])
def test_stale_flag_words_do_not_reach_the_output(T):
    """A workspace whose meta words past the offsets and tile counts hold nonzero garbage
    (as after other calls, other data or a graph replay): GEMM2 checks the set C-range
    word against the exponents, clears it, and the output is the route-kernel pair's bit
    for bit, on two calls in a row."""
    k = pkg("kernel")
    d = dict(first_tokens(config_inputs(1), T))
    flags = k.plan_flags(9, 6)
    lay = k.workspace_layout(T, flags)
    ws = torch.zeros(lay.total, dtype=torch.uint8, device="cuda")
    ref = run_forward(d, flags=k.plan_flags(5, 6))
    for rep in range(2):
        note(f"[gpu] route in GEMM1, stale flag words, T={T}, call {rep}")
        _meta(ws, lay)[35:].fill_(0x7fff0000 + 3 * rep + 1)
        torch.cuda.synchronize()
        out = _call(d, flags, ws)
        assert torch.equal(_bits(out), _bits(ref)), f"call {rep}"
        assert int(_meta(ws, lay)[C_FLAG]) == 0


@pytest.mark.parametrize("T", [4, 8])
def test_no_local_expert_gives_zeros(T):
    k = pkg("kernel")
    d = first_tokens(config_inputs(0), T)
    d["local_expert_offset"] = 256
    note(f"[gpu] route in GEMM1, no local expert, T={T}")
    out = run_forward(d, flags=k.plan_flags(9, 6))
    assert torch.equal(_bits(out), torch.zeros_like(_bits(out)))
