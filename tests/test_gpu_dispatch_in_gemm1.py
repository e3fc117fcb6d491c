"""GEMM1 with the dispatch folded in (GEMM1 variant 5, the plan for T <= 64): every
workgroup of a persistent grid computes the call's dispatch from the routing ids, and
workgroup 0 leaves it in the workspace for GEMM2 and the combine.  The output must be
bit-identical to the plan with the separate dispatch launch (variant 1), the dispatch in
the workspace identical to the dispatch kernel's, and both within the oracle's
tolerance."""
import numpy as np
import pytest
import torch

from conftest import pkg
from gpu_common import compare_to_oracle, config_inputs, first_tokens, note, run_forward

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.view(torch.int16)


@pytest.mark.parametrize("T,offset,g2", [(1, 0, 1), (5, 0, 1), (8, 0, 1), (13, 96, 1), (37, 224, 1),
                                         (64, 0, 1), (64, 32, 1)])
def test_matches_separate_dispatch_bit_for_bit(T, offset, g2):
    k = pkg("kernel")
    d = first_tokens(config_inputs(3), T)
    d["local_expert_offset"] = offset
    assert k.workspace_layout(T).dispatch_in_gemm1 == 1
    note(f"[gpu] dispatch in GEMM1 T={T} offset={offset} g2={g2}")
    folded = run_forward(d, flags=k.plan_flags(5, g2))
    separate = run_forward(d, flags=k.plan_flags(1, g2))
    assert torch.equal(_bits(folded), _bits(separate))
    if g2 == 1:
        assert torch.equal(_bits(folded), _bits(run_forward(d)))   # the default plan
    toks = sorted(np.random.default_rng(T + offset).choice(T, min(T, 16), replace=False).tolist())
    st = compare_to_oracle(d, folded, toks)
    note(f"[gpu] T={T} offset={offset} stats {st}")
    assert st["frac_within"] == 1.0, st


def test_decode_configs_match_oracle():
    """configs[0] (T=8) and configs[1] (T=64), every token."""
    for idx in (0, 1):
        d = dict(config_inputs(idx))
        T = d["routing_logits"].shape[0]
        note(f"[gpu] dispatch in GEMM1, config {idx}")
        st = compare_to_oracle(d, run_forward(d), list(range(T)))
        note(f"[gpu] config {idx} stats {st}")
        assert st["frac_within"] == 1.0, st


def test_all_local_routing():
    """Every token routed to 8 local experts: 512 rows, 64 tiles of 16 rows (the most the
    kernel's LDS tile list holds)."""
    k = pkg("kernel")
    wl = pkg("workloads")
    T = 64
    cfg = wl.Config("all_local", T, 0, hot_local_experts=tuple(range(32)), seed=20263333)
    d = dict(config_inputs(4))
    d.update(wl.make_activations(cfg, device="cuda"))
    d["output"] = torch.empty(T, 7168, dtype=torch.bfloat16, device="cuda")
    note("[gpu] dispatch in GEMM1, all-local routing")
    folded = run_forward(d)
    assert torch.equal(_bits(folded), _bits(run_forward(d, flags=k.plan_flags(1, 1))))
    st = compare_to_oracle(d, folded, list(range(0, T, 4)))
    assert st["frac_within"] == 1.0, st


def test_no_local_expert_gives_zeros():
    d = first_tokens(config_inputs(0), 8)
    d["local_expert_offset"] = 1000
    note("[gpu] dispatch in GEMM1, no local expert")
    assert bool((_bits(run_forward(d)) == 0).all())


def test_dispatch_in_workspace_matches_dispatch_kernel():
    """Workgroup 0 leaves the dispatch where the dispatch kernel puts it: offsets, tile
    list, permutation, row weights, inverse map."""
    k = pkg("kernel")
    wl = pkg("workloads")
    T = 64
    d = dict(config_inputs(1))
    lay = k.workspace_layout(T)
    ws = torch.empty(lay.total, dtype=torch.uint8, device="cuda")
    out = torch.empty_like(d["output"])
    note("[gpu] dispatch in GEMM1, workspace tables")
    k.forward(*wl.as_args({**d, "output": out}), workspace=ws)
    ids, w = k.route(d["routing_logits"], d["routing_bias"], d["routed_scaling_factor"])
    ref = k.dispatch(ids, w, d["local_expert_offset"], 16)
    torch.cuda.synchronize()

    def arr(off, n):
        return ws[off:off + n * 4].view(torch.int32)

    exp_off = arr(lay.meta, 33)
    assert torch.equal(exp_off, ref["exp_off"])
    na = int(exp_off[32].item())
    nt = int(arr(lay.meta + 33 * 4, 1).item())
    assert nt == int(ref["num_tiles"].item())
    assert torch.equal(arr(lay.tiles, 4 * nt).view(nt, 4), ref["tiles"][:nt])
    assert torch.equal(arr(lay.sorted_tokens, na), ref["sorted_tok"][:na])
    assert torch.equal(arr(lay.sorted_weights, na), ref["sorted_w"][:na].view(torch.int32))
    assert torch.equal(arr(lay.inverse_rows, 8 * T).view(T, 8), ref["inv"])


def test_calls_of_different_sizes_on_one_workspace():
    k = pkg("kernel")
    wl = pkg("workloads")
    full = config_inputs(3)
    ws = torch.empty(k.workspace_bytes(64), dtype=torch.uint8, device="cuda")
    for T in (64, 8, 64, 1, 37, 37):
        d = first_tokens(full, T)
        note(f"[gpu] dispatch in GEMM1, shared workspace T={T}")
        out = torch.full_like(d["output"], float("nan"))
        k.forward(*wl.as_args({**d, "output": out}), workspace=ws)
        ref = run_forward(d, flags=k.plan_flags(1, 1))
        assert torch.equal(_bits(out), _bits(ref)), T
