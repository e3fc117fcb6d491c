"""GEMM2 with the combine folded in (GEMM2 variant 6, for T <= 32; the default plan up to
T = 22): a workgroup
owns 32 output columns of every row tile, keeps the call's expert rows for them in LDS
and writes the bf16 output itself.  Its output must be bit-identical to the streaming
GEMM2 followed by the combine launch (variant 1), with the dispatch folded into GEMM1
or not, on the normal path, on the path where the expert rows go beyond the fp16 range
(C still inside it), and on the rare path where C itself does; and within the
oracle's tolerance."""
import numpy as np
import pytest
import torch

from conftest import pkg
from gpu_common import compare_to_oracle, config_inputs, first_tokens, note, run_forward

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.view(torch.int16)


def _flags_after(d, flags, ws=None):
    """Output and the two per-call flag words (C, expert rows beyond fp16) of one call
    (on `ws`, or a fresh workspace)."""
    k = pkg("kernel")
    wl = pkg("workloads")
    T = d["routing_logits"].shape[0]
    lay = k.workspace_layout(T, flags)
    if ws is None:
        ws = torch.empty(lay.total, dtype=torch.uint8, device="cuda")
    out = torch.full_like(d["output"], float("nan"))
    k.forward(*wl.as_args({**d, "output": out}), workspace=ws, flags=flags)
    torch.cuda.synchronize()
    return out, ws[lay.meta + 35 * 4:lay.meta + 37 * 4].view(torch.int32).cpu().tolist()


@pytest.mark.parametrize("T,offset", [(1, 0), (3, 0), (8, 0), (8, 96), (16, 0), (24, 224),
                                      (32, 0), (32, 64)])
def test_matches_separate_combine_bit_for_bit(T, offset):
    k = pkg("kernel")
    d = first_tokens(config_inputs(3), T)
    d["local_expert_offset"] = offset
    lay = k.workspace_layout(T, k.plan_flags(5, 6))
    assert lay.combine_in_gemm2 == 1 and lay.dispatch_in_gemm1 == 1
    assert k.workspace_layout(T).combine_in_gemm2 == (1 if T <= 22 else 0)
    note(f"[gpu] combine in GEMM2 T={T} offset={offset}")
    fused = run_forward(d, flags=k.plan_flags(5, 6))
    separate = run_forward(d, flags=k.plan_flags(5, 1))
    assert torch.equal(_bits(fused), _bits(separate))
    assert torch.equal(_bits(run_forward(d, flags=k.plan_flags(1, 6))), _bits(separate))
    assert torch.equal(_bits(run_forward(d)), _bits(separate))      # the default plan
    toks = sorted(np.random.default_rng(T + offset).choice(T, min(T, 16), replace=False).tolist())
    st = compare_to_oracle(d, fused, toks)
    note(f"[gpu] T={T} offset={offset} stats {st}")
    assert st["frac_within"] == 1.0, st


def test_no_local_expert_gives_zeros():
    """An offset past the expert range: no tile at all, every output exactly +0."""
    k = pkg("kernel")
    d = first_tokens(config_inputs(0), 8)
    d["local_expert_offset"] = 256
    note("[gpu] combine in GEMM2, no local expert")
    out = run_forward(d, flags=k.plan_flags(5, 6))
    assert torch.equal(_bits(out), torch.zeros_like(_bits(out)))


def test_all_local_routing_fills_the_rows():
    """T = 32 with every token routed to 8 local experts: 256 rows, the most the
    kernel's LDS holds; 8 rows per expert, 32 tiles, 8 rounds of the K-partial reduction."""
    k = pkg("kernel")
    wl = pkg("workloads")
    T = 32
    cfg = wl.Config("all_local", T, 0, hot_local_experts=tuple(range(32)), seed=20263344)
    d = dict(config_inputs(4))
    d.update(wl.make_activations(cfg, device="cuda"))
    d["output"] = torch.empty(T, 7168, dtype=torch.bfloat16, device="cuda")
    note("[gpu] combine in GEMM2, all-local routing T=32")
    ids, _ = k.route(d["routing_logits"], d["routing_bias"], 2.5)
    assert bool(((ids >= 0) & (ids < 32)).all())
    fused = run_forward(d, flags=k.plan_flags(5, 6))
    assert torch.equal(_bits(fused), _bits(run_forward(d, flags=k.plan_flags(5, 1))))
    st = compare_to_oracle(d, fused, list(range(T)))
    note(f"[gpu] all-local stats {st}")
    assert st["frac_within"] == 1.0, st


def test_expert_rows_beyond_fp16_range():
    """W2 block scales 2^16 times larger: C stays inside the fp16 range, the expert rows
    leave it, so the kernel applies the 16-column group exponents of the fp16 row form
    (and raises the expert-row flag) exactly as the separate GEMM2 and combine do."""
    k = pkg("kernel")
    d = dict(first_tokens(config_inputs(1), 16))
    d["gemm2_weights_scale"] = d["gemm2_weights_scale"] * 65536.0
    note("[gpu] combine in GEMM2, expert rows beyond fp16, T=16")
    fused, fl6 = _flags_after(d, k.plan_flags(5, 6))
    separate, fl1 = _flags_after(d, k.plan_flags(5, 1))
    assert fl6 == [0, 1] and fl1 == [0, 1]
    assert float(separate.float().abs().max()) > 65504.0
    assert torch.equal(_bits(fused), _bits(separate))


def test_c_beyond_fp16_range_takes_the_rare_path():
    """Hidden-state scales 2^10 times larger: C itself leaves the fp16 range and GEMM2
    runs its bf16 path; the fused kernel's rare path matches the separate one."""
    k = pkg("kernel")
    d = dict(first_tokens(config_inputs(1), 8))
    d["hidden_states_scale"] = d["hidden_states_scale"] * 1024.0
    note("[gpu] combine in GEMM2, C beyond fp16, T=8")
    ws = torch.empty(k.workspace_bytes(8), dtype=torch.uint8, device="cuda")
    fused, fl6 = _flags_after(d, k.plan_flags(5, 6), ws)
    separate, fl1 = _flags_after(d, k.plan_flags(5, 1))
    assert fl6 == [1, 1] and fl1 == [1, 1]
    assert torch.equal(_bits(fused), _bits(separate))
    # a normal call on the same workspace afterwards finds both flags cleared
    d2 = first_tokens(config_inputs(1), 8)
    out, fl = _flags_after(d2, k.plan_flags(5, 6), ws)
    assert fl == [0, 0]
    assert torch.equal(_bits(out), _bits(run_forward(d2, flags=k.plan_flags(5, 1))))
