"""Size-independent exact properties of the HIP path at the full benchmark sizes
(runs on the MI355X box).  None of these needs the oracle:

* determinism: two calls give bit-identical outputs (no order-dependent atomics);
* linearity in routed_scaling_factor: doubling it doubles every output exactly
  (power-of-two scaling commutes with every rounding on the path);
* token permutation: permuting the tokens permutes the output rows exactly;
* tokens with no local expert get exactly +0, and an offset with no local experts
  zeroes the whole (pre-poisoned) output;
* T = 0 is a no-op; T = 1 and odd T work.
"""
import numpy as np
import pytest
import torch

from conftest import oracle, pkg
from gpu_common import compare_to_oracle, config_inputs, first_tokens, note, run_forward

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("idx", [1, 3, 4])
def test_deterministic(idx):
    d = config_inputs(idx)
    note(f"[gpu] determinism config {idx}")
    a = run_forward(d)
    b = run_forward(d)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("idx", [1, 2])
def test_factor_doubling_is_exact(idx):
    d = config_inputs(idx)
    note(f"[gpu] factor doubling config {idx}")
    a = run_forward(d)
    b = run_forward(d, routed_scaling_factor=2 * d["routed_scaling_factor"])
    assert torch.equal((a.float() * 2).to(torch.bfloat16).view(torch.int16), b.view(torch.int16))


def test_token_permutation():
    d = config_inputs(2)
    note("[gpu] token permutation config 2")
    T = d["routing_logits"].shape[0]
    perm = torch.randperm(T, generator=torch.Generator().manual_seed(3)).cuda()
    p = dict(d)
    p["routing_logits"] = d["routing_logits"][perm].contiguous()
    p["hidden_states"] = d["hidden_states"][perm].contiguous()
    p["hidden_states_scale"] = d["hidden_states_scale"][:, perm].contiguous()
    a = run_forward(d)
    b = run_forward(p)
    assert torch.equal(a[perm].view(torch.int16), b.view(torch.int16))


def test_nonlocal_tokens_are_zero():
    d = config_inputs(1)
    out = run_forward(d)
    ids, _ = oracle().route(d["routing_logits"], d["routing_bias"], d["routed_scaling_factor"])
    off = d["local_expert_offset"]
    nonlocal_t = [t for t in range(ids.shape[0]) if not ((ids[t] >= off) & (ids[t] < off + 32)).any()]
    for t in nonlocal_t:
        assert (out[t].view(torch.int16) == 0).all()


@pytest.mark.parametrize("offset", [1000, -100])
def test_offset_without_local_experts_zeroes_output(offset):
    d = config_inputs(0)
    out = run_forward(d, local_expert_offset=offset)
    assert (out.view(torch.int16) == 0).all()


def test_partially_local_offset_matches_oracle():
    """offset 240: local experts 240..271, only 240..255 exist (moe.cu:213-214)."""
    d = dict(config_inputs(1))
    d["local_expert_offset"] = 240
    out = run_forward(d)
    st = compare_to_oracle(d, out, list(range(d["routing_logits"].shape[0])))
    note(f"[gpu] offset 240 stats {st}")
    assert st["frac_within"] == 1.0, st


def test_empty_batch_is_noop():
    k = pkg("kernel")
    wl = pkg("workloads")
    d = dict(config_inputs(0))
    d["routing_logits"] = d["routing_logits"][:0]
    d["hidden_states"] = d["hidden_states"][:0]
    d["hidden_states_scale"] = d["hidden_states_scale"][:, :0].contiguous()
    d["output"] = d["output"][:0]
    k.kernel(*wl.as_args(d))
    torch.cuda.synchronize()


@pytest.mark.parametrize("T", [1, 5, 67])
def test_small_odd_batches(T):
    d0 = config_inputs(1)
    d = dict(d0)
    d["routing_logits"] = d0["routing_logits"][:T].contiguous() if T <= 64 else torch.cat(
        [d0["routing_logits"], d0["routing_logits"][:T - 64]]).contiguous()
    d["hidden_states"] = d0["hidden_states"][:T].contiguous() if T <= 64 else torch.cat(
        [d0["hidden_states"].view(torch.uint8), d0["hidden_states"][:T - 64].view(torch.uint8)]).view(torch.float8_e4m3fn)
    d["hidden_states_scale"] = d0["hidden_states_scale"][:, :T].contiguous() if T <= 64 else torch.cat(
        [d0["hidden_states_scale"], d0["hidden_states_scale"][:, :T - 64]], dim=1).contiguous()
    d["output"] = torch.empty(T, 7168, dtype=torch.bfloat16, device="cuda")
    out = run_forward(d)
    st = compare_to_oracle(d, out, list(range(T)))
    note(f"[gpu] T={T} stats {st}")
    assert st["frac_within"] == 1.0, st


@pytest.mark.parametrize("T", [88, 89, 199, 200, 559, 560, 640, 641, 960, 961, 1344, 1345])
def test_plan_boundaries_match_oracle(T):
    """Token counts on both sides of every change of kernel plan (16-row streaming,
    32-row streaming, the token-sharing GEMM1 on 64-row tiles with three and then two
    workgroups per CU feeding the token-sharing GEMM2 and then the prefill GEMM2, 256-row
    prefill tiles) and of the dispatch (one workgroup up to T = 640, count and place
    kernels over 256-token chunks beyond)."""
    d = first_tokens(config_inputs(3), T)
    note(f"[gpu] plan boundary T={T}")
    out = run_forward(d)
    rng = np.random.default_rng(T)
    toks = sorted(rng.choice(T, 16, replace=False).tolist())
    st = compare_to_oracle(d, out, toks)
    note(f"[gpu] T={T} stats {st}")
    assert st["frac_within"] == 1.0, st


@pytest.mark.parametrize("T,g1,g2", [(64, 1, 1), (150, 1, 1), (64, 2, 3), (500, 2, 3),
                                     (1000, 4, 5), (3000, 4, 5), (1500, 2, 5), (150, 1, 5),
                                     (1000, 7, 5), (300, 7, 5), (37, 7, 5), (2000, 7, 5),
                                     (600, 8, 5), (150, 8, 5), (1500, 8, 5), (500, 2, 5),
                                     (600, 8, 7), (1000, 7, 7), (300, 8, 7), (150, 8, 7),
                                     (37, 7, 7), (1500, 8, 7)])
def test_every_gemm_variant_matches_oracle(T, g1, g2):
    """Each GEMM1 / GEMM2 kernel variant (forced with the call's plan flags) stays
    within the tolerance."""
    d = first_tokens(config_inputs(3), T)
    note(f"[gpu] variants g1={g1} g2={g2} T={T}")
    out = run_forward(d, flags=pkg("kernel").plan_flags(g1, g2))
    rng = np.random.default_rng(T + 7)
    toks = sorted(rng.choice(T, 16, replace=False).tolist())
    st = compare_to_oracle(d, out, toks)
    note(f"[gpu] T={T} g1={g1} g2={g2} stats {st}")
    assert st["frac_within"] == 1.0, st


@pytest.mark.parametrize("T,offset", [(37, 224), (77, 32), (213, 32), (611, 0), (977, 64),
                                      (1311, 224), (1777, 32), (2459, 64), (3583, 0)])
def test_batch_sizes_between_plan_boundaries(T, offset):
    """Token counts away from the tested boundaries, one in each plan range, each with
    another expert offset (config 3 sliced to T): sampled tokens match the oracle and a
    second call on the same inputs is bit-identical."""
    d = first_tokens(config_inputs(3), T)
    d["local_expert_offset"] = offset
    note(f"[gpu] batch size T={T} offset={offset}")
    a = run_forward(d)
    b = run_forward(d)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    rng = np.random.default_rng(T)
    toks = sorted(rng.choice(T, 12, replace=False).tolist())
    st = compare_to_oracle(d, a, toks)
    note(f"[gpu] T={T} offset={offset} stats {st}")
    assert st["frac_within"] == 1.0, st


def test_concurrent_streams_match_serial():
    """Five calls of different plans (T = 8: routing, dispatch-in-GEMM1 streaming; 64;
    600: token-sharing GEMM1 at three workgroups per CU; 1024: at two; 2000: prefill),
    each on its own stream and workspace, issued together three times so that their
    kernels overlap on the device: every output equals the serial one bit for bit (the
    library keeps no per-call state outside the caller's workspace)."""
    k = pkg("kernel")
    wl = pkg("workloads")
    full = config_inputs(3)
    Ts = [8, 64, 600, 1024, 2000]
    ds = [first_tokens(full, T) for T in Ts]
    note("[gpu] concurrent streams: serial reference")
    ref = [run_forward(d) for d in ds]
    streams = [torch.cuda.Stream() for _ in Ts]        # default priority
    wss = [torch.empty(k.workspace_bytes(T), dtype=torch.uint8, device="cuda") for T in Ts]
    outs = [torch.full_like(d["output"], float("nan")) for d in ds]
    torch.cuda.synchronize()
    for rep in range(3):
        note(f"[gpu] concurrent streams: round {rep}")
        for d, st, ws, o in zip(ds, streams, wss, outs):
            with torch.cuda.stream(st):
                k.forward(*wl.as_args({**d, "output": o}), workspace=ws)
        torch.cuda.synchronize()
        for T, o, r in zip(Ts, outs, ref):
            assert torch.equal(o.view(torch.int16), r.view(torch.int16)), T


_RNG_T = np.random.default_rng(20261202)
_RANDOM_BATCHES = [(int(t), int(o)) for t, o in zip(_RNG_T.integers(1, 3000, 8),
                                                    _RNG_T.choice([0, 32, 64, 96, 224], 8))]


@pytest.mark.parametrize("T,offset", _RANDOM_BATCHES)
def test_seeded_random_batches(T, offset):
    """Seeded random token counts and offsets with their own activations and routing
    logits (seed 1000 + T, not slices of a benchmark config) on config 3's weights:
    sampled tokens match the oracle and a second call is bit-identical."""
    wl = pkg("workloads")
    cfg = wl.Config(f"random_t{T}", T, offset, seed=1000 + T)
    d = dict(config_inputs(3))
    d.update(wl.make_activations(cfg, device="cuda"))
    d["local_expert_offset"] = offset
    d["output"] = torch.empty(T, 7168, dtype=torch.bfloat16, device="cuda")
    note(f"[gpu] random batch T={T} offset={offset}")
    a = run_forward(d)
    b = run_forward(d)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    toks = sorted(np.random.default_rng(T + 1).choice(T, min(T, 12), replace=False).tolist())
    st = compare_to_oracle(d, a, toks)
    note(f"[gpu] random T={T} offset={offset} stats {st}")
    assert st["frac_within"] == 1.0, st


@pytest.mark.parametrize("T", [64, 200, 1024, 3000])
def test_row_order_token_scales_change_nothing(T):
    """GEMM1 reading the token scales gathered into row order (FLAG_ROW_SCALES_ON)
    or straight by token (FLAG_ROW_SCALES_OFF) gives bit-identical outputs on every
    plan; the gathered table holds hidden_states_scale[kb][sorted_tokens[row]] for
    the rows in use."""
    d = first_tokens(config_inputs(3), T)
    k = pkg("kernel")
    wl = pkg("workloads")
    lay = k.workspace_layout(T)
    outs = []
    for flag in (k.FLAG_ROW_SCALES_OFF, k.FLAG_ROW_SCALES_ON):
        note(f"[gpu] row-order token scales flag {flag} T={T}")
        ws = torch.empty(lay.total, dtype=torch.uint8, device="cuda")
        out = torch.full_like(d["output"], float("nan"))
        k.forward(*wl.as_args({**d, "output": out}), workspace=ws, flags=flag)
        torch.cuda.synchronize()
        outs.append(out)
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    na = int(ws[lay.meta + 32 * 4:lay.meta + 33 * 4].view(torch.int32).item())
    stok = ws[lay.sorted_tokens:lay.sorted_tokens + na * 4].view(torch.int32).long()
    tab = ws[lay.row_scales:lay.row_scales + 56 * 8 * T * 4].view(torch.float32).view(56, 8 * T)
    assert torch.equal(tab[:, :na], d["hidden_states_scale"][:, stok])


@pytest.mark.parametrize("idx,T,g1,g2", [(3, 1500, 0, 0), (3, 3500, 0, 0), (4, 3500, 0, 0),
                                         (3, 700, 4, 5), (3, 300, 4, 5), (1, None, 4, 5),
                                         (0, None, 4, 5), (3, 3501, 0, 0)])
def test_ranked_item_order_changes_nothing(idx, T, g1, g2):
    """The prefill GEMM1's ranked item order (the default up to T = 3500: every case but
    the last) and tile-list order (FLAG_LIST_ORDER) give bit-identical outputs over every
    token.  Only which workgroup computes an item differs; the workspace is filled with
    0xff (fp8 / fp16 NaN) before each call, so an item that either order computed never
    would show as NaN."""
    d = config_inputs(idx) if T is None else first_tokens(config_inputs(idx), T)
    k = pkg("kernel")
    wl = pkg("workloads")
    T = d["routing_logits"].shape[0]
    base = k.plan_flags(g1, g2) if g1 else 0
    lay = k.workspace_layout(T, base)
    outs = []
    for flag in (0, k.FLAG_LIST_ORDER):
        note(f"[gpu] item order config {idx} T={T} flags {base | flag}")
        ws = torch.full((lay.total,), 255, dtype=torch.uint8, device="cuda")
        out = torch.full_like(d["output"], float("nan"))
        k.forward(*wl.as_args({**d, "output": out}), workspace=ws, flags=base | flag)
        torch.cuda.synchronize()
        assert not torch.isnan(out).any()
        outs.append(out)
        del ws
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))


@pytest.mark.parametrize("T,g1,g2", [(64, 0, 0), (600, 0, 0), (2049, 0, 0), (600, 7, 5), (1100, 0, 0)])
def test_all_local_routing_matches_oracle(T, g1, g2):
    """Every token routed to 8 local experts (bias +3 on all 32 local experts, so group 0
    always wins and holds the whole top 8): N_a = 8T rows, the most the row-tile list
    and the workspace are sized for, on the 16-row plan, the 64-row token-sharing plans
    (three workgroups per CU at T = 600, two at T = 1100, and two forced at T = 600:
    150 rows per expert, full and partial 64-row tiles) and the 256-row plan."""
    k = pkg("kernel")
    wl = pkg("workloads")
    cfg = wl.Config("all_local", T, 0, hot_local_experts=tuple(range(32)), seed=20261111)
    d = dict(config_inputs(4))                   # offset 0: reuse its weights
    d.update(wl.make_activations(cfg, device="cuda"))
    d["output"] = torch.empty(T, 7168, dtype=torch.bfloat16, device="cuda")
    note(f"[gpu] all-local routing T={T} g1={g1} g2={g2}")
    ids, w = k.route(d["routing_logits"], d["routing_bias"], d["routed_scaling_factor"])
    g = k.dispatch(ids, w, 0, 16)
    torch.cuda.synchronize()
    assert int(g["exp_off"][-1].item()) == 8 * T
    out = run_forward(d, flags=k.plan_flags(g1, g2) if g1 else 0)
    rng = np.random.default_rng(T + 11)
    toks = sorted(rng.choice(T, min(T, 12), replace=False).tolist())
    st = compare_to_oracle(d, out, toks)
    note(f"[gpu] all-local T={T} stats {st}")
    assert st["frac_within"] == 1.0, st
    assert bool(torch.isfinite(out.float()).all())


def _flags(ws, lay):
    return ws[lay.meta + 35 * 4:lay.meta + 37 * 4].view(torch.int32).cpu().tolist()


def _huge_inputs_check(d, c_flag, flags=0):
    """Hidden-state scales 2^10 times larger: |C| and the expert rows reach ~1e6, far
    beyond the fp16 range.  The call must raise the expert-row flag (meta[36]) and,
    on the streaming plans, the C flag (meta[35]); the combine and GEMM2 (or the
    conversion to the hi/lo form) then apply the 16-column group exponents of the fp16
    forms, and the output is finite and within 1e-2 of the largest output
    of the fp32 oracle (elementwise atol 1e-2 means nothing at this scale: where terms
    of 1e6 cancel, even exact fp32 staging leaves errors far above it).  A normal call
    on the same workspace afterwards finds both flags cleared and gives the same output
    as a call on a fresh workspace."""
    k = pkg("kernel")
    wl = pkg("workloads")
    T = d["routing_logits"].shape[0]
    lay = k.workspace_layout(T, flags)
    ws = torch.empty(lay.total, dtype=torch.uint8, device="cuda")
    big = dict(d)
    big["hidden_states_scale"] = d["hidden_states_scale"] * 1024.0
    out = torch.full_like(d["output"], float("nan"))
    k.forward(*wl.as_args({**big, "output": out}), workspace=ws, flags=flags)
    torch.cuda.synchronize()
    assert _flags(ws, lay) == [c_flag, 1]
    o = oracle()
    ids, w = o.route(big["routing_logits"], big["routing_bias"], big["routed_scaling_factor"])
    toks = list(range(T)) if T <= 64 else sorted(np.random.default_rng(T).choice(T, 32, replace=False).tolist())
    args = (big["hidden_states"], big["hidden_states_scale"], big["gemm1_weights"], big["gemm1_weights_scale"],
            big["gemm2_weights"], big["gemm2_weights_scale"], ids, w, big["local_expert_offset"])
    ref32 = o.expert_forward(*args, tokens=toks)
    got = out[torch.as_tensor(toks, device="cuda")].float().cpu()
    scale = float(ref32.abs().max())
    e_32 = float((got - ref32).abs().max())
    res = dict(max_ref=scale, err_fp32=e_32)
    if c_flag:
        refb = o.expert_forward(*args, tokens=toks, intermediate_dtype=torch.bfloat16)
        res["err_bf16C"] = float((got - refb).abs().max())
        assert res["err_bf16C"] <= 4e-3 * scale
    note(f"[gpu] beyond fp16 (T={T}): {res}")
    assert scale > 65504.0
    assert bool(torch.isfinite(got).all())
    assert e_32 <= 1e-2 * scale

    out2 = torch.full_like(d["output"], float("nan"))
    k.forward(*wl.as_args({**d, "output": out2}), workspace=ws, flags=flags)
    torch.cuda.synchronize()
    assert _flags(ws, lay) == [0, 0]
    ref = run_forward(d, flags=flags)
    assert torch.equal(out2.view(torch.int16), ref.view(torch.int16))


def test_values_beyond_fp16_range_streaming_plan():
    """T = 64 (streaming plan, fp16 C, GEMM1 with the dispatch folded in): C and the
    expert rows both overflow fp16; GEMM2 runs its bf16 path (the output then equals
    the oracle with C rounded to bf16, to 4e-3 of the largest output)."""
    d = dict(config_inputs(1))
    note("[gpu] values beyond the fp16 range, T=64")
    _huge_inputs_check(d, c_flag=1)


def test_values_beyond_fp16_range_separate_dispatch():
    """The same with the separate dispatch launch (plan 1/1)."""
    d = dict(config_inputs(1))
    note("[gpu] values beyond the fp16 range, T=64, separate dispatch")
    _huge_inputs_check(d, c_flag=1, flags=pkg("kernel").plan_flags(1, 1))


def test_values_beyond_fp16_range_converted_plan():
    """T = 1024 with the 32-row streaming GEMM1 forced (GEMM1 variant 2, whose two
    column groups per item write the group exponents of C) and its fp16 C converted to
    the hi/lo form for the prefill GEMM2: the conversion applies the exponents."""
    d = first_tokens(config_inputs(3), 1024)
    note("[gpu] values beyond the fp16 range, T=1024, plan 2/5")
    _huge_inputs_check(d, c_flag=1, flags=pkg("kernel").plan_flags(2, 5))


def test_values_beyond_fp16_range_32_row_streaming_plan():
    """T = 150 (the default plan there: 32-row streaming GEMM1, variant 2, and the
    32-row streaming GEMM2, variant 3, whose rare path reads C's group exponents)."""
    d = first_tokens(config_inputs(3), 150)
    note("[gpu] values beyond the fp16 range, T=150, plan 2/3")
    lay = pkg("kernel").workspace_layout(150)
    assert lay.tile_m == 32 and lay.intermediate_format == 0
    _huge_inputs_check(d, c_flag=1)


def test_values_beyond_fp16_range_token_sharing_three_per_cu():
    """T = 600 (the token-sharing GEMM1 at three workgroups per CU, the plan there)."""
    d = first_tokens(config_inputs(3), 600)
    note("[gpu] values beyond the fp16 range, T=600, GEMM1 variant 8")
    _huge_inputs_check(d, c_flag=1)


def test_values_beyond_fp16_range_token_sharing_gemm1():
    """The same at T = 1024 with the token-sharing GEMM1 (64-row tiles) forced."""
    d = first_tokens(config_inputs(3), 1024)
    note("[gpu] values beyond the fp16 range, T=1024, GEMM1 variant 7")
    _huge_inputs_check(d, c_flag=1, flags=pkg("kernel").plan_flags(7, 5))


def test_values_beyond_fp16_range_token_sharing_gemm2():
    """T = 600 with the token-sharing GEMM2 (variant 7) forced after the token-sharing
    GEMM1: its rare path rebuilds C from the group exponents, one row block at a time."""
    d = first_tokens(config_inputs(3), 600)
    note("[gpu] values beyond the fp16 range, T=600, plan 8/7")
    _huge_inputs_check(d, c_flag=1, flags=pkg("kernel").plan_flags(8, 7))


def test_values_beyond_fp16_range_prefill_plan():
    """T = 2000 (prefill plan, fp8 hi/lo C, whose per-block scale covers any range):
    only the expert rows overflow fp16."""
    d = first_tokens(config_inputs(3), 2000)
    note("[gpu] values beyond the fp16 range, T=2000")
    _huge_inputs_check(d, c_flag=0)


def test_large_batch_matches_oracle_and_is_deterministic():
    """T = 32768 (4x the largest benchmark config; 262,144 routed rows, 256 dispatch
    chunks, a 15 GB workspace): sampled tokens match the oracle and two calls agree
    bit for bit."""
    k = pkg("kernel")
    wl = pkg("workloads")
    T = 32768
    cfg = wl.Config("large", T, 0, seed=20262222)
    d = dict(config_inputs(3))                    # offset 0: reuse its weights
    d.update(wl.make_activations(cfg, device="cuda"))
    d["output"] = torch.empty(T, 7168, dtype=torch.bfloat16, device="cuda")
    note(f"[gpu] large batch T={T} (workspace {k.workspace_bytes(T) / 1e9:.1f} GB)")
    out1 = run_forward(d)
    out2 = run_forward(d)
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16))
    toks = sorted(np.random.default_rng(T).choice(T, 8, replace=False).tolist()) + [0, T - 1]
    st = compare_to_oracle(d, out1, toks)
    note(f"[gpu] large batch stats {st}")
    assert st["frac_within"] == 1.0, st
