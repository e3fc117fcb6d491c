"""Pin the CPU oracle before trusting it (CPU only).

The reference ships no golden vectors or known-answer tests for this path, so each
oracle function is pinned by something it does not share code with:

* canonical sigmoid   <- torch float64 sigmoid rounded to fp32 (library routine)
* e4m3 decode         <- torch.float8_e4m3fn -> float32 (library routine) and the
                         OCP spec's named values
* routing             <- a torch restatement of moe.cu:178-206 (torch.topk,
                         masked_fill, scatter) on tie-free inputs; closed-form special
                         cases for the tie rule; structural invariants
* dispatch            <- numpy stable argsort (library routine); bijection and
                         inverse round trip
* dequant / experts   <- numpy float64 restatement with explicit index arithmetic on
                         the e4m3 table; a hand-built closed-form layer whose answer
                         is known analytically
Each pin is also shown to fail when a plausible mistake is planted in the oracle.
"""
import numpy as np
import pytest
import torch

from conftest import oracle, pkg

H, I, E_GLOBAL, E_LOCAL, TOP_K, BLK = 7168, 2048, 256, 32, 8, 128


# --------------------------------------------------------------------------- sigmoid

def test_sigmoid_matches_float64_rounded():
    o = oracle()
    rng = np.random.default_rng(1)
    xs = np.concatenate([
        rng.standard_normal(40000).astype(np.float32) * 3,
        rng.uniform(-90, 90, 20000).astype(np.float32),
        np.array([0.0, -0.0, 1e-30, -1e-30, 20.0, -20.0, 88.0, -88.0, 103.0, -103.0,
                  700.5, -700.5, 1e38, -1e38], dtype=np.float32),
    ])
    ours = o.sigmoid(xs)
    ref = torch.sigmoid(torch.from_numpy(xs).double()).float().numpy()
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


def test_sigmoid_special_values():
    o = oracle()
    assert o.sigmoid(np.float32(0.0)) == np.float32(0.5)
    assert o.sigmoid(np.float32(np.inf)) == 1.0
    assert o.sigmoid(np.float32(-np.inf)) == 0.0
    assert np.isnan(o.sigmoid(np.float32(np.nan)))


# --------------------------------------------------------------------------- e4m3

def test_e4m3_table_matches_torch_and_spec():
    o = oracle()
    tab = o.e4m3_table()
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(tab), nan)
    assert nan.sum() == 2 and nan[0x7F] and nan[0xFF]
    assert np.array_equal(tab[~nan], ref[~nan])
    # named values of the OCP FP8 spec
    assert tab[0x7E] == 448.0 and tab[0xFE] == -448.0
    assert tab[0x01] == 2.0 ** -9 and tab[0x08] == 2.0 ** -6 and tab[0x38] == 1.0


# --------------------------------------------------------------------------- routing

def _torch_routing(logits: np.ndarray, bias_bf16: torch.Tensor, factor: float):
    """moe.cu:178-206 as torch library calls (the reference's own op sequence)."""
    lg = torch.from_numpy(logits)
    T = lg.shape[0]
    s = torch.sigmoid(lg.double()).float()           # canonical sigmoid (pinned above)
    sb = s + bias_bf16.float()
    top2 = sb.view(T, 8, 32).topk(2, dim=2).values
    gs = top2.sum(2)
    gidx = gs.topk(4, dim=1).indices
    gmask = torch.zeros_like(gs).scatter_(1, gidx, 1.0)
    smask = gmask.unsqueeze(2).expand(T, 8, 32).reshape(T, 256)
    pruned = sb.masked_fill(smask == 0, float("-inf"))
    vals, idx = pruned.topk(8, dim=1)
    sel = s.gather(1, idx)
    w = sel / (sel.sum(1, keepdim=True) + 1e-20) * factor
    return idx.numpy().astype(np.int32), w.numpy(), sb.numpy(), gs.numpy()


def _near_tie_free(sb: np.ndarray, gs: np.ndarray, ids: np.ndarray) -> np.ndarray:
    """Tokens whose selection boundaries are separated by > 4 ulp (no near-ties),
    where any correct implementation must agree exactly."""
    ok = np.ones(sb.shape[0], bool)
    for t in range(sb.shape[0]):
        g = np.sort(gs[t])[::-1]
        if abs(g[3] - g[4]) <= 4 * np.spacing(np.float32(abs(g[3]))):
            ok[t] = False
        v = np.sort(sb[t])[::-1]
        if np.min(np.abs(np.diff(v[:40]))) <= 4 * np.spacing(np.float32(abs(v[0]))):
            ok[t] = False
    return ok


@pytest.fixture(scope="module")
def routing_case():
    wl = pkg("workloads")
    cfg = wl.CONFIGS[1]
    acts = wl.make_activations(cfg, T=2048)
    lg = acts["routing_logits"].numpy()
    return lg, acts["routing_bias"], cfg.routed_scaling_factor


def test_routing_matches_torch_restatement(routing_case):
    o = oracle()
    lg, bias, f = routing_case
    ids, w = o.route(lg, bias, f)
    tids, tw, sb, gs = _torch_routing(lg, bias, f)
    ok = _near_tie_free(sb, gs, tids)
    assert ok.mean() > 0.95
    assert np.array_equal(ids[ok], tids[ok])
    np.testing.assert_allclose(w[ok], tw[ok], rtol=2e-7, atol=0)


@pytest.mark.parametrize("mutation", [1, 3, 4])
def test_routing_pin_catches_planted_mistakes(routing_case, mutation):
    """Mutations 1 (top-1 group score) and 3 (weights from s+bias) must break the
    agreement with the torch restatement; 4 (ties to the higher index) must break
    the closed-form tie case."""
    o = oracle()
    lg, bias, f = routing_case
    try:
        o.set_mutation(mutation)
        ids, w = o.route(lg, bias, f)
        tie_ids, _ = o.route(np.zeros((1, 256), np.float32), torch.zeros(256, dtype=torch.bfloat16), f)
    finally:
        o.set_mutation(0)
    tids, tw, sb, gs = _torch_routing(lg, bias, f)
    ok = _near_tie_free(sb, gs, tids)
    agree = np.array_equal(ids[ok], tids[ok]) and np.allclose(w[ok], tw[ok], rtol=2e-7, atol=0)
    tie_ok = list(tie_ids[0]) == list(range(8))
    assert not (agree and tie_ok)


def test_routing_all_equal_closed_form():
    """s = 0.5 everywhere: groups 0..3 kept (tie -> lower group), experts 0..7
    (tie -> lower index), each weight = 0.5 / 4 * factor = factor / 8 exactly."""
    o = oracle()
    for f in (2.5, 1.0, 0.75):
        ids, w = o.route(np.zeros((3, 256), np.float32), torch.zeros(256, dtype=torch.bfloat16), f)
        assert (ids == np.arange(8)).all()
        assert (w == np.float32(f / 8)).all()


def test_routing_group_tie_goes_to_lower_group():
    o = oracle()
    o.set_mutation(0)
    lg = np.zeros((1, 256), np.float32)
    # groups 5 and 6 get identical top-2 sums, strictly above the rest; groups
    # 1 and 2 tie below them; the lower of each tied pair must be kept first
    for g, v in ((5, 4.0), (6, 4.0), (1, 2.0), (2, 2.0)):
        lg[0, g * 32 + 3] = v
        lg[0, g * 32 + 9] = v
    d = o.route_token_debug(lg[0], torch.zeros(256, dtype=torch.bfloat16), 2.5)
    assert d["keep"] == (1 << 5) | (1 << 6) | (1 << 1) | (1 << 2)
    assert list(d["ids"][:8]) == [163, 169, 195, 201, 35, 41, 67, 73]
    # boundary tie: groups 5, 6, 3 are clearly best; groups 1 and 7 tie for the
    # fourth slot, which must go to group 1
    lg2 = np.zeros((1, 256), np.float32)
    for g, v in ((5, 3.0), (6, 2.5), (3, 2.0), (1, 1.0), (7, 1.0)):
        lg2[0, g * 32] = lg2[0, g * 32 + 1] = v
    zb = torch.zeros(256, dtype=torch.bfloat16)
    good = o.route_token_debug(lg2[0], zb, 2.5)
    assert good["keep"] == (1 << 5) | (1 << 6) | (1 << 3) | (1 << 1)
    assert list(good["ids"]) == [160, 161, 192, 193, 96, 97, 32, 33]
    try:
        o.set_mutation(2)
        bad = o.route_token_debug(lg2[0], zb, 2.5)
    finally:
        o.set_mutation(0)
    assert bad["keep"] != good["keep"]


def test_routing_duplicate_group_max_counts_twice():
    o = oracle()
    lg = np.zeros((1, 256), np.float32)
    lg[0, 40] = lg[0, 41] = 2.0       # group 1: two equal maxima
    lg[0, 64] = 2.5                   # group 2: larger single max, second = s(0)
    d = o.route_token_debug(lg[0], torch.zeros(256, dtype=torch.bfloat16), 2.5)
    s2 = d["s"][40]
    assert d["gscore"][1] == np.float32(s2 + s2)
    assert d["gscore"][2] == np.float32(d["s"][64] + np.float32(0.5))


def test_routing_hot_bias_always_selected():
    o = oracle()
    rng = np.random.default_rng(5)
    lg = rng.standard_normal((256, 256)).astype(np.float32)
    b = torch.zeros(256)
    hot = [3, 11, 19, 27]
    b[hot] = 3.0
    ids, _ = o.route(lg, b.to(torch.bfloat16), 2.5)
    for t in range(256):
        assert set(hot) <= set(ids[t].tolist())


def test_routing_invariants(routing_case):
    o = oracle()
    lg, bias, f = routing_case
    ids, w = o.route(lg, bias, f)
    bf = bias.float().numpy()
    for t in range(0, lg.shape[0], 7):
        row = ids[t]
        assert len(set(row.tolist())) == 8
        assert len(set((row // 32).tolist())) <= 4
        s = torch.sigmoid(torch.from_numpy(lg[t]).double()).float().numpy()
        sb = s + bf
        keys = [(-sb[e], e) for e in row]
        assert keys == sorted(keys)
        assert abs(float(w[t].sum()) - f) < 1e-5


# --------------------------------------------------------------------------- dispatch

def _dispatch_case(T=300, offset=0, seed=3):
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.choice(256, 8, replace=False) for _ in range(T)]).astype(np.int32)
    # concentrate some mass in the local range
    ids[: T // 2, 0] = rng.integers(offset, offset + 32, T // 2)
    for t in range(T // 2):
        row = ids[t]
        while len(set(row.tolist())) < 8:
            row[1:] = rng.choice(256, 7, replace=False)
    w = rng.random((T, 8)).astype(np.float32)
    return ids, w


@pytest.mark.parametrize("offset,tm", [(0, 64), (64, 16), (224, 32), (250, 64)])
def test_dispatch_matches_stable_argsort(offset, tm):
    o = oracle()
    ids, w = _dispatch_case(offset=min(offset, 224))
    d = o.dispatch(ids, w, offset, tm)
    T = ids.shape[0]
    flat_e = ids.reshape(-1).astype(np.int64) - offset
    local = (flat_e >= 0) & (flat_e < 32)
    pos = np.nonzero(local)[0]
    order = pos[np.argsort(flat_e[pos], kind="stable")]
    assert np.array_equal(d["sorted_tok"], (order // 8).astype(np.int32))
    assert np.array_equal(d["sorted_w"], w.reshape(-1)[order])
    counts = np.bincount(flat_e[local], minlength=32)
    assert np.array_equal(d["exp_off"], np.concatenate([[0], np.cumsum(counts)]).astype(np.int32))
    inv = d["inv"].reshape(-1)
    assert (inv[~local] == -1).all()
    assert np.array_equal(np.sort(inv[local]), np.arange(local.sum()))
    assert np.array_equal(inv[order], np.arange(local.sum()))
    # tiles: ascending experts, each covers <= tm rows of its own expert, all rows once
    covered = np.zeros(local.sum(), int)
    for e, r0, n, _ in d["tiles"]:
        assert 0 < n <= tm
        assert d["exp_off"][e] <= r0 and r0 + n <= d["exp_off"][e + 1]
        covered[r0:r0 + n] += 1
    assert (covered == 1).all()


@pytest.mark.parametrize("mutation", [5, 6])
def test_dispatch_pin_catches_planted_mistakes(mutation):
    o = oracle()
    ids, w = _dispatch_case()
    try:
        o.set_mutation(mutation)
        d = o.dispatch(ids, w, 0, 16)
    finally:
        o.set_mutation(0)
    flat_e = ids.reshape(-1).astype(np.int64)
    local = flat_e < 32
    pos = np.nonzero(local)[0]
    order = pos[np.argsort(flat_e[pos], kind="stable")]
    perm_ok = np.array_equal(d["sorted_tok"], (order // 8).astype(np.int32))
    tiles_ok = all(r0 + n <= d["exp_off"][e + 1] for e, r0, n, _ in d["tiles"])
    assert not (perm_ok and tiles_ok)


def test_dispatch_empty_and_nonlocal():
    o = oracle()
    d = o.dispatch(np.zeros((0, 8), np.int32), np.zeros((0, 8), np.float32), 0, 64)
    assert d["tiles"].shape[0] == 0 and d["exp_off"][-1] == 0
    ids = np.tile(np.arange(8, dtype=np.int32), (5, 1))
    d = o.dispatch(ids, np.ones((5, 8), np.float32), 100, 64)
    assert (d["inv"] == -1).all() and d["exp_off"][-1] == 0


# --------------------------------------------------------------------------- expert path

def _np_dequant(q_bytes: np.ndarray, scale: np.ndarray) -> np.ndarray:
    tab = oracle().e4m3_table().astype(np.float64)
    r = np.arange(q_bytes.shape[0])[:, None] // BLK
    c = np.arange(q_bytes.shape[1])[None, :] // BLK
    return tab[q_bytes] * scale[r, c].astype(np.float64)


def test_dequant_weight_matches_index_arithmetic():
    o = oracle()
    wl = pkg("workloads")
    g = torch.Generator().manual_seed(7)
    w = torch.randn(256, 384, generator=g) * 0.02
    q, s = wl.quantize_blocks_128(w)
    s = s * torch.tensor([[1.0, 2.0, 0.5], [4.0, 0.25, 8.0]])  # make blocks distinguishable
    ref = _np_dequant(q.view(torch.uint8).numpy(), s.numpy())
    got = o.dequant_weight(q, s).numpy()
    np.testing.assert_array_equal(got, ref.astype(np.float32))
    bad = o.dequant_weight(q, s.flip(0)).numpy()
    assert not np.array_equal(bad, ref.astype(np.float32))


def test_dequant_hidden_scale_is_block_major():
    o = oracle()
    wl = pkg("workloads")
    x = torch.randn(5, H, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    q, sc = wl.quantize_rows_128(x)          # sc is [56, T]
    assert tuple(sc.shape) == (H // BLK, 5)
    tab = o.e4m3_table().astype(np.float64)
    qb = q.view(torch.uint8).numpy()
    ref = np.empty((5, H))
    for t in range(5):
        for h0 in range(0, H, BLK):
            ref[t, h0:h0 + BLK] = tab[qb[t, h0:h0 + BLK]] * float(sc[h0 // BLK, t])
    got = o.dequant_hidden(q, sc).numpy()
    np.testing.assert_array_equal(got, ref.astype(np.float32))
    # the quantiser reproduces the bf16 input within e4m3 resolution
    assert np.max(np.abs(got - x.float().numpy()) / (np.abs(x.float().numpy()) + 0.05)) < 0.07


def _closed_form_layer(offset=0):
    """A layer whose output is known analytically.

    Expert le gets W13 gate row n = unit vector at hidden column 2n, up row n = unit
    vector at column 2n+1 (e4m3 1.0, scales 1), and W2 row h = unit vector at
    intermediate column h % 2048 with block scale 2 for h < 128.  Then for a token
    with dequantised hidden a and routing weight w:
        out[h] = w * silu(a[2j+1]) * a[2j] * (2 if h < 128 else 1),   j = h % 2048."""
    one = 0x38
    w1 = torch.zeros(E_LOCAL, 2 * I, H, dtype=torch.uint8)
    w2 = torch.zeros(E_LOCAL, H, I, dtype=torch.uint8)
    for le in (0, 5):
        n = torch.arange(I)
        w1[le, n, 2 * n] = one
        w1[le, I + n, 2 * n + 1] = one
        h = torch.arange(H)
        w2[le, h, h % I] = one
    s1 = torch.ones(E_LOCAL, 2 * I // BLK, H // BLK)
    s2 = torch.ones(E_LOCAL, H // BLK, I // BLK)
    s2[:, 0, :] = 2.0
    return (w1.view(torch.float8_e4m3fn), s1, w2.view(torch.float8_e4m3fn), s2)


def test_expert_path_closed_form():
    o = oracle()
    wl = pkg("workloads")
    T = 4
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    hs, sc = wl.quantize_rows_128(x)
    a = o.dequant_hidden(hs, sc).double()
    w1, s1, w2, s2 = _closed_form_layer()
    ids = np.array([[0, 100, 101, 102, 103, 104, 105, 106],
                    [5, 0, 200, 201, 202, 203, 204, 205],
                    [100, 101, 102, 103, 104, 105, 106, 107],
                    [5, 110, 111, 112, 113, 114, 115, 116]], np.int32)
    wts = np.array([[0.3] + [0.1] * 7, [0.25, 0.5] + [0.1] * 6, [0.1] * 8, [0.7] + [0.1] * 7], np.float32)
    acc = o.expert_forward(hs, sc, w1, s1, w2, s2, ids, wts, 0).double()
    j = torch.arange(H) % I
    c = torch.nn.functional.silu(a[:, 2 * j + 1]) * a[:, 2 * j]
    c[:, :128] *= 2.0
    expect = torch.zeros(T, H, dtype=torch.float64)
    expect[0] = 0.3 * c[0]
    expect[1] = (0.25 + 0.5) * c[1]
    expect[3] = 0.7 * c[3]
    torch.testing.assert_close(acc, expect, rtol=1e-5, atol=1e-6)
    assert (acc[2] == 0).all()


def test_expert_path_pin_catches_swapped_swiglu(monkeypatch):
    o = oracle()
    wl = pkg("workloads")
    x = torch.randn(2, H, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    hs, sc = wl.quantize_rows_128(x)
    w1, s1, w2, s2 = _closed_form_layer()
    ids = np.array([[0] + list(range(100, 107))] * 2, np.int32)
    wts = np.full((2, 8), 0.125, np.float32)
    good = o.expert_forward(hs, sc, w1, s1, w2, s2, ids, wts, 0)
    real = o.silu
    # plant: silu applied to the first half instead of the second
    monkeypatch.setattr(o, "silu", lambda v: v)
    bad = o.expert_forward(hs, sc, w1, s1, w2, s2, ids, wts, 0)
    monkeypatch.setattr(o, "silu", real)
    assert not torch.allclose(good, bad, rtol=1e-3, atol=1e-4)


def test_expert_path_matches_float64_restatement():
    """Random weights for two experts vs a per-token float64 numpy restatement."""
    o = oracle()
    wl = pkg("workloads")
    cfg = wl.Config("pin", 16, 64, seed=11)
    acts = wl.make_activations(cfg)
    ids, w = o.route(acts["routing_logits"], acts["routing_bias"], 2.5)
    le_hit = sorted({int(e) - 64 for e in ids.reshape(-1) if 0 <= int(e) - 64 < 32})[:2]
    assert le_hit
    wts = wl.make_weights(cfg, experts=le_hit)
    toks = [t for t in range(16) if any(int(e) - 64 in le_hit for e in ids[t])][:3]
    acc = o.expert_forward(acts["hidden_states"], acts["hidden_states_scale"],
                           wts["gemm1_weights"], wts["gemm1_weights_scale"],
                           wts["gemm2_weights"], wts["gemm2_weights_scale"], ids, w, 64,
                           tokens=toks).double().numpy()
    tab = o.e4m3_table().astype(np.float64)
    hs = acts["hidden_states"].view(torch.uint8).numpy()
    hsc = acts["hidden_states_scale"].numpy().astype(np.float64)
    for i, t in enumerate(toks):
        a = tab[hs[t]] * np.repeat(hsc[:, t], BLK)
        out = np.zeros(H)
        for k in range(8):
            le = int(ids[t, k]) - 64
            if le not in le_hit:
                continue
            W13 = _np_dequant(wts["gemm1_weights"][le].view(torch.uint8).numpy(),
                              wts["gemm1_weights_scale"][le].numpy())
            W2 = _np_dequant(wts["gemm2_weights"][le].view(torch.uint8).numpy(),
                             wts["gemm2_weights_scale"][le].numpy())
            g1 = W13 @ a
            x1, x2 = g1[:I], g1[I:]
            cvec = x2 / (1 + np.exp(-x2)) * x1
            out += float(w[t, k]) * (W2 @ cvec)
        np.testing.assert_allclose(acc[i], out, rtol=2e-4, atol=2e-5)


def test_combine_linear_in_factor_and_zero_for_nonlocal():
    o = oracle()
    wl = pkg("workloads")
    cfg = wl.Config("pin2", 12, 0, seed=13)
    acts = wl.make_activations(cfg)
    ids, w = o.route(acts["routing_logits"], acts["routing_bias"], 2.5)
    hit = sorted({int(e) for e in ids.reshape(-1) if int(e) < 32})
    wts = wl.make_weights(cfg, experts=hit[:1])
    args = (acts["hidden_states"], acts["hidden_states_scale"], wts["gemm1_weights"],
            wts["gemm1_weights_scale"], wts["gemm2_weights"], wts["gemm2_weights_scale"])
    a1 = o.expert_forward(*args, ids, w, 0)
    a2 = o.expert_forward(*args, ids, w * 2, 0)
    assert torch.equal(a2, a1 * 2)
    nonlocal_tok = [t for t in range(12) if not any(int(e) < 32 for e in ids[t])]
    for t in nonlocal_tok:
        assert (a1[t] == 0).all()


# --------------------------------------------------------------------------- fp8 hi/lo form of C

def _hilo_blocks():
    g = torch.Generator().manual_seed(11)
    C = torch.randn(48, I, generator=g) * torch.logspace(-3, 2, 48).unsqueeze(1)
    C[3, :128] = 0.0                                  # an all-zero block
    C[4, 128:256] = 1e-30                             # a denormal-scale block
    C[5, 256:384] = torch.linspace(-1, 1, 128)        # exact zero inside a block
    C[6, ::7] *= 1e-4                                 # elements far below the block max
    return C


def test_hilo_reconstruction_bound():
    """|s(hi + lo/16) - c| <= 2^-8 |c| + 2^-13 s for every element (lo carries the
    residual of hi with e4m3's relative precision 2^-4, or its subnormal step)."""
    o = oracle()
    C = _hilo_blocks()
    hi, lo, s = o.hilo_split(C)
    back = o.hilo_join(hi, lo, s)
    sfull = s.repeat_interleave(BLK, 1)
    err = (back - C).abs()
    assert (err <= C.abs() * 2.0 ** -8 + sfull * 2.0 ** -13).all()
    assert (back[3, :128] == 0).all()


def test_hilo_lo_term_matters():
    """Dropping lo (a plausible mistake) loses ~4 bits: the pin above then fails."""
    o = oracle()
    C = _hilo_blocks()
    hi, lo, s = o.hilo_split(C)
    no_lo = o.hilo_join(hi, torch.zeros_like(lo), s)
    sfull = s.repeat_interleave(BLK, 1)
    assert not ((no_lo - C).abs() <= C.abs() * 2.0 ** -8 + sfull * 2.0 ** -13).all()


def test_hilo_exact_for_representable_values():
    """Values of the form s * (e4m3 + e4m3/16) with s = amax/448 come back exactly."""
    o = oracle()
    codes = torch.arange(0, 126, dtype=torch.uint8)          # positive finite e4m3 codes
    vals = codes.view(torch.float8_e4m3fn).float()
    C = torch.zeros(1, I)
    C[0, :126] = vals                                          # block 0: amax = 448 -> s = 1
    C[0, 126] = 448.0
    C[0, 127] = -(1.0 + 1.0 / 16)                              # hi = -1, lo = -1
    hi, lo, s = o.hilo_split(C)
    assert float(s[0, 0]) == 1.0
    assert torch.equal(o.hilo_join(hi, lo, s)[0, :128], C[0, :128])
