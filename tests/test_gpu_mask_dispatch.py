"""The forward's one-launch dispatch for 400 <= T <= 16384: the route kernel also writes
each token's local-expert mask, and every workgroup of the dispatch counts all T tokens'
experts from the masks (a bit transpose per wave and a popcount), then places its own
256-token chunk; where GEMM1 reads the token scales in row order it also writes them.
Everything it leaves in the workspace must equal the oracle's bit for bit: the masks,
the expert offsets, both tile lists, the permutation with its weights, the inverse map
and the row-order token scales.  T = 16385 checks the count, place and gather launches
that still run beyond that range."""
import functools

import numpy as np
import pytest
import torch

from conftest import oracle, pkg
from gpu_common import config_inputs, first_tokens, note

pytestmark = pytest.mark.gpu


@functools.lru_cache(maxsize=None)
def _big_inputs() -> dict:
    """16385 tokens over config 3's weights: its 8192 tokens, then the same tokens with
    their logits rotated by 37 experts (other routes), then one more."""
    d0 = config_inputs(3)
    T0 = d0["routing_logits"].shape[0]
    idx = torch.arange(16385, device="cuda") % T0
    lg = d0["routing_logits"][idx].clone()
    lg[T0:] = torch.roll(lg[T0:], shifts=37, dims=1)
    d = dict(d0)
    d["routing_logits"] = lg.contiguous()
    d["hidden_states"] = d0["hidden_states"][idx].contiguous()
    d["hidden_states_scale"] = d0["hidden_states_scale"][:, idx].contiguous()
    d["output"] = torch.empty(16385, d0["output"].shape[1], dtype=torch.bfloat16, device="cuda")
    torch.cuda.synchronize()
    return d


def _inputs(src, T, offset):
    d = first_tokens(_big_inputs() if src == "big" else config_inputs(src), T)
    d["local_expert_offset"] = offset
    return d


@pytest.mark.parametrize("src,T,offset,flags", [
    (3, 399, 0, 0), (3, 400, 0, 0), (3, 641, 0, 0), (3, 1000, 96, 0), (2, 1024, 64, "rows_on"), (3, 1344, 224, 0),
    (3, 1345, 0, 0), (3, 2049, 32, 0), (4, 4096, 0, 0), (3, 4097, 160, 0), (3, 8192, 0, 0),
    ("big", 16384, 0, 0), ("big", 16384, 224, 0), ("big", 16385, 0, 0)])
def test_workspace_dispatch_is_bit_exact(src, T, offset, flags):
    k = pkg("kernel")
    wl = pkg("workloads")
    fl = k.FLAG_ROW_SCALES_ON if flags == "rows_on" else 0
    d = _inputs(src, T, offset)
    lay = k.workspace_layout(T, fl)
    ws = torch.empty(lay.total, dtype=torch.uint8, device="cuda")
    note(f"[gpu] mask dispatch src={src} T={T} offset={offset} flags={fl} tile_m={lay.tile_m}")
    out = torch.empty_like(d["output"])
    k.forward(*wl.as_args({**d, "output": out}), workspace=ws, flags=fl)
    torch.cuda.synchronize()

    def arr(off, n, dt):
        return ws[off:off + n * 4].view(dt).cpu().numpy()

    o = oracle()
    rids, rw = o.route(d["routing_logits"], d["routing_bias"], d["routed_scaling_factor"])
    assert np.array_equal(arr(lay.topk_ids, T * 8, torch.int32).reshape(T, 8), rids)
    le = rids.astype(np.int64) - offset
    loc = (le >= 0) & (le < 32)
    masks = np.bitwise_or.reduce(np.where(loc, np.left_shift(1, np.where(loc, le, 0)), 0), axis=1)
    if 400 <= T <= 16384:
        assert np.array_equal(arr(lay.token_masks, T, torch.int32).view(np.uint32),
                              masks.astype(np.uint32))
    r = o.dispatch(rids, rw, offset, lay.tile_m)
    meta = arr(lay.meta, 35, torch.int32)
    assert np.array_equal(meta[:33], r["exp_off"])
    nt = r["tiles"].shape[0]
    assert meta[33] == nt
    assert np.array_equal(arr(lay.tiles, nt * 4, torch.int32).reshape(nt, 4), r["tiles"])
    if lay.intermediate_format != 0:      # the plans with the 128-row second list for GEMM2
        r2 = o.dispatch(rids, rw, offset, 128)
        nt2 = r2["tiles"].shape[0]
        assert meta[34] == nt2
        off2 = lay.tiles + ((8 * T + lay.tile_m - 1) // lay.tile_m + 32) * 16   # after max_tiles(T, tile_m)
        assert np.array_equal(arr(off2, nt2 * 4, torch.int32).reshape(nt2, 4), r2["tiles"])
    na = int(r["exp_off"][-1])
    assert np.array_equal(arr(lay.sorted_tokens, na, torch.int32), r["sorted_tok"])
    assert np.array_equal(arr(lay.sorted_weights, na, torch.float32).view(np.uint32),
                          np.asarray(r["sorted_w"], np.float32).view(np.uint32))
    assert np.array_equal(arr(lay.inverse_rows, T * 8, torch.int32).reshape(T, 8), r["inv"])
    if T >= 1345 or fl:                   # GEMM1 reads the token scales in row order
        stok = torch.from_numpy(np.asarray(r["sorted_tok"], np.int64)).cuda()
        tab = ws[lay.row_scales:lay.row_scales + 56 * 8 * T * 4].view(torch.float32).view(56, 8 * T)
        assert torch.equal(tab[:, :na], d["hidden_states_scale"][:, stok])


def test_one_workspace_across_sizes():
    """Calls of different sizes on one workspace sized for the largest: each call's
    dispatch is its own (the masks and counts of a larger call before it do not leak)."""
    k = pkg("kernel")
    wl = pkg("workloads")
    o = oracle()
    ws = torch.empty(k.workspace_layout(8192).total, dtype=torch.uint8, device="cuda")
    for T in (8192, 700, 3000, 400):
        d = _inputs(3, T, 0)
        lay = k.workspace_layout(T)
        note(f"[gpu] mask dispatch on a shared workspace T={T}")
        out = torch.empty_like(d["output"])
        k.forward(*wl.as_args({**d, "output": out}), workspace=ws)
        torch.cuda.synchronize()
        rids, rw = o.route(d["routing_logits"], d["routing_bias"], d["routed_scaling_factor"])
        r = o.dispatch(rids, rw, 0, lay.tile_m)
        na = int(r["exp_off"][-1])
        got = ws[lay.sorted_tokens:lay.sorted_tokens + na * 4].view(torch.int32).cpu().numpy()
        assert np.array_equal(got, r["sorted_tok"])
        inv = ws[lay.inverse_rows:lay.inverse_rows + T * 32].view(torch.int32).cpu().numpy()
        assert np.array_equal(inv.reshape(T, 8), r["inv"])


@pytest.mark.parametrize("T", [500, 3000])
def test_no_local_expert(T):
    """An offset that selects no expert: every mask is 0, the counts and tile lists are
    empty, and the output is exactly zero."""
    k = pkg("kernel")
    wl = pkg("workloads")
    d = _inputs(3, T, 1000)
    lay = k.workspace_layout(T)
    ws = torch.empty(lay.total, dtype=torch.uint8, device="cuda")
    out = torch.full_like(d["output"], float("nan"))
    note(f"[gpu] mask dispatch, no local expert, T={T}")
    k.forward(*wl.as_args({**d, "output": out}), workspace=ws)
    torch.cuda.synchronize()
    assert (out.view(torch.int16) == 0).all()
    masks = ws[lay.token_masks:lay.token_masks + T * 4].view(torch.int32)
    assert (masks == 0).all()
    meta = ws[lay.meta:lay.meta + 35 * 4].view(torch.int32).cpu().numpy()
    assert (meta[:34] == 0).all()          # offsets, tile count
    if lay.intermediate_format != 0:       # the plans with a second tile list
        assert meta[34] == 0


def test_all_local_workspace_is_bit_exact():
    """Every token routed to 8 local experts (T = 1500: 1500 rows per expert, six full
    256-row tiles each, twelve 128-row ones): the counts reach their maximum and the
    dispatch and row-order scales still equal the oracle's bit for bit."""
    k = pkg("kernel")
    wl = pkg("workloads")
    T = 1500
    cfg = wl.Config("all_local", T, 0, hot_local_experts=tuple(range(32)), seed=20261202)
    d = dict(config_inputs(4))                   # offset 0: reuse its weights
    d.update(wl.make_activations(cfg, device="cuda"))
    d["output"] = torch.empty(T, 7168, dtype=torch.bfloat16, device="cuda")
    d["local_expert_offset"] = 0
    lay = k.workspace_layout(T)
    ws = torch.empty(lay.total, dtype=torch.uint8, device="cuda")
    note(f"[gpu] mask dispatch, all local, T={T}")
    k.forward(*wl.as_args({**d, "output": torch.empty_like(d["output"])}), workspace=ws)
    torch.cuda.synchronize()
    o = oracle()
    rids, rw = o.route(d["routing_logits"], d["routing_bias"], d["routed_scaling_factor"])
    r = o.dispatch(rids, rw, 0, lay.tile_m)
    assert int(r["exp_off"][-1]) == 8 * T
    na = 8 * T
    meta = ws[lay.meta:lay.meta + 35 * 4].view(torch.int32).cpu().numpy()
    assert np.array_equal(meta[:33], r["exp_off"])
    assert np.array_equal(ws[lay.sorted_tokens:lay.sorted_tokens + na * 4].view(torch.int32).cpu().numpy(),
                          r["sorted_tok"])
    assert np.array_equal(ws[lay.inverse_rows:lay.inverse_rows + na * 4].view(torch.int32).cpu().numpy()
                          .reshape(T, 8), r["inv"])
    m = ws[lay.token_masks:lay.token_masks + T * 4].view(torch.int32).cpu().numpy().view(np.uint32)
    assert (sum((m >> i) & 1 for i in range(32)) == 8).all()     # eight local experts each
    stok = torch.from_numpy(np.asarray(r["sorted_tok"], np.int64)).cuda()
    tab = ws[lay.row_scales:lay.row_scales + 56 * na * 4].view(torch.float32).view(56, na)
    assert torch.equal(tab, d["hidden_states_scale"][:, stok])
