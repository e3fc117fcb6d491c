"""The CPU oracle reproduces the committed golden fixtures (CPU only).

The fixtures in tests/golden/ were written by tests/golden/make_golden.py from the
pinned oracle; these tests fail if the oracle (or the synthetic weight generator
the forward fixture relies on) drifts from them.  The GPU side of the same fixtures
is tests/test_gpu_golden.py.
"""
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN_DIR, oracle, pkg, load_module


def _load(name):
    return np.load(os.path.join(GOLDEN_DIR, name), allow_pickle=False)


def _make_golden():
    return load_module("moe_make_golden", os.path.join(GOLDEN_DIR, "make_golden.py"))


def test_routing_fixture():
    f = _load("routing.npz")
    o = oracle()
    names = list(f["names"])
    assert len(names) >= 6
    for i, _ in enumerate(names):
        bias = torch.from_numpy(f[f"c{i}_bias_bits"].view(np.int16)).view(torch.bfloat16)
        ids, w = o.route(f[f"c{i}_logits"], bias, float(f[f"c{i}_factor"]))
        assert np.array_equal(ids, f[f"c{i}_ids"]), names[i]
        assert np.array_equal(w.view(np.uint32), f[f"c{i}_w_bits"]), names[i]


def test_routing_fixture_closed_forms():
    """The fixture's own closed-form cases, independent of the oracle."""
    f = _load("routing.npz")
    names = list(f["names"])
    eq = names.index("equal")
    assert (f[f"c{eq}_ids"] == np.arange(8)).all()
    assert (f[f"c{eq}_w_bits"].view(np.float32) == np.float32(2.5 / 8)).all()
    dup = names.index("dup_max")
    assert (f[f"c{dup}_ids"][:, :3] == [64, 40, 41]).all()


@pytest.mark.parametrize("off", [0, 64, 224])
@pytest.mark.parametrize("tm", [16, 64])
def test_dispatch_fixture(off, tm):
    f = _load("dispatch.npz")
    o = oracle()
    r = o.dispatch(f["ids"], f["w_bits"].view(np.float32), off, tm)
    k = f"o{off}_m{tm}"
    assert np.array_equal(r["exp_off"], f[f"{k}_exp_off"])
    assert np.array_equal(r["sorted_tok"], f[f"{k}_sorted_tok"])
    assert np.array_equal(r["sorted_w"].view(np.uint32), f[f"{k}_sorted_w_bits"])
    assert np.array_equal(r["inv"], f[f"{k}_inv"])
    assert np.array_equal(r["tiles"], f[f"{k}_tiles"])


def test_forward_fixture():
    f = _load("forward.npz")
    o = oracle()
    mg = _make_golden()
    wl = pkg("workloads")
    wts = mg.forward_weights(wl)
    assert np.array_equal(mg.weight_checksum(wts), f["weight_checksum"]), "weight generator drifted"
    hs = torch.from_numpy(f["hidden_states"]).view(torch.float8_e4m3fn)
    hs_scale = torch.from_numpy(f["hidden_states_scale"])
    bias = torch.from_numpy(f["bias_bits"].view(np.int16)).view(torch.bfloat16)
    ids, w = o.route(f["logits"], bias, float(f["factor"]))
    assert np.array_equal(ids, f["ids"])
    acc = o.expert_forward(hs, hs_scale, wts["gemm1_weights"], wts["gemm1_weights_scale"],
                           wts["gemm2_weights"], wts["gemm2_weights_scale"], ids, w,
                           int(f["local_expert_offset"]))
    ref = torch.from_numpy(f["acc"])
    # fp32 CPU GEMMs may sum in another order on another BLAS build
    assert torch.allclose(acc, ref, atol=1e-5, rtol=1e-5)
    assert (ref[5] == 0).all() and (ref[:5].abs().amax(dim=1) > 1).all()
