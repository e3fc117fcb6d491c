"""HIP path against the committed golden fixtures (through the C ABI, on the GPU).

routing and dispatch: bit-exact; forward: within |gpu - ref| <= 1e-2 + 1e-2 |ref| of
the fixture's fp32 accumulator, and exactly zero for the token with no local expert.
"""
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN_DIR, load_module, pkg
from gpu_common import ATOL, RTOL, note

pytestmark = pytest.mark.gpu


def _load(name):
    return np.load(os.path.join(GOLDEN_DIR, name), allow_pickle=False)


def _bias(bits):
    return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)


def test_golden_routing():
    k = pkg("kernel")
    f = _load("routing.npz")
    for i, name in enumerate(f["names"]):
        note(f"[gpu] golden routing case {name}")
        ids, w = k.route(torch.from_numpy(f[f"c{i}_logits"]).cuda(), _bias(f[f"c{i}_bias_bits"]).cuda(),
                         float(f[f"c{i}_factor"]))
        torch.cuda.synchronize()
        assert np.array_equal(ids.cpu().numpy(), f[f"c{i}_ids"]), name
        assert np.array_equal(w.cpu().numpy().view(np.uint32), f[f"c{i}_w_bits"]), name


@pytest.mark.parametrize("off", [0, 64, 224])
@pytest.mark.parametrize("tm", [16, 64])
def test_golden_dispatch(off, tm):
    k = pkg("kernel")
    f = _load("dispatch.npz")
    note(f"[gpu] golden dispatch offset {off} tile_m {tm}")
    g = k.dispatch(torch.from_numpy(f["ids"]).cuda(),
                   torch.from_numpy(f["w_bits"].view(np.float32)).cuda(), off, tm)
    torch.cuda.synchronize()
    key = f"o{off}_m{tm}"
    eo = f[f"{key}_exp_off"]
    na = int(eo[-1])
    nt = f[f"{key}_tiles"].shape[0]
    assert np.array_equal(g["exp_off"].cpu().numpy(), eo)
    assert int(g["num_tiles"].item()) == nt
    assert np.array_equal(g["sorted_tok"][:na].cpu().numpy(), f[f"{key}_sorted_tok"])
    assert np.array_equal(g["sorted_w"][:na].cpu().numpy().view(np.uint32), f[f"{key}_sorted_w_bits"])
    assert np.array_equal(g["inv"].cpu().numpy(), f[f"{key}_inv"])
    assert np.array_equal(g["tiles"][:nt].cpu().numpy(), f[f"{key}_tiles"])


def test_golden_forward():
    k = pkg("kernel")
    f = _load("forward.npz")
    mg = load_module("moe_make_golden", os.path.join(GOLDEN_DIR, "make_golden.py"))
    note("[gpu] golden forward: regenerating 3 experts on the CPU")
    wts = mg.forward_weights(pkg("workloads"))
    assert np.array_equal(mg.weight_checksum(wts), f["weight_checksum"]), "weight generator drifted"
    wts = {n: t.cuda() for n, t in wts.items()}
    T = f["logits"].shape[0]
    out = torch.full((T, 7168), float("nan"), dtype=torch.bfloat16, device="cuda")
    k.kernel(torch.from_numpy(f["logits"]).cuda(), _bias(f["bias_bits"]).cuda(),
             torch.from_numpy(f["hidden_states"]).view(torch.float8_e4m3fn).cuda(),
             torch.from_numpy(f["hidden_states_scale"]).cuda(),
             wts["gemm1_weights"], wts["gemm1_weights_scale"], wts["gemm2_weights"],
             wts["gemm2_weights_scale"], int(f["local_expert_offset"]), float(f["factor"]), out)
    torch.cuda.synchronize()
    got = out.float().cpu()
    ref = torch.from_numpy(f["acc"])
    err = (got - ref).abs()
    note(f"[gpu] golden forward max_abs {float(err.max()):.3e}")
    assert (err <= ATOL + RTOL * ref.abs()).all()
    assert (got[5] == 0).all()
