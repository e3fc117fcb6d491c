"""The workload runner's checks and report (tests/run_local.py), without a GPU: the
status of an output against the fp32 reference (a planted wrong element or a NaN makes
it INCORRECT_NUMERICAL), the one-line report per workload in the layout of the
reference's scripts/run_local.py:80-98, and the workload file format round trip."""
import importlib.util
import os

import pytest
import torch

from conftest import REPO


@pytest.fixture(scope="module")
def rl():
    spec = importlib.util.spec_from_file_location("run_local_under_test", os.path.join(REPO, "tests", "run_local.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


def _ref(seed=3):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(6, 7168, generator=g) * 3


def test_exact_output_passes(rl):
    ref = _ref()
    st = rl.check_output(ref.to(torch.bfloat16), ref)
    assert st["status"] == "PASSED" and st["frac_within"] == 1.0
    assert st["max_abs_error"] <= 3 * 2 ** -8 * 4 and st["checked_elements"] == 6 * 7168


@pytest.mark.parametrize("plant", ["one element off", "nan", "all scaled"])
def test_planted_wrong_output_is_incorrect(rl, plant):
    ref = _ref()
    got = ref.to(torch.bfloat16)
    if plant == "one element off":
        got[2, 100] += 0.5
    elif plant == "nan":
        got[5, 7000] = float("nan")
    else:
        got = (ref * 1.05).to(torch.bfloat16)
    st = rl.check_output(got, ref)
    assert st["status"] == "INCORRECT_NUMERICAL", st


def test_report_lines(rl):
    r = dict(status="PASSED", latency_ms=0.10712, reference_latency_ms=701.4, speedup_factor=6547.8,
             max_abs_error=8.4e-3, max_rel_error=3.1e-2)
    assert rl.format_result("decode_t64", r) == (
        "  Workload decode_t64: PASSED | 0.107 ms | ref 701.4 ms | 6547.80x speedup"
        " | abs_err=8.40e-03, rel_err=3.10e-02")
    bad = dict(status="RUNTIME_ERROR", error="RuntimeError: moe_mi355_forward failed")
    assert rl.format_result("w.safetensors", bad) == (
        "  Workload w.safetensors: RUNTIME_ERROR | RuntimeError: moe_mi355_forward failed")


def test_workload_file_round_trip(rl, tmp_path):
    """The file layout (names, dtypes, scalars); tiny tensors stand in for the real shapes."""
    g = torch.Generator().manual_seed(1)
    d = dict(routing_logits=torch.randn(3, 256, generator=g),
             routing_bias=torch.randn(256, generator=g).to(torch.bfloat16),
             hidden_states=torch.randn(3, 256, generator=g).to(torch.float8_e4m3fn),
             hidden_states_scale=torch.rand(2, 3, generator=g),
             gemm1_weights=torch.randn(2, 4, 8, generator=g).to(torch.float8_e4m3fn),
             gemm1_weights_scale=torch.rand(2, 1, 1, generator=g),
             gemm2_weights=torch.randn(2, 8, 4, generator=g).to(torch.float8_e4m3fn),
             gemm2_weights_scale=torch.rand(2, 1, 1, generator=g),
             local_expert_offset=64, routed_scaling_factor=2.5)
    p = str(tmp_path / "w.safetensors")
    rl.save_workload(p, d)
    e = rl.load_workload(p, "cpu")
    for k in rl.ARG_NAMES[:8]:
        assert e[k].dtype == d[k].dtype and torch.equal(e[k].view(torch.uint8), d[k].view(torch.uint8)), k
    assert e["local_expert_offset"] == 64 and e["routed_scaling_factor"] == 2.5
    assert tuple(e["output"].shape) == (3, 7168) and e["output"].dtype == torch.bfloat16
    from safetensors.torch import save_file
    save_file({"routing_logits": d["routing_logits"]}, str(tmp_path / "bad.safetensors"))
    with pytest.raises(ValueError, match="missing"):
        rl.load_workload(str(tmp_path / "bad.safetensors"), "cpu")
