"""The workload runner on the GPU: a config passes with its latency, the CPU reference's
latency and the speedup reported, and a planted wrong output is reported as
INCORRECT_NUMERICAL."""
import importlib.util
import os

import pytest

from conftest import REPO
from gpu_common import config_inputs, note

pytestmark = pytest.mark.gpu


def _rl():
    spec = importlib.util.spec_from_file_location("run_local_gpu", os.path.join(REPO, "tests", "run_local.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


def test_runner_passes_and_reports():
    rl = _rl()
    d = dict(config_inputs(0))
    note("[gpu] run_local on decode_t8")
    r = rl.run_workload(d, warmup=2, iterations=10, trials=2, cpu_runs=1)
    note("[gpu] " + rl.format_result("decode_t8", r))
    assert r["status"] == "PASSED", r
    assert 0 < r["latency_ms"] < 1.0 and r["reference_latency_ms"] > r["latency_ms"]
    assert r["speedup_factor"] == pytest.approx(r["reference_latency_ms"] / r["latency_ms"])
    assert r["checked_tokens"] == 8 and r["max_abs_error"] < 0.02


def test_runner_flags_a_planted_wrong_output():
    rl = _rl()
    d = dict(config_inputs(0))
    note("[gpu] run_local with a planted wrong output")

    def tamper(out):
        out[3, 1234] = out[3, 1234].float() + 0.75

    r = rl.run_workload(d, warmup=1, iterations=2, trials=1, cpu_runs=0, tamper=tamper)
    note("[gpu] " + rl.format_result("decode_t8 (tampered)", r))
    assert r["status"] == "INCORRECT_NUMERICAL", r
