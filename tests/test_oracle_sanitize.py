"""The C oracle (oracle/moe_oracle.c) built with AddressSanitizer and
UndefinedBehaviorSanitizer (gcc, host code only) runs routing and dispatch on edge
cases -- no tokens, one token, ties, saturated and NaN logits, a hot bias, offsets
past the expert range, every tile height -- without a sanitizer report, and gives the
same results bit for bit as the normal build the other tests use."""
import os
import shutil
import subprocess

import numpy as np
import pytest

from conftest import ORACLE_DIR, REPO, oracle

DRIVER = os.path.join(REPO, "tests", "oracle_sanitize_driver.c")


@pytest.fixture(scope="module")
def asan_driver(tmp_path_factory):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    d = tmp_path_factory.mktemp("asan")
    exe = str(d / "oracle_asan")
    cmd = ["gcc", "-std=c11", "-O1", "-g", "-ffp-contract=off", "-fno-fast-math",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer",
           os.path.join(ORACLE_DIR, "moe_oracle.c"), DRIVER, "-o", exe, "-lm"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return exe


def _bf16_bits(x):
    return (np.asarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def _cases():
    rng = np.random.default_rng(20260505)
    yield "empty", np.zeros((0, 256), np.float32), np.zeros(256, np.uint16), 0, 16
    yield "one token", rng.standard_normal((1, 256)).astype(np.float32), _bf16_bits(rng.standard_normal(256) * 0.1), 0, 16
    yield "all equal", np.zeros((9, 256), np.float32), np.zeros(256, np.uint16), 0, 32
    hot = rng.standard_normal(256) * 0.1
    hot[[3, 11, 19, 27]] += 3.0
    yield "hot bias", rng.standard_normal((67, 256)).astype(np.float32), _bf16_bits(hot), 0, 64
    big = rng.standard_normal((33, 256)).astype(np.float32) * 80
    big[0, :8] = np.inf
    big[1, :8] = -np.inf
    big[2, 5] = np.nan
    yield "saturated and NaN", big, _bf16_bits(rng.standard_normal(256) * 0.1), 224, 128
    yield "offset past the range", rng.standard_normal((40, 256)).astype(np.float32), _bf16_bits(np.zeros(256)), 250, 256
    yield "negative offset", rng.standard_normal((40, 256)).astype(np.float32), _bf16_bits(np.zeros(256)), -16, 16
    yield "many tokens", rng.standard_normal((1100, 256)).astype(np.float32), _bf16_bits(rng.standard_normal(256) * 0.1), 64, 16


@pytest.mark.parametrize("case", list(_cases()), ids=lambda c: c[0])
def test_sanitized_oracle_matches_normal_build(asan_driver, tmp_path, case):
    name, logits, bias, offset, tm = case
    T = logits.shape[0]
    factor = 2.5
    inp = tmp_path / "in.bin"
    with open(inp, "wb") as f:
        f.write(np.int32(T).tobytes() + np.int64(offset).tobytes() + np.int32(tm).tobytes()
                + np.float64(factor).tobytes())
        f.write(np.ascontiguousarray(logits, np.float32).tobytes())
        f.write(np.ascontiguousarray(bias, np.uint16).tobytes())
    out = tmp_path / "out.bin"
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([asan_driver, str(inp), str(out)], capture_output=True, text=True, env=env)
    assert r.returncode == 0, r.stderr
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr

    o = oracle()
    ids, w = o.route(logits, bias.view(np.uint16), factor)
    ref = o.dispatch(ids, w, offset, tm)
    buf = open(out, "rb").read()
    pos = 0

    def take(n, dt):
        nonlocal pos
        a = np.frombuffer(buf, dt, count=n, offset=pos)
        pos += n * np.dtype(dt).itemsize
        return a

    R = T * 8
    assert np.array_equal(take(R, np.int32).reshape(T, 8), ids)
    assert np.array_equal(take(R, np.uint32), w.reshape(-1).view(np.uint32))
    exp_off = take(33, np.int32)
    assert np.array_equal(exp_off, ref["exp_off"])
    nt = int(take(1, np.int32)[0])
    na = int(exp_off[32])
    assert np.array_equal(take(na, np.int32), ref["sorted_tok"])
    assert np.array_equal(take(na, np.uint32), ref["sorted_w"].view(np.uint32))
    assert np.array_equal(take(R, np.int32).reshape(T, 8), ref["inv"])
    assert np.array_equal(take(nt * 4, np.int32).reshape(nt, 4), ref["tiles"])
    assert pos == len(buf)
