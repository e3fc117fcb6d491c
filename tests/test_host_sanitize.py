"""The library's host logic (csrc/host_plan.h, used by capi.hip: the kernel plan, the
workspace layout, the argument checks of moe_mi355_forward, the offset clamp) built
with g++ for the host, once plainly and once under AddressSanitizer and
UndefinedBehaviorSanitizer, and driven by tests/host_sanitize_driver.cpp over edge-case
token counts (negative, 0, every plan boundary, the maximum and one past it,
INT32_MIN/MAX), every flag combination (all forced GEMM pairs, unknown bits) and NULL
or misaligned pointers.  The driver checks the invariants itself; both builds must
exit 0, print identical results, and the sanitized one must report nothing."""
import os
import shutil
import subprocess

import pytest

from conftest import PKG_DIR, REPO

DRIVER = os.path.join(REPO, "tests", "host_sanitize_driver.cpp")


def _build(tmp, name, extra):
    exe = str(tmp / name)
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-Wall", "-Werror",
           f"-I{os.path.join(PKG_DIR, 'csrc')}", f"-I{os.path.join(REPO, 'include')}",
           *extra, DRIVER, "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


@pytest.fixture(scope="module")
def drivers(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    d = tmp_path_factory.mktemp("host_asan")
    plain = _build(d, "host_plain", [])
    asan = _build(d, "host_asan", ["-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                                   "-fno-omit-frame-pointer"])
    return plain, asan


def _run(exe):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    return subprocess.run([exe], capture_output=True, text=True, env=env, timeout=300)


def test_host_logic_sanitized_matches_plain_build(drivers):
    plain, asan = drivers
    a, b = _run(plain), _run(asan)
    assert a.returncode == 0, a.stdout[-2000:] + a.stderr
    assert b.returncode == 0, b.stdout[-2000:] + b.stderr
    assert "runtime error" not in b.stderr and "AddressSanitizer" not in b.stderr, b.stderr
    assert a.stdout == b.stdout
    assert a.stdout.rstrip().endswith("OK (0 failures)")


def test_host_logic_default_plans(drivers):
    """The default plan at the boundaries named in capi.hip's plan table."""
    out = _run(drivers[0]).stdout
    plans = {int(l.split()[1]): l for l in out.splitlines() if l.startswith("T ") and "plan" in l}
    def g(T):
        f = plans[T].split()
        return int(f[4]), int(f[6])
    assert g(1) == (9, 6) and g(4) == (9, 6) and g(5) == (9, 6) and g(8) == (9, 6)
    assert g(9) == (5, 6) and g(22) == (5, 6)
    assert g(23) == (5, 1) and g(32) == (5, 1) and g(33) == (5, 1) and g(64) == (5, 1)
    assert g(65) == (1, 1) and g(88) == (1, 1)
    assert g(89) == (2, 3) and g(199) == (2, 3)
    assert g(200) == (8, 7) and g(559) == (8, 7)
    assert g(560) == (8, 5) and g(960) == (8, 5)
    assert g(961) == (8, 5) and g(1344) == (8, 5)
    assert g(1345) == (4, 5) and g(1 << 19) == (4, 5)
    assert "T -1 status -2" in out and f"T {(1 << 19) + 1} status -2" in out
