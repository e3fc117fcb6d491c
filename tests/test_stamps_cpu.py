"""The in-kernel timeline stamps (csrc/stamps.h) are compiled in only on request: the
product library exports no stamp reader, and a source compiled with -DMOE_MI355_STAMPS
exports its table's reader (what stamp_timeline.py loads from libmoe_mi355_stamps.so)."""
import os
import shutil
import subprocess

import pytest

from conftest import PKG_DIR, pkg


def _exports(path):
    r = subprocess.run(["nm", "-D" if path.endswith(".so") else "-g", path],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return {l.split()[-1] for l in r.stdout.splitlines() if l.strip()}


def test_product_library_has_no_stamps():
    if shutil.which("nm") is None:
        pytest.skip("nm not available")
    lib = pkg("kernel").library_path()
    if not os.path.exists(lib):
        pytest.skip("library not built")
    assert not [s for s in _exports(lib) if "stamps" in s]


def test_stamped_source_exports_its_reader(tmp_path):
    if shutil.which("nm") is None or shutil.which("hipcc") is None:
        pytest.skip("hipcc / nm not available")
    b = pkg("build")
    obj = str(tmp_path / "route.o")
    cmd = [b.HIPCC, *b.FLAGS, "-DMOE_MI355_STAMPS", "-c", os.path.join(PKG_DIR, "csrc", "route.hip"),
           "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert "moe_mi355_stamps_route" in _exports(obj)
