"""The loader never runs a library built from other sources (CPU only).

The library's version string carries a hash of the sources it was compiled from
(build.py ``source_hash``: csrc/*.hip, csrc/*.h and the C-ABI header).  In a copy of the
package this test checks that the built library counts as current for identical
sources, that editing one source file makes it stale, and that loading the package
(``kernel._build_extension``) then rebuilds it with hipcc before loading, so the
loaded library carries the new hash."""
import importlib.util
import os
import shutil

import pytest

from conftest import PKG_DIR, REPO


def _load(name, path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture()
def pkg_copy(tmp_path):
    src_lib = os.path.join(PKG_DIR, "libmoe_mi355.so")
    if not os.path.exists(src_lib):
        pytest.skip("library not built (run __graft_entry__.build() first)")
    b0 = _load("build_of_repo", os.path.join(PKG_DIR, "build.py"))
    if not b0.is_current():
        pytest.skip("the repository's library is stale: build it first")
    if shutil.which(b0.HIPCC) is None and not os.path.exists(b0.HIPCC):
        pytest.skip("hipcc not available")
    dest = tmp_path / "pkg"
    shutil.copytree(os.path.join(PKG_DIR, "csrc"), dest / "csrc")
    os.makedirs(dest / "include")
    shutil.copy(os.path.join(REPO, "include", "moe_mi355.h"), dest / "include")
    for f in ("kernel.py", "build.py", "libmoe_mi355.so"):
        shutil.copy(os.path.join(PKG_DIR, f), dest / f)
    return dest


def test_edited_source_triggers_a_rebuild(pkg_copy):
    b = _load("build_of_copy", str(pkg_copy / "build.py"))
    old = b.source_hash()
    assert b.library_hash() == old and b.is_current()

    with open(pkg_copy / "csrc" / "moe_shape.h", "a") as f:
        f.write("// an edit\n")
    assert b.source_hash() != old
    assert not b.is_current()

    k = _load("kernel_of_copy", str(pkg_copy / "kernel.py"))
    lib = k._build_extension()          # rebuilds before loading
    new = b.source_hash()
    assert b.library_hash() == new and b.is_current()
    assert lib.moe_mi355_version().decode().endswith(new)
    # a second load of the current library does not build again
    mtime = os.path.getmtime(pkg_copy / "libmoe_mi355.so")
    b.ensure_built()
    assert os.path.getmtime(pkg_copy / "libmoe_mi355.so") == mtime
