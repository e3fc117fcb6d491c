"""Packing for the harness (pack_solution.py, the counterpart of the reference's
scripts/pack_solution.py:34-91) and the builder's entry-point checks (README.md:227-257):

* solution.json has the README's layout, names the definition of config.toml, and its
  sources reproduce the package's files byte for byte;
* the unpacked tree is self-contained: its build.py finds every HIP source and the
  C-ABI header inside the tree, and its entry point passes the DPS check;
* planted entry points (one parameter too many, variadic arguments, a missing
  function) are rejected with the harness's messages.
"""
import importlib.util
import json
import os

import pytest

from conftest import REPO

PKG = os.path.join(REPO, "flash-infer-bench-starter-kit_amd")


def _load(name, path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="module")
def packer():
    return _load("pack_solution_under_test", os.path.join(PKG, "pack_solution.py"))


def test_pack_writes_the_readme_layout(packer, tmp_path):
    out = packer.pack_solution(str(tmp_path / "solution.json"))
    doc = json.load(open(out))
    assert doc["definition"] == "moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048"
    assert set(doc) >= {"name", "definition", "author", "spec", "sources"}
    spec = doc["spec"]
    assert spec["language"] == "python" and spec["entry_point"] == "kernel.py::kernel"
    assert spec["destination_passing_style"] is True and spec["dependencies"] == []
    paths = {s["path"]: s["content"] for s in doc["sources"]}
    assert paths["kernel.py"] == open(os.path.join(PKG, "kernel.py")).read()
    hips = sorted(f for f in os.listdir(os.path.join(PKG, "csrc")) if f.endswith(".hip"))
    for f in hips:
        assert paths[f"csrc/{f}"] == open(os.path.join(PKG, "csrc", f)).read()
    assert paths["include/moe_mi355.h"] == open(os.path.join(REPO, "include", "moe_mi355.h")).read()


def test_unpacked_tree_builds_from_itself(packer, tmp_path):
    out = packer.pack_solution(str(tmp_path / "solution.json"))
    dest = tmp_path / "unpacked"
    packer.unpack_solution(out, str(dest))
    b = _load("unpacked_build", str(dest / "build.py"))
    assert b.INCLUDE == str(dest / "include")
    assert os.path.exists(os.path.join(b.INCLUDE, "moe_mi355.h"))
    got = sorted(os.path.basename(p) for p in b.sources())
    want = sorted(f for f in os.listdir(os.path.join(PKG, "csrc")) if f.endswith(".hip"))
    assert got == want
    packer.check_entry_point("kernel.py::kernel", True, root=str(dest))


@pytest.mark.parametrize("src,msg", [
    ("def kernel(a, b, c, d, e, f, g, h, i, j, k, l):\n    pass\n", "expected 11 parameters, but got 12"),
    ("def kernel(a, *args):\n    pass\n", "variadic"),
    ("def kernel(a, b, c, d, e, f, g, h, i, j, k, **kw):\n    pass\n", "variadic"),
    ("def other(a):\n    pass\n", "no callable"),
])
def test_builder_check_rejects_planted_entry_points(packer, tmp_path, src, msg):
    (tmp_path / "kernel.py").write_text(src)
    with pytest.raises(ValueError, match=msg):
        packer.check_entry_point("kernel.py::kernel", True, root=str(tmp_path))


def test_value_returning_entry_allows_other_counts(packer, tmp_path):
    (tmp_path / "kernel.py").write_text("def kernel(a, b):\n    return a\n")
    packer.check_entry_point("kernel.py::kernel", False, root=str(tmp_path))


def test_unpacked_solution_builds_on_first_use_from_two_processes(packer, tmp_path):
    """A packed solution carries no library: the first call of kernel.py builds it, as
    the reference's kernel.py JIT-compiles on first use (kernel.py:57-92).  Two worker
    processes that load the solution at the same moment both end up with a working
    library: the build runs under a file lock in a private directory and is installed
    with one atomic rename, so neither loads a half-written file."""
    import subprocess
    import sys
    out = packer.pack_solution(str(tmp_path / "solution.json"))
    dest = tmp_path / "unpacked"
    packer.unpack_solution(out, str(dest))
    assert not (dest / "libmoe_mi355.so").exists()
    code = ("import importlib.util, sys\n"
            "spec = importlib.util.spec_from_file_location('k', sys.argv[1])\n"
            "m = importlib.util.module_from_spec(spec); spec.loader.exec_module(m)\n"
            "lib = m._build_extension()\n"
            "print(lib.moe_mi355_version().decode(), lib.moe_mi355_workspace_bytes(64))\n")
    procs = [subprocess.Popen([sys.executable, "-c", code, str(dest / "kernel.py")],
                              stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)
             for _ in range(2)]
    outs = [p.communicate(timeout=600) for p in procs]
    for p, (o, e) in zip(procs, outs):
        assert p.returncode == 0, e
        assert o.startswith("moe_mi355"), o
    assert outs[0][0] == outs[1][0]
    assert (dest / "libmoe_mi355.so").exists()
    assert not [f for f in os.listdir(dest) if f.startswith("_build.")]   # private dirs removed
