"""Pack this solution into ``solution.json`` for the FlashInfer-Bench harness.

Mirrors the reference's scripts/pack_solution.py:34-91: config.toml ([solution] name,
definition, author; [build] language, entry_point, destination_passing_style) ->
build spec -> Solution JSON.  The flashinfer_bench package that the reference calls
(``BuildSpec``, ``pack_solution_from_files``) is not available here, so the JSON is
written directly in the layout of the solution example in the reference's README.md
(lines 235-249): ``{name, definition, author, spec: {language, target_hardware,
entry_point, dependencies, destination_passing_style}, sources: [{path, content}]}``.

Before writing, the entry point is checked the way the harness's builder checks it
(README.md:227-257): the function exists, has no variadic parameters, and with
destination passing takes exactly the definition's 10 inputs + 1 output.

Sources: every text file the solution needs to build and run from its own directory
(kernel.py, build.py, the HIP sources and headers, the C-ABI header as
``include/moe_mi355.h``).  The compiled ``libmoe_mi355.so`` is not a source:
kernel.py builds it with hipcc (gfx950) on first use, as the reference's kernel.py
JIT-compiles its extension, or ``python build.py`` builds it ahead of time.

Usage: ``python pack_solution.py [-o solution.json]``.
"""
from __future__ import annotations

import argparse
import importlib.util
import inspect
import json
import os
import sys

try:
    import tomllib
except ImportError:  # Python < 3.11
    import tomli as tomllib

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
DPS_PARAMS = 11   # 10 inputs + 1 output of the definition (kernel.py:95-107)


def load_config(path: str | None = None) -> dict:
    with open(path or os.path.join(HERE, "config.toml"), "rb") as f:
        return tomllib.load(f)


def check_entry_point(entry_point: str, dps: bool, root: str = HERE) -> None:
    """Raise ValueError unless ``file.py::function`` under ``root`` is a valid entry."""
    if "::" not in entry_point:
        raise ValueError(f"entry_point must be 'file.py::function', got {entry_point!r}")
    fname, func = entry_point.split("::", 1)
    path = os.path.join(root, fname)
    if not os.path.exists(path):
        raise ValueError(f"entry point file not found: {path}")
    spec = importlib.util.spec_from_file_location("_packed_entry", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    fn = getattr(mod, func, None)
    if not callable(fn):
        raise ValueError(f"{fname} has no callable {func!r}")
    params = list(inspect.signature(fn).parameters.values())
    if any(p.kind in (p.VAR_POSITIONAL, p.VAR_KEYWORD) for p in params):
        raise ValueError(f"{func}: variadic parameters are not accepted by the builder")
    if dps and len(params) != DPS_PARAMS:
        raise ValueError(f"Destination-passing style callable: expected {DPS_PARAMS} parameters, "
                         f"but got {len(params)}")


def source_files() -> list[tuple[str, str]]:
    """(path inside the solution, absolute path) of every packed file."""
    out = [(f, os.path.join(HERE, f)) for f in ("kernel.py", "build.py", "config.toml")]
    csrc = os.path.join(HERE, "csrc")
    for f in sorted(os.listdir(csrc)):
        if f.endswith((".hip", ".h")):
            out.append((f"csrc/{f}", os.path.join(csrc, f)))
    out.append(("include/moe_mi355.h", os.path.join(REPO, "include", "moe_mi355.h")))
    return out


def pack_solution(output_path: str | None = None, config_path: str | None = None) -> str:
    cfg = load_config(config_path)
    sol, build = cfg["solution"], cfg["build"]
    language = build["language"]
    if language != "python":
        raise ValueError(f"this solution is packed as language 'python', config says {language!r}")
    entry = build["entry_point"]
    dps = bool(build.get("destination_passing_style", True))
    check_entry_point(entry, dps)
    doc = {
        "name": sol["name"],
        "definition": sol["definition"],
        "author": sol["author"],
        "spec": {
            "language": language,
            "target_hardware": list(build.get("target_hardware", ["gfx950"])),
            "entry_point": entry,
            "dependencies": list(build.get("dependencies", [])),
            "destination_passing_style": dps,
        },
        "sources": [{"path": rel, "content": open(p, encoding="utf-8").read()}
                    for rel, p in source_files()],
    }
    output_path = output_path or os.path.join(REPO, "solution.json")
    with open(output_path, "w", encoding="utf-8") as f:
        json.dump(doc, f, indent=2)
    print(f"Solution packed: {output_path}")
    print(f"  Name: {doc['name']}\n  Definition: {doc['definition']}\n  Author: {doc['author']}"
          f"\n  Language: {language}\n  Sources: {len(doc['sources'])} files")
    return output_path


def unpack_solution(path: str, dest: str) -> list[str]:
    """Write the sources of a packed solution under ``dest``; returns their paths."""
    with open(path, encoding="utf-8") as f:
        doc = json.load(f)
    written = []
    for src in doc["sources"]:
        p = os.path.join(dest, src["path"])
        os.makedirs(os.path.dirname(p), exist_ok=True)
        with open(p, "w", encoding="utf-8") as f:
            f.write(src["content"])
        written.append(p)
    return written


def main() -> int:
    ap = argparse.ArgumentParser(description="Pack solution files into solution.json")
    ap.add_argument("-o", "--output", default=None, help="output path (default: ./solution.json)")
    a = ap.parse_args()
    try:
        pack_solution(a.output)
    except Exception as e:   # the reference's script reports and exits 1 the same way
        print(f"Error: {e}", file=sys.stderr)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
