"""Compile the gfx950 HIP sources of this directory into ``libmoe_mi355.so``.

Usage: ``python build.py [--jobs N] [--stamps]``.  Each ``csrc/*.hip`` file is compiled
to an object (in parallel), then linked into ``libmoe_mi355.so`` next to this file, where
``kernel.py`` loads it.  hipcc cross-compiles for gfx950 without a GPU.  ``--stamps``
builds ``libmoe_mi355_stamps.so`` instead: the same library with the decode chain's
in-kernel timeline stamps compiled in (``csrc/stamps.h``, read by ``stamp_timeline.py``).

Several processes may build at once (harness workers that each load the solution on
first use): a build holds an exclusive ``fcntl`` lock on ``libmoe_mi355.so.lock`` next
to the library, compiles and links inside a private temporary directory, and installs
the result with one atomic ``os.replace``, so no process ever loads a half-written
library or links another process's objects.

The library carries a hash of the sources it was built from (``csrc/*.hip``,
``csrc/*.h`` and the C-ABI header) in its version string, ``moe_mi355_version()``.
``ensure_built`` builds when the library is missing or its hash differs from the
sources next to it (an edited kernel is never tested with the old binary), re-checking
under the lock.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import contextlib
import fcntl
import hashlib
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libmoe_mi355.so")
STAMPS_LIB = os.path.join(HERE, "libmoe_mi355_stamps.so")
LOCK = LIB + ".lock"
# the C-ABI header: include/ next to this file in a packed solution, else the repo's
INCLUDE = os.path.join(HERE, "include") if os.path.isdir(os.path.join(HERE, "include")) \
    else os.path.join(REPO, "include")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC", "-fvisibility=hidden",
    "-fno-gpu-flush-denormals-to-zero",
    # packed fp32 VALU ops are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


# prefix of the source hash inside the library's version string (capi.hip)
HASH_TAG = b"moe_mi355 src "


def source_hash() -> str:
    """Hash of everything the library is compiled from: every csrc/*.hip and csrc/*.h
    file (name and bytes, in name order), then the C-ABI header."""
    h = hashlib.sha256()
    names = sorted(f for f in os.listdir(CSRC) if f.endswith((".hip", ".h")))
    for path in [os.path.join(CSRC, f) for f in names] + [os.path.join(INCLUDE, "moe_mi355.h")]:
        h.update(os.path.basename(path).encode() + b"\0")
        with open(path, "rb") as f:
            h.update(f.read())
        h.update(b"\0")
    return h.hexdigest()[:16]


def library_hash(path: str = LIB):
    """The source hash a built library carries (from its version string), or None."""
    if not os.path.exists(path):
        return None
    with open(path, "rb") as f:
        data = f.read()
    i = data.find(HASH_TAG)
    if i < 0:
        return None
    return data[i + len(HASH_TAG):i + len(HASH_TAG) + 16].decode("ascii", "replace")


def is_current(path: str = LIB) -> bool:
    """The library exists and was built from the sources next to it."""
    return library_hash(path) == source_hash()


def _compile(src: str, outdir: str, src_hash: str, stamps: bool = False) -> str:
    obj = os.path.join(outdir, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, f'-DMOE_MI355_SRC_HASH="{src_hash}"',
           *(["-DMOE_MI355_STAMPS"] if stamps else []), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    noise = "is not a recognized feature for this target"
    msg = "\n".join(l for l in r.stderr.splitlines() if noise not in l).strip()
    if msg:
        print(msg, file=sys.stderr)
    return obj


@contextlib.contextmanager
def _build_lock():
    fd = os.open(LOCK, os.O_RDWR | os.O_CREAT, 0o644)
    try:
        fcntl.flock(fd, fcntl.LOCK_EX)
        yield
    finally:
        fcntl.flock(fd, fcntl.LOCK_UN)
        os.close(fd)


def _build_locked(jobs: int, verbose: bool, stamps: bool = False) -> str:
    out = STAMPS_LIB if stamps else LIB
    work = tempfile.mkdtemp(prefix="_build.", dir=HERE)
    try:
        srcs = sources()
        src_hash = source_hash()
        with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs)))) as ex:
            objs = list(ex.map(lambda s: _compile(s, work, src_hash, stamps), srcs))
        tmp = os.path.join(work, os.path.basename(out))
        cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
        os.replace(tmp, out)
    finally:
        shutil.rmtree(work, ignore_errors=True)
    if verbose:
        print(f"built {out}")
    return out


def build(jobs: int = 8, verbose: bool = True, stamps: bool = False) -> str:
    """Compile and link the library (always, even when one is present); with stamps,
    the timeline-stamped build, libmoe_mi355_stamps.so."""
    with _build_lock():
        return _build_locked(jobs, verbose, stamps)


def ensure_built(jobs: int = 8, verbose: bool = False, stamps: bool = False) -> str:
    """Build the library if it is missing or was built from other sources (the first
    use of a packed solution, or a kernel edited since the last build)."""
    out = STAMPS_LIB if stamps else LIB
    if is_current(out):
        return out
    with _build_lock():
        if is_current(out):           # another process built it while this one waited
            return out
        return _build_locked(jobs, verbose, stamps)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=8)
    ap.add_argument("--stamps", action="store_true",
                    help="build libmoe_mi355_stamps.so (in-kernel timeline stamps) instead")
    a = ap.parse_args()
    build(a.jobs, stamps=a.stamps)
