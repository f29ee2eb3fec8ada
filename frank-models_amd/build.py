"""Builds libfmoe.so (the gfx950 kernels + C ABI) in-tree with hipcc.

Every ``csrc/*.hip`` and ``csrc/*.cpp`` file is compiled to an object in
``_build/`` (in parallel), then linked into ``libfmoe.so`` next to this file.
``build(force=True)`` recompiles everything; otherwise objects newer than
their source and the headers are reused.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
INCLUDE = PKG_DIR.parent / "include"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libfmoe.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    "-O3",
    "-fPIC",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
    "-Wall",
    "-Wno-unused-function",
    # Packed fp32 ops are kept out of generated code on this platform.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _sources():
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _headers():
    return sorted(list(CSRC.glob("*.h")) + list(INCLUDE.glob("*.h")))


def _compile(src: Path, force: bool) -> Path:
    obj = BUILD_DIR / (src.name + ".o")
    newest_dep = max([src.stat().st_mtime] + [h.stat().st_mtime for h in _headers()])
    if not force and obj.exists() and obj.stat().st_mtime >= newest_dep:
        return obj
    cmd = [HIPCC, *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    if src.suffix == ".hip":
        cmd[1:1] = ["-x", "hip"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(force: bool = True, jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile all sources for gfx950 and link libfmoe.so; returns its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = _sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 2) - 1), 8)
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, force), srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(objs)} objects", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build(force="--force" in sys.argv, verbose=True)
