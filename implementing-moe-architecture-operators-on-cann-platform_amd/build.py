"""Build libmoe_mi355x.so (gfx950) in place: every csrc/*.hip and csrc/*.cpp through hipcc, then one link.

Run as a script (``python build.py``) or through ``__graft_entry__.build()``. Always recompiles: this is the
"does it build" check, and a stale object must never hide a broken source.
"""
from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

PKG_DIR = pathlib.Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
INCLUDE = PKG_DIR.parent / "include"
BUILD_DIR = CSRC / "_build"
LIB_NAME = "libmoe_mi355x.so"
ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU ops for plain float code.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found; the MI355X library cannot be built")
    return exe


def _compile(src: pathlib.Path) -> pathlib.Path:
    obj = BUILD_DIR / (src.name + ".o")
    lang = ["-x", "hip"] if src.suffix == ".hip" else []
    cmd = [hipcc(), *COMMON_FLAGS, *lang, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def build_library(verbose: bool = False) -> pathlib.Path:
    """Compile and link the library; returns its path. Raises RuntimeError on any failure."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        objs = list(pool.map(_compile, sources))
    out = PKG_DIR / LIB_NAME
    tmp = PKG_DIR / (LIB_NAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out} from {len(sources)} sources")
    return out


if __name__ == "__main__":
    try:
        build_library(verbose=True)
    except RuntimeError as exc:  # pragma: no cover - command-line use
        print(exc, file=sys.stderr)
        sys.exit(1)
