"""The C ABI's host code under AddressSanitizer and UBSan: libmoe_mi355x.so is rebuilt from its sources into a
temporary directory with the sanitizers on the host side of every compile (-Xarch_host; the device code is built
as usual), and tests/host_fuzz_abi.cpp calls every entry point with seeded random and edge-case sizes. It checks:
- no sanitizer report;
- statuses in range, with a message on failure;
- InferShape outputs as the reference's rules (op_host/moe_ops.cpp:181-214, 363-386, 495-515);
- plans that agree with the workspace query;
- a workspace never smaller than the buffers it holds, so no size product overflows into an under-sized buffer;
- launch calls that reject null pointers and a workspace one byte short before launching anything.
The reference's own host checks are GRAPH_FAILED returns (op_host/moe_ops.cpp:71-90, 241-258); this covers the
sizes it never checks. CPU only: skipped where a GPU is present (the GPU suite runs there)."""
from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess

import pytest

from conftest import ROOT

PKG = ROOT / "implementing-moe-architecture-operators-on-cann-platform_amd"
SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined", "-Xarch_host",
       "-fno-omit-frame-pointer"]


def _hipcc() -> str | None:
    return shutil.which("hipcc") or (("/opt/rocm/bin/hipcc") if os.path.exists("/opt/rocm/bin/hipcc") else None)


@pytest.mark.skipif(_hipcc() is None, reason="hipcc is not installed")
@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="CPU-only test: a GPU is present")
def test_abi_host_code_under_asan_and_ubsan(tmp_path: pathlib.Path):
    hipcc = _hipcc()
    flags = ["--offload-arch=gfx950", "-O2", "-g", "-std=c++17", "-fPIC", "-Xclang", "-target-feature", "-Xclang",
             "-packed-fp32-ops", *SAN, f"-I{ROOT / 'include'}", f"-I{PKG / 'csrc'}"]
    sources = sorted((PKG / "csrc").glob("*.hip")) + sorted((PKG / "csrc").glob("*.cpp"))

    def compile_one(src: pathlib.Path) -> pathlib.Path:
        obj = tmp_path / (src.name + ".o")
        lang = ["-x", "hip"] if src.suffix == ".hip" else []
        res = subprocess.run([hipcc, *flags, *lang, "-c", str(src), "-o", str(obj)], capture_output=True, text=True)
        assert res.returncode == 0, res.stderr[-3000:]
        return obj

    with concurrent.futures.ThreadPoolExecutor(max_workers=8) as pool:
        objs = list(pool.map(compile_one, sources))
    lib = tmp_path / "libmoe_san.so"
    res = subprocess.run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *SAN[:4], *map(str, objs), "-o", str(lib)],
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-3000:]
    exe = tmp_path / "host_fuzz_abi"
    res = subprocess.run([hipcc, "-O1", "-g", "-std=c++17", *SAN, f"-I{ROOT / 'include'}",
                          str(ROOT / "tests" / "host_fuzz_abi.cpp"), f"-L{tmp_path}", "-lmoe_san",
                          f"-Wl,-rpath,{tmp_path}", "-o", str(exe)], capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-3000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    res = subprocess.run([str(exe), "200000"], capture_output=True, text=True, env=env, timeout=300)
    print(res.stdout[-2000:])
    assert res.returncode == 0, (res.stdout[-3000:], res.stderr[-3000:])
    assert res.stdout.strip().endswith("ok")
