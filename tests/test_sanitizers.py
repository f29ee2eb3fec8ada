"""The C ABI's host code under AddressSanitizer + UndefinedBehaviorSanitizer.

capi.cpp is compiled with the sanitizers on its host code only (every
sanitizer flag is preceded by -Xarch_host, so no GPU code is instrumented),
linked with the kernel objects of the in-tree build and a C driver
(tests/native/abi_checks.c) that calls every entry point with invalid
arguments and, on a machine without a GPU, valid ones that must report
FMOE_ERR_NO_DEVICE.  Runs on the CPU only."""

import os
import shutil
import subprocess
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "frank-models_amd"
BUILD = PKG / "_build"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
       "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer"]


@pytest.mark.skipif(torch.cuda.is_available(), reason="the no-device checks need a machine without a GPU")
@pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not available")
def test_abi_host_code_under_asan_ubsan(tmp_path):
    kernels = sorted(p for p in BUILD.glob("*.hip.o"))
    if not kernels:
        pytest.skip("kernel objects missing: run __graft_entry__.build() first")
    inc = ["-I", str(ROOT / "include"), "-I", str(PKG / "csrc")]
    capi = tmp_path / "capi_san.o"
    subprocess.run([HIPCC, "-std=c++17", "-O1", "-g", "-fPIC", f"--offload-arch=gfx950", *SAN, *inc, "-c",
                    str(PKG / "csrc" / "capi.cpp"), "-o", str(capi)], check=True, capture_output=True, text=True)
    exe = tmp_path / "abi_checks"
    subprocess.run([HIPCC, "-O1", "-g", f"--offload-arch=gfx950", *SAN, *inc, "-x", "c",
                    str(ROOT / "tests" / "native" / "abi_checks.c"), "-x", "none", str(capi),
                    *map(str, kernels), "-o", str(exe)], check=True, capture_output=True, text=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1",
               HIP_VISIBLE_DEVICES="")
    assert b"__asan_init" in exe.read_bytes() and b"__ubsan_handle" in exe.read_bytes(), "not instrumented"
    r = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "abi checks ok" in r.stdout
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr
