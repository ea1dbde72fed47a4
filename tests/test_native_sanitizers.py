"""The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer.

tests/native/host_abi_driver.cpp is linked with the C-ABI, allocator and
log sources (csrc/pal_abi.cpp, page_pool.cpp, pal_log.cpp), built by g++
with -fsanitize=address,undefined (host code only: the kernel launchers are
stand-ins), and run on the CPU: every validation path, the workspace
layout, random allocate/free/compaction histories and the error strings.
Any sanitizer report, or a failed check, fails the test.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "proxy-attention-lab_amd" / "csrc"
ROCM = Path("/opt/rocm")


@pytest.mark.skipif(shutil.which("g++") is None or not (ROCM / "include" / "hip").exists(),
                    reason="needs g++ and the ROCm headers")
def test_host_abi_under_asan_ubsan(tmp_path):
    exe = tmp_path / "host_abi_driver"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}", f"-I{CSRC}",
           f"-I{ROOT / 'include'}", str(ROOT / "tests" / "native" / "host_abi_driver.cpp"),
           str(CSRC / "pal_abi.cpp"), str(CSRC / "page_pool.cpp"), str(CSRC / "pal_log.cpp"),
           f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}", "-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-4000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1",
               PAL_LOG="1")
    run = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
    assert run.returncode == 0, (run.stdout + run.stderr)[-4000:]
    assert "all checks passed" in run.stdout
    assert "runtime error" not in run.stderr and "AddressSanitizer" not in run.stderr
    assert "[pal] page_pool create" in run.stderr  # PAL_LOG reaches stderr
