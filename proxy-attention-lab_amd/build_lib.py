"""Build libpal_hip.so (gfx950) in-tree with hipcc.

Usage: python proxy-attention-lab_amd/build_lib.py [--jobs N] [--debug] [--debug-checks]

Every csrc/*.hip and csrc/*.cpp file is compiled to an object under
_build/ (in parallel) and linked into proxy_attention_lab/libpal_hip.so, the
library the Python layer loads.  All device code is built for gfx950 only,
with packed-FP32 instruction selection disabled.  --debug-checks builds the
bounds-checked variant (PAL_DEBUG_CHECKS: kernels record out-of-range page
ids, lengths and fill destinations, read back by pal_debug_flags) as
proxy_attention_lab/libpal_hip_debug.so, from objects under _build_debug/;
set PAL_HIP_LIB to its path to run the package on it.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
CSRC = PKG_ROOT / "csrc"
BUILD = PKG_ROOT / "_build"
OUT = PKG_ROOT / "proxy_attention_lab" / "libpal_hip.so"
BUILD_DEBUG = PKG_ROOT / "_build_debug"
OUT_DEBUG = PKG_ROOT / "proxy_attention_lab" / "libpal_hip_debug.so"
REPO_INCLUDE = PKG_ROOT.parent / "include"

ARCH = "gfx950"
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    "-I",
    str(CSRC),
    "-I",
    str(REPO_INCLUDE),
]
# Keep the compiler from selecting packed-FP32 (v_pk_*_f32) instructions.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
# Keep MFMA accumulators in ordinary VGPRs: the kernels rescale them with VALU
# ops, and AGPR accumulators would cost a copy in and out around every rescale.
DEVICE_FLAGS += ["-mllvm", "-amdgpu-mfma-vgpr-form"]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; ROCm is required to build libpal_hip.so")
    return exe


def _compile(src: Path, debug: bool, checks: bool = False) -> Path:
    obj = (BUILD_DEBUG if checks else BUILD) / (src.name + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    if src.suffix == ".hip":
        cmd[1:1] = ["-x", "hip"]
        cmd += DEVICE_FLAGS
    if debug:
        cmd += ["-g"]
    if checks:
        cmd += ["-DPAL_DEBUG_CHECKS"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    # hipcc's host pass warns that it does not know the packed-fp32 feature; drop that noise.
    noise = "packed-fp32-ops' is not a recognized feature"
    warn = "\n".join(ln for ln in res.stderr.splitlines() if noise not in ln and ln.strip())
    if warn:
        print(warn, file=sys.stderr)
    return obj


def build(jobs: int | None = None, debug: bool = False, checks: bool = False) -> Path:
    (BUILD_DEBUG if checks else BUILD).mkdir(exist_ok=True)
    out = OUT_DEBUG if checks else OUT
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    if not sources:
        raise RuntimeError(f"no sources in {CSRC}")
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 4)), 16)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, debug, checks), sources))
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    return out


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--debug", action="store_true", help="device and host debug info (-g)")
    ap.add_argument("--debug-checks", action="store_true", help="the bounds-checked variant (libpal_hip_debug.so)")
    args = ap.parse_args()
    out = build(args.jobs, args.debug, args.debug_checks)
    print(f"built {out}")


if __name__ == "__main__":
    main()
