"""Builds the gfx950 library ``qw38_amd/libqw38_hip.so`` in-tree with hipcc.

Sources: every ``*.hip`` and ``*.cpp`` under ``qw38_amd/csrc`` (kernels and the
C-ABI) and ``qw38_amd/cpp/src`` (the qw38::cuda C++ API mirror). Objects go to
``qw38_amd/_build``; the shared library next to the package so it travels with
the tree. Always recompiles (the build check must compile every time).
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libqw38_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

ARCH = "gfx950"
COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC",
    # Exact FP semantics: every fused multiply-add in the kernels is written
    # explicitly; no contraction, no fast-math; IEEE div/sqrt (HIP default).
    "-ffp-contract=off",
    # Never emit packed FP32 VALU ops (v_pk_{add,mul,fma}_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    "-I", os.path.join(ROOT, "include"),
    "-I", os.path.join(PKG, "csrc"),
    "-I", os.path.join(PKG, "cpp"),
]


# Per-source extra hipcc flags. The batched decode kernel keeps its MFMA results
# in VGPRs (no v_accvgpr_read per result); the 512-register MMQ tiles keep the
# compiler's AGPR choice.
EXTRA = {
    "q4k_decode_mfma.hip": ["-mllvm", "--amdgpu-mfma-vgpr-form"],
}


def sources():
    srcs = sorted(glob.glob(os.path.join(PKG, "csrc", "*.hip")))
    srcs += sorted(glob.glob(os.path.join(PKG, "csrc", "*.cpp")))
    srcs += sorted(glob.glob(os.path.join(PKG, "cpp", "src", "*.cpp")))
    return srcs


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, *COMMON, *EXTRA.get(os.path.basename(src), []), "-c", src, "-o", obj]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    # roctx (rocprofiler-sdk) for the opt-in operation ranges
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs,
           "-L/opt/rocm/lib", "-Wl,-rpath,/opt/rocm/lib", "-lrocprofiler-sdk-roctx"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
