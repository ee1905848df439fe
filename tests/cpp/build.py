"""Builds tests/cpp/qw38_api_test, the C++ test of the qw38::cuda interfaces,
against the in-tree libqw38_hip.so (run by tests/test_gpu_cpp_api.py)."""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
OUT = os.path.join(HERE, "qw38_api_test")


def build() -> str:
    cmd = [HIPCC, "-x", "hip", "--offload-arch=gfx950", "-O2", "-std=c++20",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-Wno-unused-command-line-argument",
           "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "qw38_amd", "cpp"),
           os.path.join(HERE, "qw38_api_test.cpp"), "-o", OUT + ".tmp",
           "-L", os.path.join(ROOT, "qw38_amd"), "-lqw38_hip",
           "-Wl,-rpath,$ORIGIN/../../qw38_amd"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"C++ API test build failed:\n{r.stderr}")
    os.replace(OUT + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    print("built", build())
    sys.exit(0)
