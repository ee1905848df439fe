"""Builds the C++ tests against the in-tree libqw38_hip.so: tests/cpp/qw38_api_test
(the qw38::cuda interfaces, run by tests/test_gpu_cpp_api.py) and
tests/cpp/qw38_artifact_test (the `.qw38` reader and Model::upload, run by
tests/test_artifact.py)."""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
TESTS = ("qw38_api_test", "qw38_artifact_test", "qw38_runtime_test")


def build_one(name: str) -> str:
    out = os.path.join(HERE, name)
    cmd = [HIPCC, "-x", "hip", "--offload-arch=gfx950", "-O2", "-std=c++20",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-Wno-unused-command-line-argument",
           "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "qw38_amd", "cpp"),
           "-I", os.path.join(ROOT, "oracle"),
           os.path.join(HERE, name + ".cpp"), "-o", out + ".tmp",
           "-L", os.path.join(ROOT, "qw38_amd"), "-lqw38_hip",
           "-Wl,-rpath,$ORIGIN/../../qw38_amd",
           # the oracle (test infrastructure) as the checker of the runtime test
           "-L", os.path.join(ROOT, "oracle"), "-loracle", "-Wl,-rpath,$ORIGIN/../../oracle"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"C++ test build failed for {name}:\n{r.stderr}")
    os.replace(out + ".tmp", out)
    return out


def build() -> list:
    return [build_one(n) for n in TESTS]


if __name__ == "__main__":
    for p in build():
        print("built", p)
    sys.exit(0)
