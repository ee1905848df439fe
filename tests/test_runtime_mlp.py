"""Runtime MLP callers over an uploaded `.qw38` model
(tests/cpp/qw38_runtime_test, built by __graft_entry__.build()): the bound
plan's Q8 route equals a direct q4k_q8_mlp bitwise for a 0x020D layer and a
GGML-order (repacked) layer, the BF16 route agrees within the Q8 budget, a
captured decode token equals the eager submission on every replay, a
nonfinite activation is reported at completion and poisons the session, and
prefill chunks equal their direct calls."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "qw38_runtime_test")


def test_runtime_test_binary_built():
    if not os.path.exists(BIN):
        pytest.fail("tests/cpp/qw38_runtime_test missing: run __graft_entry__.build()")
    r = subprocess.run([BIN, "--list"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "runtime_mlp" in r.stdout


@pytest.mark.gpu
def test_runtime_mlp_on_gpu(torch_gpu):
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=300)
    print(r.stdout[-4000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-2000:]
    assert "0 failure(s)" in r.stdout
    assert "captured decode token equals" in r.stdout
