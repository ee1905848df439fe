"""Runs the C++ test of the qw38::cuda interfaces (tests/cpp/qw38_api_test,
built by __graft_entry__.build()) on the GPU: fixtures and closed forms of
tests/q4k_q8_test.cpp and tests/decode_mmv_unit_test.cpp restated in C++,
the PrefillEngine contract, runtime handles and graph replays."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "qw38_api_test")


def test_binary_lists_its_checks():
    """CPU: the test program is built and links libqw38_hip (no device use)."""
    if not os.path.exists(BIN):
        pytest.fail("tests/cpp/qw38_api_test missing: run __graft_entry__.build()")
    r = subprocess.run([BIN, "--list"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "decode_onehot" in r.stdout


@pytest.mark.gpu
def test_cpp_api_on_gpu(torch_gpu):
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=240)
    print(r.stdout[-4000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "0 failure(s)" in r.stdout
