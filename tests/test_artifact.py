"""The `.qw38` reader and Model::upload (tests/cpp/qw38_artifact_test, built by
__graft_entry__.build()): SHA-256 known-answer vectors, record round trip,
alias resolution and typed rejections on the CPU; on the GPU, the uploaded
Q4_K 0x020D tensor equals the file bytes and every uploaded weight (0x020D as
stored, GGML-order Q4_K repacked to 0x0240 / 0x020D, GGML-order Q6_K
repacked to 0x0241) projects integer activations exactly."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "qw38_artifact_test")


def _run(args, timeout):
    if not os.path.exists(BIN):
        pytest.fail("tests/cpp/qw38_artifact_test missing: run __graft_entry__.build()")
    r = subprocess.run([BIN, *args], capture_output=True, text=True, timeout=timeout)
    print(r.stdout[-4000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "0 failure(s)" in r.stdout
    return r.stdout


def test_reader_on_host():
    out = _run(["--host"], 120)
    assert "SHA-256 of abc" in out and "manifest bit flip rejected" in out


@pytest.mark.gpu
def test_model_upload_on_gpu(torch_gpu):
    out = _run([], 240)
    assert "repacked to 0x0241" in out
