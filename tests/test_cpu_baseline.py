"""The CPU baseline that bench.py times (oracle/cpu_baseline.c, built with
-O3 -march=native) computes the same contraction as the oracle: Q4_K and
Q6_K straight from the packed GGML blocks, within the north-star tolerance of
the oracle's float64 result."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

import oracle
from _fix import normal, outlier_rows

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def cpub(tmp_path_factory):
    so = str(tmp_path_factory.mktemp("cpub") / "libcpu_baseline.so")
    subprocess.run(["gcc", "-O3", "-march=native", "-fopenmp", "-fPIC", "-shared", "-o", so,
                    os.path.join(ROOT, "oracle", "cpu_baseline.c")], check=True)
    L = C.CDLL(so)
    V, U, I = C.c_void_p, C.c_uint32, C.c_int
    L.cpub_q4k.argtypes = [V, U, U, V, V, V, U, V, I]
    L.cpub_q6k.argtypes = [V, U, U, V, V, U, V, I]
    return L


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


@pytest.mark.parametrize("m", [1, 3, 8])
def test_cpu_baseline_q4k_matches_oracle(cpub, m):
    n, k = 136, 1024
    w = oracle.quantize_q4k(normal((n, k), 3, 0.02))
    x = oracle.fp32_to_bf16(outlier_rows(m, k, 4))
    q = oracle.pack_q8(x, m, k)
    ref, _, _ = oracle.q4k_q8_contract(w, q)
    blocks = np.ascontiguousarray(w.ggml())
    out = np.zeros((m, n), np.float32)
    assert cpub.cpub_q4k(_p(blocks), n, k, _p(q.codes), _p(q.scales), _p(q.sums), m, _p(out), 2) == 0
    ok, ma, mr = oracle.parity_ok(out, ref)
    assert ok, (ma, mr)


@pytest.mark.parametrize("m", [1, 8])
def test_cpu_baseline_q6k_matches_oracle(cpub, m):
    n, k = 72, 2048
    w = oracle.quantize_q6k(normal((n, k), 5, 0.02))
    x = oracle.fp32_to_bf16(normal((m, k), 6))
    q = oracle.pack_q8(x, m, k)
    ref, _, _ = oracle.q6k_q8_contract(w, q)
    blocks = np.ascontiguousarray(w.ggml())
    out = np.zeros((m, n), np.float32)
    assert cpub.cpub_q6k(_p(blocks), n, k, _p(q.codes), _p(q.scales), m, _p(out), 2) == 0
    ok, ma, mr = oracle.parity_ok(out, ref)
    assert ok, (ma, mr)
