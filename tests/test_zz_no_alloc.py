"""qw38_q4k_q8_mlp_static (allocation-free Q8 MLP over the library's static
device scratch) against qw38_q4k_q8_mlp with a caller workspace, called
through the C-ABI: two calls in a row, the second with fewer tokens (the
scratch keeps the first call's contents, so stale data must not leak), both
bitwise equal to the workspace entry point (same kernels, same order); plus
the capacity rejection, the nonfinite-producer error and no allocation."""
import ctypes as C

import numpy as np
import pytest

import oracle
from _fix import normal, random_q4k, random_q6k

pytestmark = pytest.mark.gpu


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.fixture(scope="module")
def weights(torch_gpu):
    import qw38_amd.ops as ops
    out = {}
    for name, wl, layout in (("gate", random_q4k(17408, 5120, 141), oracle.LAYOUT_Q4K_W64),
                             ("up", random_q4k(17408, 5120, 142), oracle.LAYOUT_Q4K_SEQ)):
        co, mo = wl.physical(layout)
        out[name] = ops.PrefillWeight.from_bytes(co, mo, layout, wl.n, wl.k)
    d6 = random_q6k(5120, 17408, 144)
    co, mo = d6.physical()
    out["down"] = ops.PrefillWeight.from_bytes(co, mo, oracle.LAYOUT_Q6K_W64, 5120, 17408)
    return out


def _static(torch, w, res, gamma, out, m, pending=None):
    import qw38_amd
    L = qw38_amd.lib()
    g, u, d = w["gate"].struct(), w["up"].struct(), w["down"].struct()
    submitted = C.c_int(0)
    st = L.qw38_q4k_q8_mlp_static(C.byref(g), C.byref(u), C.byref(d), res.data_ptr(),
                                  gamma.data_ptr(), 1e-6, out.data_ptr(), m,
                                  torch.cuda.current_stream().cuda_stream, C.byref(submitted),
                                  None if pending is None else pending.data_ptr())
    return st, submitted.value


def test_static_mlp_matches_workspace_entry(torch_gpu, weights):
    torch = torch_gpu
    import qw38_amd
    import qw38_amd.ops as ops
    L = qw38_amd.lib()
    assert L.qw38_q8_mlp_static_scratch_bytes() == ops.q8_mlp_workspace_bytes(64)
    gamma = _dev(torch, oracle.fp32_to_bf16(normal(5120, 150, 0.1)).view(np.int16))
    for m in (37, 5):  # second call smaller: stale scratch must not leak
        print(f"static mlp m={m}", flush=True)
        res = _dev(torch, normal((m, 5120), 160 + m))
        ws = torch.zeros(ops.q8_mlp_workspace_bytes(m), dtype=torch.uint8, device="cuda")
        want = torch.full((m, 5120), float("nan"), device="cuda")
        assert ops.q4k_q8_mlp(weights["gate"], weights["up"], weights["down"], res, gamma, 1e-6,
                              want, m, ws)
        got = torch.full((m, 5120), float("nan"), device="cuda")
        before = L.qw38_malloc_count()
        st, submitted = _static(torch, weights, res, gamma, got, m)
        torch.cuda.synchronize()
        assert st == 0 and submitted == 1
        assert L.qw38_malloc_count() == before
        assert torch.equal(got, want), f"m={m}: static-scratch MLP differs from the workspace MLP"


def test_static_mlp_rejections(torch_gpu, weights):
    torch = torch_gpu
    gamma = _dev(torch, oracle.fp32_to_bf16(normal(5120, 150, 0.1)).view(np.int16))
    m = 65  # over the scratch capacity: rejected before any launch
    res = torch.zeros(m, 5120, device="cuda")
    out = torch.zeros(m, 5120, device="cuda")
    st, submitted = _static(torch, weights, res, gamma, out, m)
    assert st == 2 and submitted == 0
    # a nonfinite producer is reported as the workspace entry point reports it,
    # and the flag is cleared again for the next call
    m = 3
    r = normal((m, 5120), 170)
    r[1, 3] = np.inf
    res = _dev(torch, r)
    out = torch.zeros(m, 5120, device="cuda")
    st, submitted = _static(torch, weights, res, gamma, out, m)
    assert st == 2 and submitted == 1
    res = _dev(torch, normal((m, 5120), 171))
    st, submitted = _static(torch, weights, res, gamma, out, m)
    torch.cuda.synchronize()
    assert st == 0 and submitted == 1
    assert torch.isfinite(out).all()
