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
    """Gate and up in both Q4_K layouts (mixed layouts run the unfused chain;
    equal layouts the fused gate+up launch), Q6_K down."""
    import qw38_amd.ops as ops
    out = {}
    for name, wl in (("gate", random_q4k(17408, 5120, 141)), ("up", random_q4k(17408, 5120, 142))):
        for tag, layout in (("w64", oracle.LAYOUT_Q4K_W64), ("seq", oracle.LAYOUT_Q4K_SEQ)):
            co, mo = wl.physical(layout)
            out[f"{name}_{tag}"] = ops.PrefillWeight.from_bytes(co, mo, layout, wl.n, wl.k)
    d6 = random_q6k(5120, 17408, 144)
    co, mo = d6.physical()
    out["down"] = ops.PrefillWeight.from_bytes(co, mo, oracle.LAYOUT_Q6K_W64, 5120, 17408)
    return out


def _pick(weights, gate, up):
    return {"gate": weights[f"gate_{gate}"], "up": weights[f"up_{up}"], "down": weights["down"]}


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


# (gate layout, up layout, m): mixed layouts take the unfused chain; equal
# layouts take the fused gate+up launch (m = 1 on 0x020D: the streaming GLU
# kernel; m > 8: the MMQ with the SwiGLU->Q8 epilogue), whose input operand
# sits in the gate slab of the scratch. Each group's second call is smaller.
CASES = [("w64", "seq", 37), ("w64", "seq", 5),
         ("seq", "seq", 1), ("w64", "w64", 37), ("w64", "w64", 9)]


def test_static_mlp_matches_workspace_entry(torch_gpu, weights):
    torch = torch_gpu
    import qw38_amd
    import qw38_amd.ops as ops
    L = qw38_amd.lib()
    assert L.qw38_q8_mlp_static_scratch_bytes() == ops.q8_mlp_workspace_bytes(64)
    gamma = _dev(torch, oracle.fp32_to_bf16(normal(5120, 150, 0.1)).view(np.int16))
    for gl, ul, m in CASES:
        print(f"static mlp gate={gl} up={ul} m={m}", flush=True)
        w = _pick(weights, gl, ul)
        res = _dev(torch, normal((m, 5120), 160 + m))
        ws = torch.zeros(ops.q8_mlp_workspace_bytes(m), dtype=torch.uint8, device="cuda")
        want = torch.full((m, 5120), float("nan"), device="cuda")
        assert ops.q4k_q8_mlp(w["gate"], w["up"], w["down"], res, gamma, 1e-6, want, m, ws)
        got = torch.full((m, 5120), float("nan"), device="cuda")
        before = L.qw38_malloc_count()
        st, submitted = _static(torch, w, res, gamma, got, m)
        torch.cuda.synchronize()
        assert st == 0 and submitted == 1
        assert L.qw38_malloc_count() == before
        assert torch.equal(got, want), f"{gl}/{ul} m={m}: static-scratch MLP differs from the workspace MLP"


def test_static_mlp_rejections(torch_gpu, weights):
    torch = torch_gpu
    weights = _pick(weights, "w64", "seq")
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


def test_static_mlp_rejects_overlap_on_another_stream(torch_gpu, weights):
    """Calls must be serialized per device: while a call's work is still queued
    on one stream, a call on another stream is rejected before any launch
    (submitted stays 0); a call on the same stream is ordered by it and
    accepted; once the first stream drains the other stream is accepted."""
    torch = torch_gpu
    w = _pick(weights, "w64", "seq")
    gamma = _dev(torch, oracle.fp32_to_bf16(normal(5120, 150, 0.1)).view(np.int16))
    m = 4
    res = _dev(torch, normal((m, 5120), 180))
    pending = torch.zeros(1, dtype=torch.int32, device="cuda")
    outs = [torch.full((m, 5120), float("nan"), device="cuda") for _ in range(3)]
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(s1):
        torch.cuda._sleep(200_000_000)  # keeps s1 busy (~0.1 s) so its MLP is still queued below
        st, submitted = _static(torch, w, res, gamma, outs[0], m, pending)
        assert st == 0 and submitted == 1
        st, submitted = _static(torch, w, res, gamma, outs[1], m, pending)
        assert st == 0 and submitted == 1, "same stream: ordered, accepted"
    with torch.cuda.stream(s2):
        st, submitted = _static(torch, w, res, gamma, outs[2], m, pending)
    assert st == 2 and submitted == 0, "overlapping call on another stream must be rejected"
    s1.synchronize()
    with torch.cuda.stream(s2):
        st, submitted = _static(torch, w, res, gamma, outs[2], m, pending)
        assert st == 0 and submitted == 1
    torch.cuda.synchronize()
    assert int(pending.item()) == 0
    assert torch.isfinite(outs[0]).all()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
