"""BF16-activation decode GEMV over Q4_K 0x020D (cuda/decode_mmv.cu:121-250)
through the C-ABI: the exact one-hot operand test of
tests/decode_mmv_unit_test.cpp:405-478 restated, random projections against
the oracle (float64 sum of the rebuilt BF16 operands), every epilogue, the
paired and ranged launches, odd super-block counts and ragged N."""
import numpy as np
import pytest

import oracle
from _fix import normal, random_q4k

pytestmark = pytest.mark.gpu


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _weight(ops, wl):
    co, mo = wl.physical(oracle.LAYOUT_Q4K_SEQ)
    return ops.PrefillWeight.from_bytes(co, mo, oracle.LAYOUT_Q4K_SEQ, wl.n, wl.k)


def _bf16(torch, x):
    return _dev(torch, oracle.fp32_to_bf16(np.asarray(x, np.float32)).view(np.int16))


def _tol_ok(y, ref):
    """The reference's own decode budget (cuda/decode_mmv.hpp:108-112:
    |y - ref| <= 1e-3 + 1e-4 |ref|) and the north-star tolerance."""
    ok_ref = np.all(np.abs(y - ref) <= 1e-3 + 1e-4 * np.abs(ref))
    ok, ma, mr = oracle.parity_ok(y, ref)
    return ok_ref and ok, ma, mr


def _onehot_fixture():
    """tests/decode_mmv_unit_test.cpp:409-446: eight rows with fp16 d/dmin from
    zero and subnormals up to normal values, patterned 6-bit scales/minima and
    codes (col + 5 row) % 16."""
    n, k = 8, 256
    d_bits = [0, 1, 2, 0x3FF, 0x400, 0x1400, 0x2400, 0x3400]
    m_bits = [0, 3, 1, 0x201, 0x3FF, 0x1000, 0x2000, 0x3000]
    codes = np.zeros((n, k), np.uint8)
    meta = np.zeros((n, 1, 16), np.uint8)
    for row in range(n):
        sc = [(g * 9 + row * 13) % 64 for g in range(8)]
        mn = [(63 - g * 7 + row * 3) % 64 for g in range(8)]
        m = meta[row, 0]
        m[0], m[1] = d_bits[row] & 255, d_bits[row] >> 8
        m[2], m[3] = m_bits[row] & 255, m_bits[row] >> 8
        for g in range(4):
            m[4 + g] = sc[g] | ((sc[g + 4] >> 4) << 6)
            m[8 + g] = mn[g] | ((mn[g + 4] >> 4) << 6)
            m[12 + g] = (sc[g + 4] & 15) | ((mn[g + 4] & 15) << 4)
        codes[row] = [(col + 5 * row) % 16 for col in range(k)]
    return oracle.Q4K(codes, meta, n, k)


def test_onehot_exact_operands(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    wl = _onehot_fixture()
    w = _weight(ops, wl)
    y = torch.zeros(8, dtype=torch.float32, device="cuda")
    xs = torch.zeros(256, 256, dtype=torch.int16, device="cuda")
    for col in range(256):
        xs[col, col] = 0x3F80  # BF16 1.0
    got = np.zeros((256, 8), np.float32)
    for col in range(256):
        ops.decode_mmv(ops.decode_desc(w, xs[col], y, ops.DECODE_STORE_FP32))
        got[col] = y.cpu().numpy()
    for col in range(256):
        x = np.zeros(256, np.uint16)
        x[col] = 0x3F80
        exp = oracle.q4k_bf16_gemv(wl, x).astype(np.float32)
        assert np.array_equal(got[col].view(np.uint32), exp.view(np.uint32)), f"col {col}"


@pytest.mark.parametrize("n,k", [(5120, 5120), (37, 768), (2000, 17408)])
def test_random_projection_vs_oracle(torch_gpu, n, k):
    torch = torch_gpu
    import qw38_amd.ops as ops
    wl = random_q4k(n, k, n + k)
    w = _weight(ops, wl)
    x = normal(k, n * 3 + k)
    xb = oracle.fp32_to_bf16(x)
    y = torch.full((n,), float("nan"), device="cuda")
    ops.decode_mmv(ops.decode_desc(w, _bf16(torch, x), y, ops.DECODE_STORE_FP32))
    got = y.cpu().numpy()
    ref = oracle.q4k_bf16_gemv(wl, xb)
    ok, ma, mr = _tol_ok(got, ref)
    print(f"decode_bf16 n={n} k={k}: max_abs/rms={ma:.3g} mean_rel={mr:.3g}", flush=True)
    assert ok


def test_epilogues_and_inplace_residual(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 136, 1024
    wl = random_q4k(n, k, 5)
    w = _weight(ops, wl)
    x = _bf16(torch, normal(k, 6))
    f32 = torch.empty(n, device="cuda")
    ops.decode_mmv(ops.decode_desc(w, x, f32, ops.DECODE_STORE_FP32))
    base = f32.cpu().numpy()
    b16 = torch.empty(n, dtype=torch.int16, device="cuda")
    ops.decode_mmv(ops.decode_desc(w, x, b16, ops.DECODE_STORE_BF16))
    assert np.array_equal(b16.cpu().numpy().view(np.uint16), oracle.fp32_to_bf16(base))
    res = normal(n, 7)
    r = _dev(torch, res)
    out = torch.empty(n, device="cuda")
    ops.decode_mmv(ops.decode_desc(w, x, out, ops.DECODE_RESIDUAL_ADD_FP32, residual=r))
    assert np.array_equal(out.cpu().numpy(), (res + base).astype(np.float32))
    assert np.array_equal(r.cpu().numpy(), res), "separate output leaves the residual intact"
    ops.decode_mmv(ops.decode_desc(w, x, None, ops.DECODE_RESIDUAL_ADD_FP32, residual=r))
    assert np.array_equal(r.cpu().numpy(), (res + base).astype(np.float32)), "in-place update"


def test_paired_and_ranges(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 1000, 2560
    gl, ul = random_q4k(n, k, 11), random_q4k(n, k, 12)
    g, u = _weight(ops, gl), _weight(ops, ul)
    x = _bf16(torch, normal(k, 13))
    ga, ua = torch.empty(n, device="cuda"), torch.empty(n, device="cuda")
    ops.decode_mmv(ops.decode_desc(g, x, ga, ops.DECODE_STORE_FP32))
    ops.decode_mmv(ops.decode_desc(u, x, ua, ops.DECODE_STORE_FP32))
    gs, us = ga.cpu().numpy(), ua.cpu().numpy()
    # paired, separate FP32 outputs: bitwise equal to the single launches
    pa, pb = torch.empty(n, device="cuda"), torch.empty(n, device="cuda")
    ops.decode_mmv_paired(ops.decode_desc(g, x, pa, ops.DECODE_STORE_FP32),
                          ops.decode_desc(u, x, pb, ops.DECODE_STORE_FP32))
    assert np.array_equal(pa.cpu().numpy(), gs) and np.array_equal(pb.cpu().numpy(), us)
    # paired SwiGLU -> BF16 into A's output; B declares no output
    sw = torch.empty(n, dtype=torch.int16, device="cuda")
    ops.decode_mmv_paired(ops.decode_desc(g, x, sw, ops.DECODE_SWIGLU_BF16),
                          ops.decode_desc(u, x, None, ops.DECODE_SWIGLU_BF16))
    gd, ud = gs.astype(np.float64), us.astype(np.float64)
    ref = oracle.bf16_to_fp32(oracle.fp32_to_bf16((gd / (1 + np.exp(-gd)) * ud).astype(np.float32)))
    got = oracle.bf16_to_fp32(sw.cpu().numpy().view(np.uint16))
    ulp = np.abs(ref.view(np.int32).astype(np.int64) - got.view(np.int32).astype(np.int64))
    assert np.all(ulp <= 65536), "SwiGLU within one BF16 ulp of the float64 formula"
    # ranges: BF16 stores equal to single launches
    outs = [torch.empty(n, dtype=torch.int16, device="cuda") for _ in range(2)]
    ops.decode_mmv_ranges([ops.decode_desc(g, x, outs[0], ops.DECODE_STORE_BF16),
                           ops.decode_desc(u, x, outs[1], ops.DECODE_STORE_BF16)])
    assert np.array_equal(outs[0].cpu().numpy().view(np.uint16), oracle.fp32_to_bf16(gs))
    assert np.array_equal(outs[1].cpu().numpy().view(np.uint16), oracle.fp32_to_bf16(us))


def test_gate_up_config_shape(torch_gpu):
    """Config-2 shape through the BF16 path: gate+up as one N=34816 matrix,
    row-sampled against the oracle."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 34816, 5120
    wl = random_q4k(n, k, 21)
    w = _weight(ops, wl)
    x = normal(k, 22)
    y = torch.empty(n, device="cuda")
    ops.decode_mmv(ops.decode_desc(w, _bf16(torch, x), y, ops.DECODE_STORE_FP32))
    rows = np.sort(np.random.Generator(np.random.PCG64(3)).choice(n, 512, replace=False))
    sub = oracle.Q4K(wl.codes[rows], wl.meta[rows], len(rows), k)
    ref = oracle.q4k_bf16_gemv(sub, oracle.fp32_to_bf16(x))
    ok, ma, mr = _tol_ok(y.cpu().numpy()[rows], ref)
    print(f"decode_bf16 config2: max_abs/rms={ma:.3g} mean_rel={mr:.3g}", flush=True)
    assert ok
