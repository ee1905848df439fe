"""Bit-exactness of the per-group integer dots inside the production kernels.

The reference's contraction (cuda/q4k_q8.cu:97,140,245) is, per row r, token t
and K32 group g, a_tg * (d_r s_rg dot_rtg - dmin_r m_rg sum_tg) with an exact
int32 dot. With fp16 d = dmin = 1 (Q4_K) or d = 1 (Q6_K) and activations
whose every K32 group peaks at exactly +-127 (so the Q8 scale is
a = RN(127/127) = 1 and the codes equal the integer inputs), every output is
the exact integer sum_g (s_rg dot_rtg - m_rg sum_tg) (Q4_K) or
sum_sub sc_r,sub dot_r,t,sub (Q6_K). The inputs bound the sum of the absolute
values of all terms below 2^24, so every FP32 partial sum in any order is an
exact integer: a production kernel (GEMV at M = 1..8 on both Q4_K layouts and
the Q6_K layout, the MMQ at every tile shape the dispatcher picks, including
the tail split) must then match the closed form BIT-EXACTLY. A wrong code,
nibble order, scale/min index or dropped group shows up as an integer
mismatch, not as a tolerance question (tests/q4k_q8_test.cpp:121-131 states
the same closed form in double).

The expected values are computed here in float64 over integers (exact below
2^53), independently of the C oracle.
"""
import numpy as np
import pytest

import oracle


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def pack_scale_min(s, m):
    """12-byte 6-bit scale/min packing of arrays s, m [..., 8] (the inverse of
    llama.cpp get_scale_min_k4, third_party/llama.cpp-q4k/reference.hpp)."""
    s = s.astype(np.uint8)
    m = m.astype(np.uint8)
    p = np.zeros(s.shape[:-1] + (12,), np.uint8)
    for g in range(8):
        if g < 4:
            p[..., g] |= s[..., g]
            p[..., g + 4] |= m[..., g]
        else:
            p[..., g + 4] |= (s[..., g] & 15) | ((m[..., g] & 15) << 4)
            p[..., g - 4] |= (s[..., g] >> 4) << 6
            p[..., g] |= (m[..., g] >> 4) << 6
    return p


def integer_q4k(n, k, seed, smax):
    """Q4_K with d = dmin = 1.0 and random s, m in [0, smax]; returns the
    logical weight and the integer effective matrix s*w - m [n][k]."""
    rng = np.random.Generator(np.random.PCG64(seed))
    assert k % 256 == 0
    kbs = k // 256
    codes = rng.integers(0, 16, size=(n, k), dtype=np.uint8)
    s = rng.integers(0, smax + 1, size=(n, kbs, 8))
    mn = rng.integers(0, smax + 1, size=(n, kbs, 8))
    meta = np.zeros((n, kbs, 16), np.uint8)
    meta[..., 0], meta[..., 1] = 0x00, 0x3C  # fp16 1.0
    meta[..., 2], meta[..., 3] = 0x00, 0x3C
    meta[..., 4:] = pack_scale_min(s, mn)
    sg = np.repeat(s.reshape(n, kbs * 8), 32, axis=1)
    mg = np.repeat(mn.reshape(n, kbs * 8), 32, axis=1)
    weff = sg * codes.astype(np.int64) - mg
    return oracle.Q4K(codes, meta, n, k), weff


def integer_q6k(n, k, seed, scmax):
    """Q6_K with d = 1.0 and sub-block scales in [-scmax, scmax]."""
    rng = np.random.Generator(np.random.PCG64(seed))
    q = rng.integers(0, 64, size=(n, k), dtype=np.uint8)
    sc = rng.integers(-scmax, scmax + 1, size=(n, k // 16)).astype(np.int8)
    d = np.full((n, k // 256), 0x3C00, np.uint16)
    weff = np.repeat(sc.astype(np.int64), 16, axis=1) * (q.astype(np.int64) - 32)
    return oracle.Q6K(q, sc, d, n, k), weff


def integer_rows(m, k, seed):
    """Integer activations in {-1, 0, 1} with one +-127 per K32 group, so each
    group's Q8 scale is exactly 1 and the codes are the values themselves."""
    rng = np.random.Generator(np.random.PCG64(seed))
    x = rng.integers(-1, 2, size=(m, k)).astype(np.float32)
    g = k // 32
    pos = rng.integers(0, 32, size=(m, g))
    sign = np.where(rng.integers(0, 2, size=(m, g)) == 1, 127.0, -127.0).astype(np.float32)
    x.reshape(m, g, 32)[np.arange(m)[:, None], np.arange(g)[None, :], pos] = sign
    return x


def _q8(torch, ops, x):
    m, k = x.shape
    bf = oracle.fp32_to_bf16(x)
    q = ops.Q8Input.empty(m, k)
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    ops.pack_q8(_dev(torch, bf.view(np.int16)), q, flag)
    torch.cuda.synchronize()
    assert int(flag.item()) == 0
    assert np.all(q.scales.cpu().numpy() == 1.0)
    assert np.array_equal(q.codes.cpu().numpy().astype(np.float32), x)
    return q


def _run(torch, ops, w, q, m, n):
    out = torch.full((m, n), float("nan"), device="cuda")
    ops.q4k_q8_project(w, q, out)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _exact(weff, x):
    bound = np.abs(weff).astype(np.float64) @ np.abs(x.T).astype(np.float64)
    assert bound.max() < 2 ** 24, "test inputs must keep every FP32 partial sum exact"
    return (weff.astype(np.float64) @ x.T.astype(np.float64)).T.astype(np.float32)


def _assert_exact(y, ref, label):
    bad = np.argwhere(y != ref)
    print(f"{label}: {len(bad)} mismatches", flush=True)
    assert len(bad) == 0, f"{label}: first mismatch at {bad[0]}: {y[tuple(bad[0])]} != {ref[tuple(bad[0])]}"


@pytest.mark.gpu
@pytest.mark.parametrize("layout", [oracle.LAYOUT_Q4K_SEQ, oracle.LAYOUT_Q4K_W64], ids=["020D", "0240"])
@pytest.mark.parametrize("n,k", [(264, 5120), (4104, 2560)])
def test_gemv_q4k_integer_exact(torch_gpu, layout, n, k):
    """Decode GEMV kernels (streaming M <= 2, 8-row kernel M 3..8, and the
    0x0240 kernel) at config-1 K and a row count that fills every CU."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    w, weff = integer_q4k(n, k, 11 + n, 31 if k > 2560 else 63)
    co, mo = w.physical(layout)
    dw = ops.PrefillWeight.from_bytes(co, mo, layout, n, k)
    for m in range(1, 9):
        x = integer_rows(m, k, 100 + m)
        y = _run(torch, ops, dw, _q8(torch, ops, x), m, n)
        _assert_exact(y, _exact(weff, x), f"Q4_K GEMV layout={layout:#x} n={n} k={k} M={m}")


@pytest.mark.gpu
@pytest.mark.parametrize("layout", [oracle.LAYOUT_Q4K_SEQ, oracle.LAYOUT_Q4K_W64], ids=["020D", "0240"])
@pytest.mark.parametrize("n,m", [(4104, 25), (4104, 40), (34816, 64), (4104, 130), (34816, 512), (5120, 512),
                                 (12288, 512), (8192, 512)])
def test_mmq_q4k_integer_exact(torch_gpu, layout, n, m):
    """MMQ tile shapes: direct-copy 128x16 / 128x32 on 0x020D, mmq_kernel's
    128x32 on 0x0240 (M=25, 40 on 4104 rows; M = 9..24 on small weights runs
    batched-decode passes instead), 128x64 (M=64 on 34816
    rows), 256x128 (M=130), 256x128 plus the 128x32 tail split (M=512 on
    34816 rows, config 2's N) and the eight-wave 80x128, 192x128 and 128x128
    tiles (M=512 on 5120, 12288 and 8192 rows)."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    k = 2560
    w, weff = integer_q4k(n, k, 7 * n + m, 63)
    co, mo = w.physical(layout)
    dw = ops.PrefillWeight.from_bytes(co, mo, layout, n, k)
    x = integer_rows(m, k, 500 + m)
    y = _run(torch, ops, dw, _q8(torch, ops, x), m, n)
    _assert_exact(y, _exact(weff, x), f"Q4_K MMQ layout={layout:#x} n={n} M={m}")


@pytest.mark.gpu
@pytest.mark.parametrize("n,k", [(264, 2048), (5120, 2048), (776, 2304)])
def test_q6k_integer_exact(torch_gpu, n, k):
    """Q6_K (layout 0x0241): streaming GEMV (M <= 2), int8-MFMA decode (M 3..8,
    and M = 9 as two such passes where the cost model picks them) and the MMQ
    (M = 40, 130, 512: split tiles up to M = 128, the direct-copy 160x128 tile
    above; K = 2304 gives it an odd super-block count in one K segment and a
    partial last row tile)."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    w, weff = integer_q6k(n, k, 3 * n, 16)
    co, mo = w.physical()
    dw = ops.PrefillWeight.from_bytes(co, mo, oracle.LAYOUT_Q6K_W64, n, k)
    for m in (1, 2, 3, 5, 8, 9, 40, 130, 512):
        x = integer_rows(m, k, 900 + m)
        y = _run(torch, ops, dw, _q8(torch, ops, x), m, n)
        _assert_exact(y, _exact(weff, x), f"Q6_K n={n} k={k} M={m}")


def test_integer_fixture_matches_oracle():
    """The closed form used above agrees with the oracle's contraction on the
    same integer weights (CPU only: ties the fixture to the checked oracle)."""
    n, k, m = 24, 512, 3
    w, weff = integer_q4k(n, k, 5, 63)
    x = integer_rows(m, k, 6)
    q = oracle.pack_q8(oracle.fp32_to_bf16(x), m, k)
    ref, _, _ = oracle.q4k_q8_contract(w, q)
    assert np.array_equal(ref.astype(np.float32), _exact(weff, x))
    w6, weff6 = integer_q6k(n, k, 7, 16)
    ref6, _, _ = oracle.q6k_q8_contract(w6, q)
    assert np.array_equal(ref6.astype(np.float32), _exact(weff6, x))
