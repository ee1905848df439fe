"""FP8 (OCP E4M3FN) projections through the C-ABI (cuda/fp8.hpp, cuda/fp8.cu):
pack_fp8 bit-exact against the oracle (the checks of tests/fp8_test.cpp:
77-92), GEMV / decode_mmv layout 0x020F and GEMM against the oracle's double
contraction within the reference's budget |y - ref| < 1e-4 + 1e-5 * l1
(tests/fp8_test.cpp:100, 116), a one-hot GEMM that returns every weight code's
value times its block scale exactly, and the BF16 store."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _pattern(m, k):
    """tests/fp8_test.cpp:44-49 input pattern as BF16 bits."""
    r = np.arange(m)[:, None]
    c = np.arange(k)[None, :]
    x = (((r * 23 + c * 17) % 97) - 48) * 0.03125 * (1 + r // 128 + c // 128)
    return oracle.fp32_to_bf16(x.astype(np.float32))


def _quantize_weight(w_bf16, n, k):
    """128 x 128 block weight quantizer (the offline compiler's, as checked by
    tests/fp8_test.cpp:57-71): scale = max(peak/448, FLT_MIN) (1 for a zero
    block), code = RNE(w / scale); padded to multiples of 128."""
    pn, pk = oracle.pad128(n), oracle.pad128(k)
    wf = np.zeros((pn, pk), np.float32)
    wf[:n, :k] = oracle.bf16_to_fp32(w_bf16)
    scales = np.zeros((pk // 128, pn // 128), np.float32)
    codes = np.zeros((pn, pk), np.uint8)
    for br in range(pn // 128):
        for bc in range(pk // 128):
            blk = wf[br * 128:(br + 1) * 128, bc * 128:(bc + 1) * 128]
            peak = np.float32(np.abs(blk).max())
            s = np.float32(1.0) if peak == 0 else max(peak / np.float32(448), np.float32(2.0 ** -126))
            scales[bc, br] = s
            codes[br * 128:(br + 1) * 128, bc * 128:(bc + 1) * 128] = oracle.fp32_to_e4m3(blk / s)
    return codes, scales, pn, pk


def _close(y, ref, l1, what):
    bad = np.abs(y.astype(np.float64) - ref) >= 1e-4 + 1e-5 * l1
    assert np.all(np.isfinite(y)) and not bad.any(), f"{what}: {np.argwhere(bad)[:5]}"


@pytest.mark.parametrize("m", [1, 130, 256])
def test_pack_fp8_bit_exact(torch_gpu, m):
    torch = torch_gpu
    import qw38_amd.ops as ops
    k = 387
    x = _pattern(m, k)
    x[0, 0] = oracle.fp32_to_bf16(np.array([80.0], np.float32))[0]
    if m > 2:
        x[1, :] = 0                   # zero row: scale 1, zero codes
        x[2, 200] = 0x7F80            # +inf: NaN scale for its block
    codes, scales = ops.pack_fp8(_dev(torch, x.view(np.int16)), m, k)
    wc, ws = oracle.pack_fp8(x, m, k)
    got_c, got_s = codes.cpu().numpy(), scales.cpu().numpy()
    assert np.array_equal(np.isnan(got_s), np.isnan(ws))
    fin = ~np.isnan(ws)
    assert np.array_equal(got_s[fin].view(np.uint32), ws[fin].view(np.uint32))
    assert np.array_equal(got_c, wc)
    if m > 2:
        assert np.isnan(ws[1, 2]) and np.all(wc[2, 128:256] & 127 == 127)


def test_fp8_gemv_and_decode(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 259, 500
    w = _pattern(n, k)
    w[0, 0] = oracle.fp32_to_bf16(np.array([80.0], np.float32))[0]
    codes, scales, pn, pk = _quantize_weight(w, n, k)
    xv = np.zeros(pk, np.uint16)
    xv[:k] = _pattern(1, k)[0]
    ref, l1 = oracle.fp8_gemv(codes, scales, pn, pk, xv)
    dc, ds = _dev(torch, codes), _dev(torch, scales)
    x = _dev(torch, xv.view(np.int16))
    y = torch.full((pn,), float("nan"), device="cuda")
    ops.fp8_gemv(ops.fp8_weight_struct(dc, ds, pn, pk), x, y)
    ys = y.cpu().numpy()
    _close(ys, ref, l1, "fp8_gemv")
    # decode_mmv layout 0x020F: the same contraction and every epilogue
    # (K must be a multiple of 256 there, cuda/decode_mmv.cu:331)
    yd = torch.full((pn,), float("nan"), device="cuda")
    ops.decode_mmv(ops.fp8_decode_desc(dc, ds, pn, pk, x, yd, ops.DECODE_STORE_FP32))
    assert np.array_equal(yd.cpu().numpy(), ys)
    yb = torch.empty(pn, dtype=torch.int16, device="cuda")
    ops.decode_mmv(ops.fp8_decode_desc(dc, ds, pn, pk, x, yb, ops.DECODE_STORE_BF16))
    assert np.array_equal(yb.cpu().numpy().view(np.uint16), oracle.fp32_to_bf16(ys))
    res = np.linspace(-1, 1, pn).astype(np.float32)
    r = _dev(torch, res)
    out = torch.empty(pn, device="cuda")
    ops.decode_mmv(ops.fp8_decode_desc(dc, ds, pn, pk, x, out, ops.DECODE_RESIDUAL_ADD_FP32, residual=r))
    assert np.array_equal(out.cpu().numpy(), (ys + res).astype(np.float32))
    ops.decode_mmv(ops.fp8_decode_desc(dc, ds, pn, pk, x, None, ops.DECODE_RESIDUAL_ADD_FP32, residual=r))
    assert np.array_equal(r.cpu().numpy(), (ys + res).astype(np.float32))
    # ranged launch (one FP8 projection per range, cuda/decode_mmv.cu:826-832)
    o1 = torch.empty(pn, dtype=torch.int16, device="cuda")
    o2 = torch.empty(pn, dtype=torch.int16, device="cuda")
    dc2, ds2 = dc.clone(), ds.clone()
    ops.decode_mmv_ranges([ops.fp8_decode_desc(dc, ds, pn, pk, x, o1, ops.DECODE_STORE_BF16),
                           ops.fp8_decode_desc(dc2, ds2, pn, pk, x, o2, ops.DECODE_STORE_BF16)])
    assert np.array_equal(o1.cpu().numpy(), yb.cpu().numpy())
    assert np.array_equal(o2.cpu().numpy(), yb.cpu().numpy())


@pytest.mark.parametrize("m", [128, 256])
def test_fp8_gemm_vs_oracle(torch_gpu, m):
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 259, 387
    w = _pattern(n, k)
    w[0, 0] = oracle.fp32_to_bf16(np.array([80.0], np.float32))[0]
    codes, scales, pn, pk = _quantize_weight(w, n, k)
    xb = np.zeros((m, pk), np.uint16)
    xb[:, :k] = _pattern(m, k)
    xc, xs = ops.pack_fp8(_dev(torch, xb.view(np.int16)), m, pk)
    dc, ds = _dev(torch, codes), _dev(torch, scales)
    y = torch.full((m, pn), float("nan"), device="cuda")
    work = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    sm = ops.fp8_prepare()
    assert sm > 0
    ops.fp8_gemm(ops.fp8_weight_struct(dc, ds, pn, pk), ops.fp8_input_struct(xc, xs, m, pk), y, work, sm)
    ref, l1 = oracle.fp8_gemm(codes, scales, pn, pk, xc.cpu().numpy(), xs.cpu().numpy(), m)
    _close(y.cpu().numpy(), ref, l1, f"fp8_gemm m={m}")
    # a sibling consumer of the same pack gets identical results, pack untouched
    y2 = torch.empty_like(y)
    ops.fp8_gemm(ops.fp8_weight_struct(dc, ds, pn, pk), ops.fp8_input_struct(xc, xs, m, pk), y2, work, sm)
    assert torch.equal(y, y2)


def test_fp8_gemm_onehot_every_code(torch_gpu):
    """Weights hold every non-NaN code; one-hot activations (code 0x38 = 1.0,
    scale 1) make each output one product: value(code) * weight scale, exact."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k, m = 256, 256, 128
    codes = np.arange(n * k, dtype=np.int64).reshape(n, k) % 254
    codes = np.where(codes >= 127, codes + 1, codes).astype(np.uint8)  # skip 0x7F, 0xFF
    rng = np.random.Generator(np.random.PCG64(3))
    scales = (rng.random((k // 128, n // 128)) + 0.5).astype(np.float32)
    xc = np.zeros((m, k), np.uint8)
    cols = (np.arange(m) * 7) % k
    xc[np.arange(m), cols] = 0x38
    xs = np.ones((k // 128, m), np.float32)
    y = torch.empty(m, n, device="cuda")
    work = torch.empty(256, dtype=torch.uint8, device="cuda")
    # the structs hold raw pointers: keep every tensor alive across the call
    dw, dws, dx, dxs = _dev(torch, codes), _dev(torch, scales), _dev(torch, xc), _dev(torch, xs)
    ops.fp8_gemm(ops.fp8_weight_struct(dw, dws, n, k), ops.fp8_input_struct(dx, dxs, m, k), y, work, 1)
    vals = oracle.e4m3_to_fp32(codes).astype(np.float64)
    want = (vals[:, cols].T * scales[cols // 128][:, np.arange(n) // 128]).astype(np.float32)
    got = y.cpu().numpy()
    bad = np.argwhere(got != want)   # +-0 compare equal
    assert not bad.size, [(int(t), int(r), int(codes[r, cols[t]]), float(got[t, r]), float(want[t, r]))
                          for t, r in bad[:8]] + [len(bad)]


@pytest.mark.parametrize("n,k,m", [(12288, 6144, 512), (1024, 17408, 128)])
def test_fp8_gemm_large_sampled(torch_gpu, n, k, m):
    torch = torch_gpu
    import qw38_amd.ops as ops
    print(f"fp8 gemm n={n} k={k} m={m}", flush=True)
    rng = np.random.Generator(np.random.PCG64(n + k))
    codes = rng.integers(0, 256, (n, k)).astype(np.uint8)
    codes[(codes & 127) == 127] = 0
    scales = (rng.random((k // 128, n // 128)) * 1e-3).astype(np.float32)
    xb = oracle.fp32_to_bf16(rng.standard_normal((m, k)).astype(np.float32))
    xc, xs = ops.pack_fp8(_dev(torch, xb.view(np.int16)), m, k)
    y = torch.empty(m, n, device="cuda")
    work = torch.empty(256, dtype=torch.uint8, device="cuda")
    dw, dws = _dev(torch, codes), _dev(torch, scales)
    ops.fp8_gemm(ops.fp8_weight_struct(dw, dws, n, k), ops.fp8_input_struct(xc, xs, m, k), y, work,
                 ops.fp8_prepare())
    toks = np.array([0, 1, m // 2, m - 1])
    xcs, xss = xc.cpu().numpy()[toks], xs.cpu().numpy()[:, toks]
    yh = y.cpu().numpy()[toks]
    for blk in (0, n // 128 - 1):   # two whole 128-row blocks, each with its own scales
        rows = slice(blk * 128, blk * 128 + 128)
        ref, l1 = oracle.fp8_gemm(codes[rows], np.ascontiguousarray(scales[:, blk:blk + 1]), 128, k,
                                  xcs, xss, len(toks))
        _close(yh[:, rows], ref, l1, f"fp8_gemm {n}x{k} m={m} block {blk}")


def test_fp8_store_bf16(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    rng = np.random.Generator(np.random.PCG64(4))
    x = (rng.standard_normal(100003) * 1e3).astype(np.float32)
    x[:4] = [np.inf, -np.inf, np.nan, 0.0]
    y = torch.empty(x.size, dtype=torch.int16, device="cuda")
    ops.fp8_store_bf16(_dev(torch, x), y)
    got = y.cpu().numpy().view(np.uint16)
    want = oracle.fp32_to_bf16(x)
    fin = np.isfinite(x)
    assert np.array_equal(got[fin], want[fin])
    assert got[0] == 0x7F80 and got[1] == 0xFF80 and (got[2] & 0x7FFF) > 0x7F80


@pytest.mark.parametrize("tokens", [1, 77, 300])
def test_fp8_project_epilogues(torch_gpu, tokens):
    """The fused prefill epilogues equal the reference's two-pass order:
    fp8_gemm into FP32, then BF16 RNE / FP32 / residual + value per valid
    token (cuda/prefill.cu:116-134, 583-593); padded tokens are not written."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 384, 512
    rng = np.random.Generator(np.random.PCG64(tokens))
    codes = rng.integers(0, 256, (n, k)).astype(np.uint8)
    codes[(codes & 127) == 127] = 1
    scales = (rng.random((k // 128, n // 128)) * 1e-2).astype(np.float32)
    xb = oracle.fp32_to_bf16(rng.standard_normal((tokens, k)).astype(np.float32))
    xc, xs = ops.pack_fp8(_dev(torch, xb.view(np.int16)), tokens, k)
    w = ops.fp8_weight_struct(_dev(torch, codes), _dev(torch, scales), n, k)
    xin = ops.fp8_input_struct(xc, xs, xc.shape[0], k)
    raw = torch.empty(xc.shape[0], n, device="cuda")
    work = torch.empty(256, dtype=torch.uint8, device="cuda")
    ops.fp8_gemm(w, xin, raw, work, 1)
    rawv = raw.cpu().numpy()[:tokens]
    yb = torch.full((tokens + 1, n), -1, dtype=torch.int16, device="cuda")
    ops.fp8_project(w, xin, tokens, yb, ops.DECODE_STORE_BF16)
    ybv = yb.cpu().numpy().view(np.uint16)
    assert np.array_equal(ybv[:tokens], oracle.fp32_to_bf16(rawv))
    assert np.all(ybv[tokens] == 0xFFFF)
    yf = torch.full((tokens + 1, n), 7.0, device="cuda")
    ops.fp8_project(w, xin, tokens, yf, ops.DECODE_STORE_FP32)
    assert np.array_equal(yf.cpu().numpy()[:tokens], rawv) and torch.all(yf[tokens] == 7.0)
    res = rng.standard_normal((tokens, n)).astype(np.float32)
    yr = torch.empty(tokens, n, device="cuda")
    ops.fp8_project(w, xin, tokens, yr, ops.DECODE_RESIDUAL_ADD_FP32, residual=_dev(torch, res))
    assert np.array_equal(yr.cpu().numpy(), res + rawv)
    ref, l1 = oracle.fp8_gemm(codes, scales, n, k, xc.cpu().numpy(), xs.cpu().numpy(), xc.shape[0])
    _close(rawv, ref[:tokens], l1[:tokens], f"fp8_project tokens={tokens}")
