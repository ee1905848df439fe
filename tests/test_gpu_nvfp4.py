"""NVFP4 through the C-ABI (cuda/nvfp4.hpp, the NVFP4 branches of
cuda/prefill.cu and decode_mmv layout 0x020E), in the order of the
reference's tests/nvfp4_test.cpp: packer bytes against the exhaustive
nearest-value oracle (midpoints, ties, tails, padding, NaN scale), the fused
RMS producers against RMS + pack, the W4A4 contraction against the double
closed form within the reference's budget (1e-3 + 1e-4 |ref|, and 1e-5 of
the L1 norm), fused prefill epilogues equal to the raw tile, paired SwiGLU,
decode single/paired/epilogues, ranged launches rejected, and the NVFP4 MLP
equal to its stages."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _input(m, k, seed):
    """tests/nvfp4_test.cpp:40-46 input pattern as BF16 bits (first 16 zero)."""
    i = np.arange(m * k)
    x = oracle.fp32_to_bf16((((i * 17 + seed) % 131) - 65).astype(np.float32) / np.float32(27))
    x[:16] = 0
    return x.reshape(m, k)


def _close(y, ref, l1, what):
    y = np.asarray(y, np.float64)
    bad = (np.abs(y - ref) > 1e-3 + 1e-4 * np.abs(ref)) | (np.abs(y - ref) > 1e-6 + 1e-5 * l1)
    assert np.all(np.isfinite(y)) and not bad.any(), f"{what}: {np.argwhere(bad)[:5]}"


def _weight(torch, n, k, seed):
    import qw38_amd.ops as ops
    codes, scales = oracle.quantize_nvfp4(_input(n, k, seed), n, k)
    dc, ds = _dev(torch, codes), _dev(torch, scales)
    return ops.nvfp4_weight(dc, ds, n, k), codes, scales


def test_pack_nvfp4_bytes(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    m, k = 3, 5120
    x = _input(m, k, 2)
    for b in range(1, 126):  # scale midpoints (tests/nvfp4_test.cpp:131-134)
        mid = (oracle.ue4m3_value(b) + oracle.ue4m3_value(b + 1)) * 3
        x.reshape(-1)[b * 16:b * 16 + 16] = oracle.fp32_to_bf16(np.array([mid], np.float32))[0]
    t = np.array([.25, .75, 1.25, 1.75, 2.5, 3.5, 5., 6.], np.float32)
    x.reshape(-1)[128 * 16:128 * 16 + 16] = oracle.fp32_to_bf16(np.concatenate([t, -t]))
    x.reshape(-1)[k + 17] = oracle.fp32_to_bf16(np.array([3000.], np.float32))[0]
    codes, scales = ops.pack_nvfp4(_dev(torch, x.view(np.int16)), m, k)
    wc, ws = oracle.pack_nvfp4(x, m, k)
    assert np.array_equal(scales.cpu().numpy(), ws)
    assert np.array_equal(codes.cpu().numpy(), wc)
    # same-row chunk independence (tests/nvfp4_test.cpp:149-152)
    c1, _ = ops.pack_nvfp4(_dev(torch, x[:1].view(np.int16)), 1, k)
    assert np.array_equal(c1.cpu().numpy()[0], wc[0])
    # ragged K, zero rows, nonfinite block -> NaN scale 127 and zero codes
    m, k = 130, 387
    rng = np.random.Generator(np.random.PCG64(1))
    x = oracle.fp32_to_bf16((rng.standard_normal((m, k)) * 5).astype(np.float32))
    x[7] = 0
    x[9, 100] = 0x7FC0
    codes, scales = ops.pack_nvfp4(_dev(torch, x.view(np.int16)), m, k)
    wc, ws = oracle.pack_nvfp4(x, m, k)
    assert np.array_equal(scales.cpu().numpy(), ws)
    assert np.array_equal(codes.cpu().numpy(), wc)
    assert ws[oracle.nvfp4_sf_index(9, 6, 512)] == 127


def test_fused_rms_producers_equal_rms_then_pack(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    for m in (3, 130):
        print(f"rms producers m={m}", flush=True)
        h = ((np.arange(m * 5120) % 71) - 35).astype(np.float32).reshape(m, 5120) * np.float32(.3)
        h[1] *= 1e-3
        gamma = _input(1, 5120, 7)[0]
        dh, dg = _dev(torch, h), _dev(torch, gamma.view(np.int16))
        bf = torch.empty(m, 5120, dtype=torch.int16, device="cuda")
        ops.hidden_rms_bf16(dh, dg, 1e-6, m, bf)
        c0, s0 = ops.pack_nvfp4(bf, m, 5120)
        c1 = torch.full_like(c0, 0xAB)
        s1 = torch.full_like(s0, 0xCD)
        ops.hidden_rms_nvfp4(dh, dg, 1e-6, m, c1, s1)
        assert torch.equal(c0, c1) and torch.equal(s0, s1), "fused RMS NVFP4 preserves exact rounding"
        f0, g0 = ops.pack_fp8(bf, m, 5120)
        f1, g1 = torch.empty_like(f0), torch.empty_like(g0)
        comp = torch.empty_like(bf)
        ops.hidden_rms_fp8(dh, dg, 1e-6, m, f1, g1, companion=comp)
        assert torch.equal(f0, f1) and torch.equal(g0, g1), "fused RMS FP8 preserves exact rounding"
        assert torch.equal(comp, bf)


@pytest.mark.parametrize("m", [1, 2, 3, 129, 256])
def test_gemm_tile_vs_oracle(torch_gpu, m):
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 136, 5120
    w, wc, ws = _weight(torch, n, k, 27)
    x = _input(m, k, 13)
    xc, xs = ops.pack_nvfp4(_dev(torch, x.view(np.int16)), m, k)
    y = torch.full((m, n), 123.0, device="cuda")
    ops.nvfp4_gemm_tile(w.codes, w.scales, xc, xs, m, n, k, 0, y)
    ref, l1 = oracle.nvfp4_gemm(wc, ws, n, k, xc.cpu().numpy(), xs.cpu().numpy(), m)
    _close(y.cpu().numpy(), ref, l1, f"nvfp4 gemm m={m}")


def test_gemm_tile_row_start(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k, m = 384, 1024, 40
    w, wc, ws = _weight(torch, n, k, 5)
    x = _input(m, k, 3)
    xc, xs = ops.pack_nvfp4(_dev(torch, x.view(np.int16)), m, k)
    full = torch.empty(m, n, device="cuda")
    ops.nvfp4_gemm_tile(w.codes, w.scales, xc, xs, m, n, k, 0, full)
    tile = torch.empty(m, 136, device="cuda")
    ops.nvfp4_gemm_tile(w.codes, w.scales, xc, xs, m, 136, k, 128, tile)
    assert torch.equal(tile, full[:, 128:264])


@pytest.mark.parametrize("m", [1, 2, 77, 256])
def test_project_epilogues(torch_gpu, m):
    """Fused prefill epilogues equal the raw tile (cuda/prefill.cu:116-134)."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 136, 5120
    w, wc, ws = _weight(torch, n, k, 27)
    x = _dev(torch, _input(m, k, 13).view(np.int16))
    work = torch.empty(ops.nvfp4_workspace_bytes(m), dtype=torch.uint8, device="cuda")
    xc, xs = ops.pack_nvfp4(x, m, k)
    raw = torch.empty(m, n, device="cuda")
    ops.nvfp4_gemm_tile(w.codes, w.scales, xc, xs, m, n, k, 0, raw)
    rawv = raw.cpu().numpy()
    y = torch.full((m + 1, n), 123.0, device="cuda")
    ops.nvfp4_project(w, x, m, y, work)
    yv = y.cpu().numpy()
    assert np.array_equal(yv[:m], rawv) and np.all(yv[m] == 123.0), "logical output guard"
    yb = torch.empty(m, n, dtype=torch.int16, device="cuda")
    ops.nvfp4_project(w, x, m, yb, work, epilogue=ops.DECODE_STORE_BF16)
    assert np.array_equal(yb.cpu().numpy().view(np.uint16), oracle.fp32_to_bf16(rawv))
    res = np.linspace(-2, 2, m * n, dtype=np.float32).reshape(m, n)
    yr = torch.empty(m, n, device="cuda")
    ops.nvfp4_project(w, x, m, yr, work, epilogue=ops.DECODE_RESIDUAL_ADD_FP32, residual=_dev(torch, res))
    assert np.array_equal(yr.cpu().numpy(), res + rawv)
    if m <= 2:  # native M=1/M=2 handoff: token 0 identical (tests/nvfp4_test.cpp:199-202)
        y1 = torch.empty(1, n, device="cuda")
        ops.nvfp4_project(w, x, 1, y1, work)
        assert np.array_equal(y1.cpu().numpy()[0], rawv[0])


def test_paired_swiglu(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 136, 5120
    wa, _, _ = _weight(torch, n, k, 4)
    wb, _, _ = _weight(torch, n, k, 29)
    for m in (1, 2, 3, 200):
        x = _dev(torch, _input(m, k, 13).view(np.int16))
        work = torch.empty(ops.nvfp4_workspace_bytes(m), dtype=torch.uint8, device="cuda")
        g = torch.empty(m, n, device="cuda")
        u = torch.empty(m, n, device="cuda")
        ops.nvfp4_project(wa, x, m, g, work)
        ops.nvfp4_project(wb, x, m, u, work)
        sw = torch.empty(m, n, dtype=torch.int16, device="cuda")
        ops.nvfp4_paired_swiglu(wa, wb, x, sw, m, work)
        gv, uv = g.cpu().numpy().astype(np.float64), u.cpu().numpy().astype(np.float64)
        e = np.exp(-np.abs(gv))  # never overflows; logistic(gv) on both signs
        sig = np.where(gv >= 0, 1 / (1 + e), e / (1 + e))
        want = oracle.bf16_to_fp32(oracle.fp32_to_bf16((gv * sig * uv).astype(np.float32)))
        got = oracle.bf16_to_fp32(sw.cpu().numpy().view(np.uint16))
        assert np.all(np.isfinite(got))
        assert np.all(np.abs(got - want) <= .008 * np.abs(want) + .001), f"paired SwiGLU m={m}"


def test_decode_single_paired_and_ranges(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 136, 5120
    wa, ca, sa = _weight(torch, n, k, 4)
    wb, cb, sb = _weight(torch, n, k, 29)
    xv = _input(1, k, 13)[0]
    x = _dev(torch, xv.view(np.int16))
    ref_a, l1_a = oracle.nvfp4_gemv(ca, sa, n, k, xv, k)
    ref_b, l1_b = oracle.nvfp4_gemv(cb, sb, n, k, xv, k)
    ya = torch.empty(n, device="cuda")
    ops.decode_mmv(ops.nvfp4_decode_desc(wa, x, ya))
    yav = ya.cpu().numpy()
    _close(yav, ref_a, l1_a, "nvfp4 decode")
    yb16 = torch.empty(n, dtype=torch.int16, device="cuda")
    ops.decode_mmv(ops.nvfp4_decode_desc(wa, x, yb16, ops.DECODE_STORE_BF16))
    assert np.array_equal(yb16.cpu().numpy().view(np.uint16), oracle.fp32_to_bf16(yav))
    res = np.linspace(-1, 1, n, dtype=np.float32)
    r = _dev(torch, res)
    ops.decode_mmv(ops.nvfp4_decode_desc(wa, x, None, ops.DECODE_RESIDUAL_ADD_FP32, residual=r))
    assert np.array_equal(r.cpu().numpy(), res + yav)
    # paired: both epilogues, and SwiGLU
    o1, o2 = torch.empty(n, device="cuda"), torch.empty(n, device="cuda")
    ops.decode_mmv_paired(ops.nvfp4_decode_desc(wa, x, o1), ops.nvfp4_decode_desc(wb, x, o2))
    assert np.array_equal(o1.cpu().numpy(), yav)
    _close(o2.cpu().numpy(), ref_b, l1_b, "nvfp4 paired decode")
    sw = torch.empty(n, dtype=torch.int16, device="cuda")
    ops.decode_mmv_paired(ops.nvfp4_decode_desc(wa, x, sw, ops.DECODE_SWIGLU_BF16),
                          ops.nvfp4_decode_desc(wb, x, None, ops.DECODE_SWIGLU_BF16))
    g, u = yav.astype(np.float64), o2.cpu().numpy().astype(np.float64)
    e = np.exp(-np.abs(g))
    sig = np.where(g >= 0, 1 / (1 + e), e / (1 + e))
    want = oracle.bf16_to_fp32(oracle.fp32_to_bf16((g * sig * u).astype(np.float32)))
    got = oracle.bf16_to_fp32(sw.cpu().numpy().view(np.uint16))
    assert np.all(np.abs(got - want) <= .008 * np.abs(want) + .001)
    # ranged launches reject NVFP4 before any write (tests/nvfp4_test.cpp:236-244)
    s1 = torch.full((n,), 0x3F80, dtype=torch.int16, device="cuda")
    s2 = torch.full((n,), 0x3F80, dtype=torch.int16, device="cuda")
    with pytest.raises(Exception):
        ops.decode_mmv_ranges([ops.nvfp4_decode_desc(wa, x, s1, ops.DECODE_STORE_BF16),
                               ops.nvfp4_decode_desc(wb, x, s2, ops.DECODE_STORE_BF16)])
    torch.cuda.synchronize()
    assert torch.all(s1 == 0x3F80) and torch.all(s2 == 0x3F80)


def test_decode_head_shape(torch_gpu):
    """A head-class N with K = 5120 (n not a multiple of 128)."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 4104, 5120
    w, wc, ws = _weight(torch, n, k, 11)
    xv = _input(1, k, 9)[0]
    y = torch.empty(n, device="cuda")
    ops.decode_mmv(ops.nvfp4_decode_desc(w, _dev(torch, xv.view(np.int16)), y))
    rows = np.arange(0, n, 37)
    ref, l1 = oracle.nvfp4_gemv(wc, ws, n, k, xv, k)
    _close(y.cpu().numpy()[rows], ref[rows], l1[rows], "nvfp4 head decode")


def test_mlp_nvfp4_equals_stages(torch_gpu):
    """PrefillEngine::mlp with NVFP4 gate/up (cuda/prefill.cu:766-779) equals
    RMS -> BF16, paired NVFP4 SwiGLU, Q4_K down + residual, bit for bit."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    m = 5
    rng = np.random.Generator(np.random.PCG64(12))
    print("nvfp4 mlp: building weights", flush=True)
    gc = rng.integers(0, 256, (17408, 2560), dtype=np.uint8)
    us = rng.integers(0, 256, (17408, 2560), dtype=np.uint8)
    sfg = rng.integers(24, 60, 256 + 17408 * 320, dtype=np.uint8)
    sfu = rng.integers(24, 60, 256 + 17408 * 320, dtype=np.uint8)
    for sf in (sfg, sfu):
        sf[:256] = 0
        sf[:4] = np.array([2.0 ** -6], np.float32).view(np.uint8)
    gate = ops.nvfp4_weight(_dev(torch, gc), _dev(torch, sfg), 17408, 5120)
    up = ops.nvfp4_weight(_dev(torch, us), _dev(torch, sfu), 17408, 5120)
    down_codes = rng.integers(0, 256, ops.code_bytes(0x020D, 5120, 17408), dtype=np.uint8)
    down_meta = np.zeros(ops.scale_bytes(0x020D, 5120, 17408), np.uint8).reshape(-1, 16)
    down_meta[:, 0:2] = np.array([0x1400], np.uint16).view(np.uint8)   # d = 2^-10
    down_meta[:, 2:4] = np.array([0x1000], np.uint16).view(np.uint8)   # dmin = 2^-11
    down_meta[:, 4:16] = rng.integers(0, 256, (down_meta.shape[0], 12), dtype=np.uint8)
    down = ops.PrefillWeight(_dev(torch, down_codes), _dev(torch, down_meta.ravel()), 0x020D, 0x0105,
                             5120, 17408, 5120, 17408)
    h = (rng.standard_normal((m, 5120)) * 2).astype(np.float32)
    gamma = oracle.fp32_to_bf16((rng.standard_normal(5120) * .1).astype(np.float32))
    dh, dg = _dev(torch, h), _dev(torch, gamma.view(np.int16))
    ws = torch.empty(ops.prefill_mlp_workspace_bytes(m), dtype=torch.uint8, device="cuda")
    out = torch.empty(m, 5120, device="cuda")
    print("nvfp4 mlp: fused", flush=True)
    ops.prefill_mlp(gate, up, down, dh, dg, 1e-6, out, m, ws)
    print("nvfp4 mlp: stages", flush=True)
    bf = torch.empty(m, 5120, dtype=torch.int16, device="cuda")
    ops.hidden_rms_bf16(dh, dg, 1e-6, m, bf)
    work = torch.empty(ops.nvfp4_workspace_bytes(m), dtype=torch.uint8, device="cuda")
    sw = torch.empty(m, 17408, dtype=torch.int16, device="cuda")
    ops.nvfp4_paired_swiglu(gate, up, bf, sw, m, work)
    out2 = torch.empty(m, 5120, device="cuda")
    ops.prefill_project(down, sw, m, out2, ops.DECODE_RESIDUAL_ADD_FP32, residual=dh)
    assert torch.all(torch.isfinite(out))
    assert torch.equal(out, out2)
