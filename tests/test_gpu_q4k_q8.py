"""GPU parity for pack_q8 and q4k_q8_project, mirroring the reference's
tests/q4k_q8_test.cpp (odd shape N=137, K=259; m sweep; ties/saturation/zero
token/padding; aligned vs unaligned loads with guard words; schedule
invariance; reuse; truncated-span and nonfinite rejection). All calls go
through the C-ABI of libqw38_hip.so; the oracle is the checker only."""
import numpy as np
import pytest

import oracle
from _fix import REF_K, REF_N, ref_fixture_input, ref_fixture_weight

pytestmark = pytest.mark.gpu

M_SWEEP = [1, 2, 3, 5, 8, 9, 16, 17, 31, 32, 33, 64, 65, 127, 128, 129, 256, 257, 511, 512]
LAYOUTS = [oracle.LAYOUT_Q4K_SEQ, oracle.LAYOUT_Q4K_W64]


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _np(t):
    return t.cpu().numpy()


def independent_pack(bf16, m, k):
    """tests/q4k_q8_test.cpp:83-92 restated in numpy (not the C oracle)."""
    pk = oracle.pad256(k)
    x = np.zeros((m, pk), np.float32)
    x[:, :k] = oracle.bf16_to_fp32(bf16).reshape(m, k)
    g = x.reshape(m, pk // 32, 32)
    peak = np.abs(g).max(axis=2)
    a = np.where(peak == 0, np.float32(1), peak / np.float32(127)).astype(np.float32)
    z = np.clip(np.rint(g / a[:, :, None]), -127, 127).astype(np.int32)
    return z.reshape(m, pk).astype(np.int8), a, z.sum(axis=2).astype(np.int32)


@pytest.fixture(scope="module")
def weights(torch_gpu):
    w = ref_fixture_weight()
    out = {}
    import qw38_amd.ops as ops
    for layout in LAYOUTS:
        co, mo = w.physical(layout)
        out[layout] = ops.PrefillWeight.from_bytes(co, mo, layout, REF_N, REF_K)
    return w, out


def test_pack_bit_exact_and_edge_cases(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    for m in [1, 3, 33, 129, 512]:
        print(f"pack m={m}", flush=True)
        x = ref_fixture_input(m)
        dx = _dev(torch, x.view(np.int16))
        q = ops.Q8Input.empty(m, REF_K)
        flag = torch.zeros(1, dtype=torch.int32, device="cuda")
        ops.pack_q8(dx, q, flag)
        torch.cuda.synchronize()
        assert int(flag.item()) == 0
        z, a, s = _np(q.codes), _np(q.scales), _np(q.sums)
        rz, ra, rs = independent_pack(x, m, REF_K)
        assert np.array_equal(z, rz), "exact independent codes, RNE and padding"
        assert np.array_equal(a.view(np.uint32), ra.view(np.uint32)), "exact scales"
        assert np.array_equal(s, rs), "exact sums"
        assert np.abs(s).max() <= 32 * 127
        ob = oracle.pack_q8(x, m, REF_K)
        assert np.array_equal(z, ob.codes) and np.array_equal(s, ob.sums)
        assert np.array_equal(a.view(np.uint32), ob.scales.view(np.uint32))
        assert list(z[0, :5]) == [127, 0, 2, 0, -2], "halfway ties and saturation endpoint"
        if m > 2:
            assert s[2].sum() == 0 and np.all(z[2] == 0), "whole zero token"
        assert s[0, 2] < 0, "negative activation sum fixture"


def test_pack_nonfinite_rejected(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    m = 3
    x = ref_fixture_input(m)
    for bits in (0x7F80, 0xFF80, 0x7FC0):
        xb = x.copy()
        xb[0, 0] = bits
        q = ops.Q8Input.empty(m, REF_K)
        flag = torch.zeros(1, dtype=torch.int32, device="cuda")
        ops.pack_q8(_dev(torch, xb.view(np.int16)), q, flag)
        torch.cuda.synchronize()
        assert int(flag.item()) == 1
        sc = _np(q.scales)
        assert np.isnan(sc[0, 0]), "nonfinite pack rejected with NaN scale, not finite zero"
        assert np.all(_np(q.codes)[0, :32] == 0)
        assert np.all(np.isfinite(sc[1:])), "other groups unaffected"


@pytest.mark.parametrize("layout", LAYOUTS, ids=["020D", "0240"])
def test_project_m_sweep(torch_gpu, weights, layout):
    torch = torch_gpu
    import qw38_amd.ops as ops
    wl, wd = weights
    w = wd[layout]
    mmq_prev = {}
    gemv_first = {}
    for m in M_SWEEP:
        print(f"project layout={layout:#x} m={m}", flush=True)
        x = ref_fixture_input(m)
        q = ops.Q8Input.empty(m, REF_K)
        flag = torch.zeros(1, dtype=torch.int32, device="cuda")
        ops.pack_q8(_dev(torch, x.view(np.int16)), q, flag)
        out = torch.full((m, REF_N), float("nan"), device="cuda")
        ops.q4k_q8_project(w, q, out)
        torch.cuda.synchronize()
        y = _np(out)
        ob = oracle.pack_q8(x, m, REF_K)
        ref64, _, dots = oracle.q4k_q8_contract(wl, ob, want_dots=True)
        assert np.abs(dots).max() <= 32 * 15 * 127, "raw dot bound"
        # reference tolerance (tests/q4k_q8_test.cpp:129)
        assert np.all(np.isfinite(y))
        bad = np.abs(y - ref64) > 0.02 + 0.002 * np.abs(ref64)
        assert not bad.any(), f"m={m}: affine contraction off at {np.argwhere(bad)[:5]}"
        ok, ma, mr = oracle.parity_ok(y, ref64)
        assert ok, f"m={m}: max_abs/rms={ma:.3g} mean_rel={mr:.3g}"
        # reuse: identical sibling output, pack untouched
        out2 = torch.empty_like(out)
        ops.q4k_q8_project(w, q, out2)
        torch.cuda.synchronize()
        assert np.array_equal(_np(out2).view(np.uint32), y.view(np.uint32))
        assert np.array_equal(_np(q.codes), ob.codes)
        # schedule invariance within the MMQ tilings (J32 == J128 analogue):
        # every token row must equal the same row computed at any other M > 8.
        if m > 8:
            for pm, py in mmq_prev.items():
                t = min(pm, m)
                assert np.array_equal(py[:t].view(np.uint32), y[:t].view(np.uint32)), \
                    f"MMQ tiles m={pm} and m={m} disagree bitwise"
            mmq_prev[m] = y
        else:
            # Batched GEMV: token 0 equals the same kernel family's first result
            # bitwise. 0x020D: M=1 streams the strip linearly, M=2..8 run the
            # int8-MFMA kernel (T=4 and T=8 share one operation order per
            # (row, token)); 0x0240: M <= 2 and 3..8.
            fam = 0 if (m == 1 if layout == oracle.LAYOUT_Q4K_SEQ else m <= 2) else 1
            if fam not in gemv_first:
                gemv_first[fam] = y[0].copy()
            assert np.array_equal(gemv_first[fam].view(np.uint32), y[0].view(np.uint32))


def test_unaligned_and_residual_guards(torch_gpu, weights):
    """tests/q4k_q8_test.cpp:96-117: 4-byte aligned code spans and Q8 codes
    match the aligned path exactly; residual added; row-tail guard words."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    wl, wd = weights
    layout = oracle.LAYOUT_Q4K_SEQ
    w = wd[layout]
    m = 1
    x = ref_fixture_input(m)
    q = ops.Q8Input.empty(m, REF_K)
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    ops.pack_q8(_dev(torch, x.view(np.int16)), q, flag)
    out = torch.empty(m, REF_N, device="cuda")
    ops.q4k_q8_project(w, q, out)
    torch.cuda.synchronize()
    y = _np(out)[0]
    co, mo = wl.physical(layout)
    shifted_w = np.zeros(co.size + 8, np.uint8)
    shifted_w[4:4 + co.size] = co
    dshift_w = _dev(torch, shifted_w)
    z = _np(q.codes)[0]
    shifted_q = np.full(z.size + 8, 99, np.int8)
    shifted_q[4:4 + z.size] = z
    dshift_q = _dev(torch, shifted_q)
    residual = ((np.arange(REF_N) % 17).astype(np.float32) - 8) * 0.125
    dres = _dev(torch, residual)
    for variant in range(4):
        print(f"unaligned variant={variant}", flush=True)
        guards = torch.full((REF_N + 2,), -12345.0, device="cuda")
        wv = ops.PrefillWeight(w.codes, w.scales, w.layout, w.quantizer, w.n, w.k, w.padded_n,
                               w.padded_k, w.codes_bytes, w.scales_bytes)
        if variant & 1:
            wv.codes = dshift_w
            wv.codes_ptr = dshift_w.data_ptr() + 4
        qv = ops.Q8Input(q.codes, q.scales, q.sums, q.m, q.k, q.padded_k)
        if variant & 2:
            qv.codes = dshift_q
            qv.codes_ptr = dshift_q.data_ptr() + 4
            qv.codes_len = z.size
        ops.q4k_q8_project(wv, qv, guards, residual=dres,
                           output_ptr=guards.data_ptr() + 4, output_len=REF_N)
        torch.cuda.synchronize()
        r = _np(guards)
        assert np.array_equal(r[1:-1], (y + residual).astype(np.float32)), \
            "aligned/unaligned Q4 loads and residual exactly agree"
        assert r[0] == -12345.0 and r[-1] == -12345.0, "row-tail output guards"


def test_rejections(torch_gpu, weights):
    torch = torch_gpu
    import qw38_amd.ops as ops
    from qw38_amd import Qw38Error
    _, wd = weights
    w = wd[oracle.LAYOUT_Q4K_SEQ]
    m = 3
    q = ops.Q8Input.empty(m, REF_K)
    out = torch.empty(m, REF_N, device="cuda")
    bad = ops.Q8Input(q.codes, q.scales, q.sums, m, REF_K, q.padded_k, codes_len=1)
    with pytest.raises(Qw38Error) as e:
        ops.q4k_q8_project(w, bad, out)
    assert e.value.status == 2, "truncated input rejected"
    badw = ops.PrefillWeight(w.codes, w.scales, w.layout, w.quantizer, w.n, w.k, w.padded_n,
                             w.padded_k, w.codes_bytes - 1, w.scales_bytes)
    with pytest.raises(Qw38Error):
        ops.q4k_q8_project(badw, q, out)
    with pytest.raises(Qw38Error) as e:  # aliasing output over the codes
        ops.q4k_q8_project(w, q, out, output_ptr=q.codes.data_ptr(), output_len=m * REF_N)
    host = np.zeros(m * REF_N, np.float32)
    with pytest.raises(Qw38Error):  # host memory is not device memory
        ops.q4k_q8_project(w, q, out, output_ptr=host.ctypes.data, output_len=m * REF_N)


def test_group_dots_exact(torch_gpu, weights):
    torch = torch_gpu
    import qw38_amd.ops as ops
    wl, wd = weights
    m = 5
    x = ref_fixture_input(m)
    ob = oracle.pack_q8(x, m, REF_K)
    _, _, rdots = oracle.q4k_q8_contract(wl, ob, want_dots=True)
    for layout in LAYOUTS:
        q = ops.Q8Input(_dev(torch, ob.codes), _dev(torch, ob.scales), _dev(torch, ob.sums),
                        m, REF_K, ob.pk)
        dots = torch.zeros(m * REF_N * (ob.pk // 32), dtype=torch.int32, device="cuda")
        ops.group_dots(wd[layout], q, dots)
        torch.cuda.synchronize()
        assert np.array_equal(_np(dots).reshape(rdots.shape), rdots), "per-group int32 dots"
