"""Fused producers and the whole Q8 MLP (cuda/q4k_q8.cu:347-398) on the GPU:
RMS->Q8 and SwiGLU->Q8 are bit-exact against the oracle; the MLP output is
checked against the oracle chain; failure semantics follow the reference
(typed error on a nonfinite producer, submitted flag, deferred pending flag,
no device allocation inside the call)."""
import numpy as np
import pytest

import oracle
from _fix import normal, random_q4k, random_q6k

pytestmark = pytest.mark.gpu


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def test_rms_q8_bit_exact(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    for m in (1, 3, 17):
        res = (normal((m, 5120), 10 + m) * 3).astype(np.float32)
        res[0, :7] = 0
        if m > 2:
            res[2] = 0.0  # all-zero row: scale 1 path
        gamma = oracle.fp32_to_bf16(normal(5120, 20, 0.1))
        q = ops.Q8Input.empty(m, 5120)
        flag = torch.zeros(1, dtype=torch.int32, device="cuda")
        ops.hidden_rms_q8(_dev(torch, res), _dev(torch, gamma.view(np.int16)), 1e-6, m, q, flag)
        torch.cuda.synchronize()
        ref, _ = oracle.rms_q8(res, gamma, 1e-6)
        assert int(flag.item()) == 0
        assert np.array_equal(q.codes.cpu().numpy(), ref.codes)
        assert np.array_equal(q.scales.cpu().numpy().view(np.uint32), ref.scales.view(np.uint32))
        assert np.array_equal(q.sums.cpu().numpy(), ref.sums)
    res[1, 100] = np.nan
    ops.hidden_rms_q8(_dev(torch, res), _dev(torch, gamma.view(np.int16)), 1e-6, m, q, flag)
    torch.cuda.synchronize()
    assert int(flag.item()) == 1


def test_swiglu_q8_bit_exact(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    m, n = 5, 17408
    g = (normal((m, n), 30) * 5).astype(np.float32)
    u = normal((m, n), 31)
    g[0, :4] = [0.0, -120.0, 95.0, 1e-30]  # exp overflow / underflow / tiny
    q = ops.Q8Input.empty(m, n)
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    ops.swiglu_q8(_dev(torch, g), _dev(torch, u), m, n, q, flag)
    torch.cuda.synchronize()
    ref, _ = oracle.swiglu_q8(g, u)
    assert int(flag.item()) == 0
    assert np.array_equal(q.codes.cpu().numpy(), ref.codes)
    assert np.array_equal(q.scales.cpu().numpy().view(np.uint32), ref.scales.view(np.uint32))
    assert np.array_equal(q.sums.cpu().numpy(), ref.sums)
    g[3, 5000] = np.inf
    ops.swiglu_q8(_dev(torch, g), _dev(torch, u), m, n, q, flag)
    torch.cuda.synchronize()
    assert int(flag.item()) == 1


@pytest.fixture(scope="module")
def mlp_weights(torch_gpu):
    import qw38_amd.ops as ops
    out = {}
    gl = random_q4k(17408, 5120, 41)
    ul = random_q4k(17408, 5120, 42)
    dl4 = random_q4k(5120, 17408, 43)
    dl6 = random_q6k(5120, 17408, 44)
    for name, wl, layout in (("gate", gl, oracle.LAYOUT_Q4K_W64), ("up", ul, oracle.LAYOUT_Q4K_W64),
                             ("down4", dl4, oracle.LAYOUT_Q4K_SEQ)):
        co, mo = wl.physical(layout)
        out[name] = (ops.PrefillWeight.from_bytes(co, mo, layout, wl.n, wl.k), wl)
    co, mo = dl6.physical()
    out["down6"] = (ops.PrefillWeight.from_bytes(co, mo, oracle.LAYOUT_Q6K_W64, 5120, 17408), dl6)
    return out


def _workspace_views(ws, m):
    """The reference workspace layout (cuda/q4k_q8.cu:367-372): Q8 codes
    [m][17408], scales/sums [m][544], gate and up fp32 [m][17408]."""
    b = ws.cpu().numpy()
    o = 0
    codes = b[o:o + m * 17408].view(np.int8).reshape(m, 17408); o += m * 17408
    scales = b[o:o + m * 544 * 4].view(np.float32).reshape(m, 544); o += m * 544 * 4
    sums = b[o:o + m * 544 * 4].view(np.int32).reshape(m, 544); o += m * 544 * 4
    g = b[o:o + m * 17408 * 4].view(np.float32).reshape(m, 17408); o += m * 17408 * 4
    u = b[o:o + m * 17408 * 4].view(np.float32).reshape(m, 17408)
    return codes, scales, sums, g, u


@pytest.mark.parametrize("down", ["down4", "down6"])
def test_q8_mlp_end_to_end(torch_gpu, mlp_weights, down):
    """Stage by stage on the same inputs: RMS->Q8 pack (bit-exact, checked in
    test_rms_q8_bit_exact), gate/up projections (tolerance), the SwiGLU->Q8
    pack of the device's own gate/up values (bit-exact), down + residual
    (tolerance)."""
    torch = torch_gpu
    import qw38_amd
    import qw38_amd.ops as ops
    gate, gl = mlp_weights["gate"]
    up, ul = mlp_weights["up"]
    dn, dl = mlp_weights[down]
    gamma = oracle.fp32_to_bf16(normal(5120, 50, 0.1))
    for m in (1, 3, 129):
        print(f"mlp {down} m={m}", flush=True)
        res = normal((m, 5120), 60 + m)
        ws = torch.zeros(ops.q8_mlp_workspace_bytes(m), dtype=torch.uint8, device="cuda")
        out = torch.full((m, 5120), float("nan"), device="cuda")
        dres, dgam = _dev(torch, res), _dev(torch, gamma.view(np.int16))
        before = qw38_amd.lib().qw38_malloc_count()
        assert ops.q4k_q8_mlp(gate, up, dn, dres, dgam, 1e-6, out, m, ws)
        assert qw38_amd.lib().qw38_malloc_count() == before, "no allocation on the hot path"
        y = out.cpu().numpy()
        codes, scales, sums, g, u = _workspace_views(ws, m)
        q1, _ = oracle.rms_q8(res, gamma, 1e-6)
        if m > 8:
            # the fused gate+up launch writes no FP32 slabs: take the device's
            # own projections of the same (bit-exact) RMS->Q8 operand
            qx = ops.Q8Input.empty(m, 5120)
            flag = torch.zeros(1, dtype=torch.int32, device="cuda")
            ops.hidden_rms_q8(dres, dgam, 1e-6, m, qx, flag)
            gd = torch.empty(m, 17408, device="cuda")
            ud = torch.empty(m, 17408, device="cuda")
            ops.q4k_q8_project(gate, qx, gd)
            ops.q4k_q8_project(up, qx, ud)
            torch.cuda.synchronize()
            g, u = gd.cpu().numpy(), ud.cpu().numpy()
        g64, _, _ = oracle.q4k_q8_contract(gl, q1)
        u64, _, _ = oracle.q4k_q8_contract(ul, q1)
        for name, dev, ref in (("gate", g, g64), ("up", u, u64)):
            ok, ma, mr = oracle.parity_ok(dev, ref)
            print(f"  {name}: max_abs/rms={ma:.3g} mean_rel={mr:.3g}", flush=True)
            assert ok
        q2, _ = oracle.swiglu_q8(g, u)
        assert np.array_equal(codes, q2.codes), "SwiGLU->Q8 pack of the device gate/up"
        assert np.array_equal(scales.view(np.uint32), q2.scales.view(np.uint32))
        assert np.array_equal(sums, q2.sums)
        if isinstance(dl, oracle.Q6K):
            d64, _, _ = oracle.q6k_q8_contract(dl, q2)
        else:
            d64, _, _ = oracle.q4k_q8_contract(dl, q2)
        ok, ma, mr = oracle.parity_ok(y - res, d64)
        print(f"  down: max_abs/rms={ma:.3g} mean_rel={mr:.3g}", flush=True)
        assert ok


def test_q8_mlp_failure_semantics(torch_gpu, mlp_weights):
    torch = torch_gpu
    import qw38_amd.ops as ops
    from qw38_amd import Qw38Error
    gate, _ = mlp_weights["gate"]
    up, _ = mlp_weights["up"]
    dn, _ = mlp_weights["down4"]
    m = 2
    gamma = oracle.fp32_to_bf16(normal(5120, 50, 0.1))
    res = normal((m, 5120), 70)
    res[1, 9] = np.nan
    ws = torch.zeros(ops.q8_mlp_workspace_bytes(m), dtype=torch.uint8, device="cuda")
    out = torch.zeros(m, 5120, device="cuda")
    dres, dgam = _dev(torch, res), _dev(torch, gamma.view(np.int16))
    with pytest.raises(Qw38Error) as e:
        ops.q4k_q8_mlp(gate, up, dn, dres, dgam, 1e-6, out, m, ws)
    assert e.value.operation == "q8.producer" and e.value.status == 2
    assert e.value.submitted
    # internal submission: enqueue only, sticky flag read by the owner
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    assert ops.q4k_q8_mlp(gate, up, dn, dres, dgam, 1e-6, out, m, ws, pending_failure=flag)
    torch.cuda.synchronize()
    assert int(flag.item()) == 1
    # prelaunch rejection: bad eps, short workspace
    with pytest.raises(Qw38Error) as e:
        ops.q4k_q8_mlp(gate, up, dn, dres, dgam, -1.0, out, m, ws)
    assert not e.value.submitted
    with pytest.raises(Qw38Error):
        ops.q4k_q8_mlp(gate, up, dn, dres, dgam, 1e-6, out, m, ws[:-8])


@pytest.mark.parametrize("layout", [oracle.LAYOUT_Q4K_W64, oracle.LAYOUT_Q4K_SEQ])
def test_gate_up_swiglu_fused_bitwise(torch_gpu, mlp_weights, layout):
    """The fused gate+up launch (SwiGLU->Q8 in the projection's epilogue)
    equals the unfused chain -- two projections, then the oracle-pinned
    SwiGLU->Q8 pack -- bit for bit: the decode kernel at m = 1 on 0x020D, and
    the MMQ at m > 24 covering every tile shape and the big-tile + tail split; a
    group whose input scale is NaN is flagged in both."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    _, gl = mlp_weights["gate"]
    _, ul = mlp_weights["up"]
    gate = ops.PrefillWeight.from_bytes(*gl.physical(layout), layout, gl.n, gl.k)
    up = ops.PrefillWeight.from_bytes(*ul.physical(layout), layout, ul.n, ul.k)
    gamma = oracle.fp32_to_bf16(normal(5120, 80, 0.1))
    dgam = _dev(torch, gamma.view(np.int16))
    # m = 1 on 0x020D: the streaming-GEMV family (fused: one wave per strip,
    # unfused: four waves split K); m > 24: the MMQ family on both sides (at
    # m = 9..24 an unfused projection may run as batched-decode passes, a
    # different family, while the fused launch stays on the MMQ)
    ms = ((1,) if layout == oracle.LAYOUT_Q4K_SEQ else ()) + (25, 40, 64, 130, 512)
    for m in ms:
        print(f"gate_up layout=0x{layout:04x} m={m}", flush=True)
        res = normal((m, 5120), 90 + m) * 2
        qx = ops.Q8Input.empty(m, 5120)
        flag = torch.zeros(1, dtype=torch.int32, device="cuda")
        ops.hidden_rms_q8(_dev(torch, res), dgam, 1e-6, m, qx, flag)
        if m >= 40:
            qx.scales.view(m, 160)[m - 3, 17] = float("nan")
        gd = torch.empty(m, 17408, device="cuda")
        ud = torch.empty(m, 17408, device="cuda")
        ops.q4k_q8_project(gate, qx, gd)
        ops.q4k_q8_project(up, qx, ud)
        ref = ops.Q8Input.empty(m, 17408)
        rflag = torch.zeros(1, dtype=torch.int32, device="cuda")
        ops.swiglu_q8(gd, ud, m, 17408, ref, rflag)
        out = ops.Q8Input.empty(m, 17408)
        out.codes.fill_(55)
        out.scales.fill_(7.0)
        out.sums.fill_(-1)
        fflag = torch.zeros(1, dtype=torch.int32, device="cuda")
        ops.q4k_q8_gate_up_swiglu(gate, up, qx, out, fflag)
        torch.cuda.synchronize()
        assert int(fflag.item()) == int(rflag.item()) == (1 if m >= 40 else 0)
        assert torch.equal(out.codes, ref.codes)
        assert torch.equal(out.scales.view(torch.int32), ref.scales.view(torch.int32))
        assert torch.equal(out.sums, ref.sums)
        if m == 40:  # the fused launch's small-M tiles (m = 9): its rows are the m = 40 rows
            q9 = ops.Q8Input.empty(9, 5120)
            q9.codes.copy_(qx.codes[:9]); q9.scales.copy_(qx.scales[:9]); q9.sums.copy_(qx.sums[:9])
            o9 = ops.Q8Input.empty(9, 17408)
            f9 = torch.zeros(1, dtype=torch.int32, device="cuda")
            ops.q4k_q8_gate_up_swiglu(gate, up, q9, o9, f9)
            torch.cuda.synchronize()
            assert int(f9.item()) == 0
            assert torch.equal(o9.codes, out.codes[:9])
            assert torch.equal(o9.scales.view(torch.int32), out.scales[:9].view(torch.int32))
            assert torch.equal(o9.sums, out.sums[:9])


def test_gate_up_swiglu_rejections(torch_gpu, mlp_weights):
    torch = torch_gpu
    import qw38_amd.ops as ops
    from qw38_amd import Qw38Error
    gate, _ = mlp_weights["gate"]
    up, _ = mlp_weights["up"]
    dn6, _ = mlp_weights["down6"]
    qx = ops.Q8Input.empty(16, 5120)
    out = ops.Q8Input.empty(16, 17408)
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    with pytest.raises(Qw38Error):  # Q6_K gate
        ops.q4k_q8_gate_up_swiglu(dn6, up, qx, out, flag)
    with pytest.raises(Qw38Error):  # output token count mismatch
        ops.q4k_q8_gate_up_swiglu(gate, up, qx, ops.Q8Input.empty(8, 17408), flag)
    with pytest.raises(Qw38Error):  # failure flag length
        ops.q4k_q8_gate_up_swiglu(gate, up, qx, out, torch.zeros(2, dtype=torch.int32, device="cuda"))


@pytest.mark.parametrize("down", ["down4", "down6"])
def test_q8_mlp_m1_fused_equals_chain(torch_gpu, mlp_weights, down):
    """M = 1 on 0x020D runs the RMS->Q8 producer, then gate, up and SwiGLU->Q8
    as ONE streaming launch, then down + residual. The output and the down
    operand equal the unfused chain of separate entry points bit for bit; a
    NaN in the residual raises the flag."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    from qw38_amd import Qw38Error
    _, gl = mlp_weights["gate"]
    _, ul = mlp_weights["up"]
    seq = oracle.LAYOUT_Q4K_SEQ
    gate = ops.PrefillWeight.from_bytes(*gl.physical(seq), seq, gl.n, gl.k)
    up = ops.PrefillWeight.from_bytes(*ul.physical(seq), seq, ul.n, ul.k)
    dn, _ = mlp_weights[down]
    gamma = oracle.fp32_to_bf16(normal(5120, 110, 0.1))
    dgam = _dev(torch, gamma.view(np.int16))
    for seed in (111, 112):
        res = _dev(torch, normal((1, 5120), seed) * 3)
        ws = torch.zeros(ops.q8_mlp_workspace_bytes(1), dtype=torch.uint8, device="cuda")
        out = torch.empty(1, 5120, device="cuda")
        ops.q4k_q8_mlp(gate, up, dn, res, dgam, 1e-6, out, 1, ws)
        qx = ops.Q8Input.empty(1, 5120)
        flag = torch.zeros(1, dtype=torch.int32, device="cuda")
        ops.hidden_rms_q8(res, dgam, 1e-6, 1, qx, flag)
        gd = torch.empty(1, 17408, device="cuda")
        ud = torch.empty(1, 17408, device="cuda")
        ops.q4k_q8_project(gate, qx, gd)
        ops.q4k_q8_project(up, qx, ud)
        qh = ops.Q8Input.empty(1, 17408)
        ops.swiglu_q8(gd, ud, 1, 17408, qh, flag)
        ref = torch.empty(1, 5120, device="cuda")
        ops.q4k_q8_project(dn, qh, ref, residual=res)
        torch.cuda.synchronize()
        assert int(flag.item()) == 0
        codes, scales, sums, _, _ = _workspace_views(ws, 1)
        assert np.array_equal(codes, qh.codes.cpu().numpy())
        assert np.array_equal(scales.view(np.uint32), qh.scales.cpu().numpy().view(np.uint32))
        assert np.array_equal(sums, qh.sums.cpu().numpy())
        assert torch.equal(out, ref)
    bad = res.clone()
    bad[0, 4000] = float("nan")
    with pytest.raises(Qw38Error) as e:
        ops.q4k_q8_mlp(gate, up, dn, bad, dgam, 1e-6, out, 1, ws)
    assert e.value.operation == "q8.producer"
    # the next call clears the flag again (at M=1 the RMS->Q8 launch does it)
    again = torch.empty(1, 5120, device="cuda")
    ops.q4k_q8_mlp(gate, up, dn, res, dgam, 1e-6, again, 1, ws)
    torch.cuda.synchronize()
    assert torch.equal(again, ref)
