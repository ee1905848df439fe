"""GPU parity at the BASELINE.json configurations (configs 1-4) plus the Q6_K
path, against the oracle on the same inputs. Weights are fitted on the GPU by
the library (bit-exactness of that fitter is tested separately) and handed to
the oracle as the same GGML bytes. Tolerance (north star): max|y-ref| <=
1e-3*rms(ref) and mean|y-ref|/mean|ref| <= 1e-5, ref in float64."""
import numpy as np
import pytest

import oracle
from _fix import normal, outlier_rows, random_q6k, silu_rows

pytestmark = pytest.mark.gpu


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _fit_q4k(torch, ops, n, k, seed, layout):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn(n, k, generator=g, device="cuda") * 0.02
    fail = torch.zeros(1, dtype=torch.int32, device="cuda")
    blocks = ops.quantize_q4k_blocks(x, n, k, fail)
    w = ops.upload_q4k_blocks(blocks, n, k, layout=layout)
    torch.cuda.synchronize()
    assert int(fail.item()) == 0
    return w, oracle.Q4K.from_ggml(blocks.cpu().numpy(), n, k)


def _fit_q6k(torch, ops, n, k, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn(n, k, generator=g, device="cuda") * 0.02
    blocks = ops.quantize_q6k_blocks(x, n, k)
    w = ops.upload_q6k_blocks(blocks, n, k)
    torch.cuda.synchronize()
    return w, oracle.Q6K.from_ggml(blocks.cpu().numpy(), n, k)


def _q8(torch, ops, x_f32):
    m, k = x_f32.shape
    bf = oracle.fp32_to_bf16(x_f32)
    q = ops.Q8Input.empty(m, k)
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    ops.pack_q8(_dev(torch, bf.view(np.int16)), q, flag)
    torch.cuda.synchronize()
    assert int(flag.item()) == 0
    ob = oracle.pack_q8(bf, m, k)
    assert np.array_equal(q.codes.cpu().numpy(), ob.codes)
    return q, ob


def _project(torch, ops, w, q, m, n):
    out = torch.full((m, n), float("nan"), device="cuda")
    ops.q4k_q8_project(w, q, out)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _check(y, ref, label):
    ok, ma, mr = oracle.parity_ok(y, ref)
    print(f"{label}: max_abs/rms={ma:.3g} mean_rel={mr:.3g}", flush=True)
    assert ok, f"{label}: max_abs/rms={ma:.3g} mean_rel={mr:.3g}"


@pytest.mark.parametrize("layout", [oracle.LAYOUT_Q4K_SEQ, oracle.LAYOUT_Q4K_W64], ids=["020D", "0240"])
def test_config1_gemv_5120(torch_gpu, layout):
    torch = torch_gpu
    import qw38_amd.ops as ops
    n = k = 5120
    w, wl = _fit_q4k(torch, ops, n, k, 101, layout)
    q, ob = _q8(torch, ops, normal((1, k), 102))
    y = _project(torch, ops, w, q, 1, n)
    ref, _, _ = oracle.q4k_q8_contract(wl, ob)
    _check(y, ref, f"config1 layout={layout:#x}")


@pytest.mark.parametrize("layout", [oracle.LAYOUT_Q4K_SEQ, oracle.LAYOUT_Q4K_W64], ids=["020D", "0240"])
def test_config2_fused_gate_up(torch_gpu, layout):
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 34816, 5120
    w, wl = _fit_q4k(torch, ops, n, k, 201, layout)
    for m in (1, 2, 4, 8):
        q, ob = _q8(torch, ops, outlier_rows(m, k, 202 + m))
        y = _project(torch, ops, w, q, m, n)
        ref, _, _ = oracle.q4k_q8_contract(wl, ob)
        _check(y, ref, f"config2 layout={layout:#x} M={m}")


def test_config3_q6k_down(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 5120, 17408
    w, wl = _fit_q6k(torch, ops, n, k, 301)
    # M=3 runs the M 3..4 ring kernel whose blocks loop over several 16-row
    # tiles at this K (320 tiles on the CUs)
    for m in (1, 2, 3, 8, 40):
        q, ob = _q8(torch, ops, silu_rows(m, k, 302 + m))
        y = _project(torch, ops, w, q, m, n)
        ref, _, _ = oracle.q6k_q8_contract(wl, ob)
        _check(y, ref, f"config3 Q6_K M={m}")


def test_q6k_split_k_rows_independent_of_m(torch_gpu):
    """Q6_K MMQ sums K in fixed segments (four at K = 17408) whatever the
    launch: M <= 128 splits the segments over mmq_kernel blocks and adds them
    in a second kernel (M = 25, 40, 128), M > 128 runs the direct-copy
    160 x 128 tile, one segment per block (M = 256, 512, and 2048 in four
    token chunks). Every token row must be bitwise the same at every M,
    M = 40 matches the oracle, and the split launches must really have run
    split: the library scratch counters show each of them granted (a refused
    request silently takes the no-scratch path, which gives the same bits)."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 5120, 17408
    w, wl = _fit_q6k(torch, ops, n, k, 311)
    xs = silu_rows(2048, k, 312)
    q, ob = _q8(torch, ops, xs)
    full = None
    # 2048 / 512 / 256: direct-copy tile; 40 / 128: 80 x 128 split; 25: the
    # smallest M above the batched-decode passes
    for m in (2048, 512, 40, 128, 256, 25):
        print(f"Q6_K split-K family M={m}", flush=True)
        qm = ops.Q8Input.empty(m, k)
        qm.codes.copy_(q.codes[:m]); qm.scales.copy_(q.scales[:m]); qm.sums.copy_(q.sums[:m])
        res = torch.from_numpy(normal((m, n), 313 + m)).cuda() if m == 128 else None
        y = torch.full((m, n), float("nan"), device="cuda")
        torch.cuda.synchronize()
        before = ops.scratch_stats()
        ops.q4k_q8_project(w, qm, y, residual=res)
        torch.cuda.synchronize()
        after = ops.scratch_stats()
        assert after[0] == before[0] + 1 and after[1:] == before[1:], \
            f"M={m}: split launch did not get the scratch ({before} -> {after})"
        yn = y.cpu().numpy()
        if res is not None:
            want = (full[:m] + res.cpu().numpy()).astype(np.float32)
            assert np.array_equal(yn.view(np.uint32), want.view(np.uint32)), "residual epilogue of the split launch"
        elif full is None:
            full = yn
        else:
            assert np.array_equal(yn.view(np.uint32), full[:m].view(np.uint32)), f"M={m} rows differ from M=512"
        if m == 40:
            ref, _, _ = oracle.q6k_q8_contract(wl, oracle.Q8(ob.codes[:m], ob.scales[:m], ob.sums[:m], m, k, ob.pk))
            _check(yn, ref, "Q6_K split-K M=40")


_Q6_SPLIT_SCRIPT = r"""
import sys, numpy as np, torch
sys.path.insert(0, sys.argv[1]); sys.path.insert(0, sys.argv[1] + "/tests")
import oracle, qw38_amd.ops as ops
from _fix import silu_rows
n, m, out = int(sys.argv[2]), int(sys.argv[3]), sys.argv[4]
k = 17408
g = torch.Generator(device="cuda"); g.manual_seed(341)
x = torch.randn(n, k, generator=g, device="cuda") * 0.02
w = ops.upload_q6k_blocks(ops.quantize_q6k_blocks(x, n, k), n, k)
bf = oracle.fp32_to_bf16(silu_rows(m, k, 342))
q = ops.Q8Input.empty(m, k)
flag = torch.zeros(1, dtype=torch.int32, device="cuda")
ops.pack_q8(torch.from_numpy(bf.view(np.int16)).cuda(), q, flag)
rows = []
for t0 in ((0, 560) if m == 700 else (0, 34)):
    qm = ops.Q8Input.empty(96, k)
    qm.codes.copy_(q.codes[t0:t0 + 96]); qm.scales.copy_(q.scales[t0:t0 + 96]); qm.sums.copy_(q.sums[t0:t0 + 96])
    y = torch.empty(96, n, device="cuda")
    ops.q4k_q8_project(w, qm, y)
    torch.cuda.synchronize()
    rows.append(y.cpu().numpy())
np.save(out, np.concatenate(rows))
"""


@pytest.mark.parametrize("n", [5120, 776])
def test_q6k_mmq_direct_copy_matches_tiles(torch_gpu, n, tmp_path):
    """Q6_K MMQ runs the direct-copy kernel (q4k_mmq_dma.hip: one fixed K
    segment per block): 160 x 128 tiles for M > 128, in token chunks of at
    most what the scratch holds (512 + 188 at M = 700), and 160 x 64 tiles
    for M <= 128 (the M = 96 calls here). Its rows, with a residual, must equal
    bitwise the direct-copy M = 96 rows of the same tokens plus the residual,
    and those equal mmq_kernel's split tiles (a child process with
    QW38_MMQ_DMA=0). n = 776: a partial last row tile (776 = 4 x 160 + 136)."""
    import os
    import subprocess
    import sys
    torch = torch_gpu
    import qw38_amd.ops as ops
    k = 17408
    w, _ = _fit_q6k(torch, ops, n, k, 341)
    m = 700 if n == 5120 else 130
    q, _ = _q8(torch, ops, silu_rows(m, k, 342))
    res = torch.from_numpy(normal((m, n), 343)).cuda()
    y = torch.full((m, n), float("nan"), device="cuda")
    torch.cuda.synchronize()
    before = ops.scratch_stats()
    print(f"Q6_K direct-copy n={n} M={m}", flush=True)
    ops.q4k_q8_project(w, q, y, residual=res)
    torch.cuda.synchronize()
    after = ops.scratch_stats()
    assert after[0] == before[0] + 1 and after[1:] == before[1:], f"scratch not granted ({before} -> {after})"
    yn, rn = y.cpu().numpy(), res.cpu().numpy()
    windows = []
    for t0 in ((0, 560) if m == 700 else (0, 34)):
        print(f"Q6_K M=96 n={n} tokens {t0}..{t0 + 95}", flush=True)
        qm = ops.Q8Input.empty(96, k)
        qm.codes.copy_(q.codes[t0:t0 + 96]); qm.scales.copy_(q.scales[t0:t0 + 96]); qm.sums.copy_(q.sums[t0:t0 + 96])
        ym = _project(torch, ops, w, qm, 96, n)
        windows.append(ym)
        want = (ym + rn[t0:t0 + 96]).astype(np.float32)
        assert np.array_equal(yn[t0:t0 + 96].view(np.uint32), want.view(np.uint32)), f"tokens {t0}.. differ"
    print(f"Q6_K M=96 n={n} with QW38_MMQ_DMA=0", flush=True)
    out = str(tmp_path / "q6_split.npy")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _Q6_SPLIT_SCRIPT, root, str(n), str(m), out],
                       env=dict(os.environ, QW38_MMQ_DMA="0"), timeout=110, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    split = np.load(out)
    assert np.array_equal(split.view(np.uint32), np.concatenate(windows).view(np.uint32)), \
        "mmq_kernel's split tiles differ from the direct-copy rows"


@pytest.mark.parametrize("fmt,n,k", [("q4k", 5120, 5120), ("q6k", 5120, 17408)])
def test_decode_passes_rows_match_decode(torch_gpu, fmt, n, k):
    """M = 9..24 on small weights runs ceil(M / 8) batched-decode passes of
    4..8 tokens instead of the MMQ (the cost model's pick here). The decode
    kernels' rows for a token do not depend on the call's other tokens, so
    the rows of the M = 9 / 16 / 24 call must equal bitwise those of M = 8
    calls on the same tokens; M = 9 also matches the oracle."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    if fmt == "q4k":
        w, wl = _fit_q4k(torch, ops, n, k, 351, oracle.LAYOUT_Q4K_SEQ)
        x = normal((24, k), 352)
    else:
        w, wl = _fit_q6k(torch, ops, n, k, 353)
        x = silu_rows(24, k, 354)
    q, ob = _q8(torch, ops, x)

    def sub(t0, m):
        qm = ops.Q8Input.empty(m, k)
        qm.codes.copy_(q.codes[t0:t0 + m]); qm.scales.copy_(q.scales[t0:t0 + m]); qm.sums.copy_(q.sums[t0:t0 + m])
        return qm

    eights = {t0: _project(torch, ops, w, sub(t0, 8), 8, n) for t0 in (0, 8, 16)}
    for m in (9, 16, 24):
        print(f"{fmt} decode passes M={m}", flush=True)
        y = _project(torch, ops, w, sub(0, m), m, n)
        for t0, y8 in eights.items():
            hi = min(m, t0 + 8)
            if hi > t0:
                assert np.array_equal(y[t0:hi].view(np.uint32), y8[:hi - t0].view(np.uint32)), \
                    f"{fmt} M={m}: tokens {t0}..{hi - 1} differ from the M=8 call"
        if m == 16:  # the passes' residual epilogue adds exactly
            res = torch.from_numpy(normal((16, n), 355)).cuda()
            yr = torch.full((16, n), float("nan"), device="cuda")
            ops.q4k_q8_project(w, sub(0, 16), yr, residual=res)
            torch.cuda.synchronize()
            want = (y + res.cpu().numpy()).astype(np.float32)
            assert np.array_equal(yr.cpu().numpy().view(np.uint32), want.view(np.uint32)), f"{fmt} passes residual"
        if m == 9:
            q9 = oracle.Q8(ob.codes[:9], ob.scales[:9], ob.sums[:9], 9, k, ob.pk)
            if fmt == "q4k":
                rows = np.sort(np.random.Generator(np.random.PCG64(9)).choice(n, 512, replace=False))
                ref, _, _ = oracle.q4k_q8_contract(oracle.Q4K(wl.codes[rows], wl.meta[rows], len(rows), k), q9)
                _check(y[:, rows], ref, "Q4_K decode passes M=9")
            else:
                ref, _, _ = oracle.q6k_q8_contract(wl, q9)
                _check(y, ref, "Q6_K decode passes M=9")


_OWN_SCRIPT = r"""
import sys, numpy as np, torch
sys.path.insert(0, sys.argv[1]); sys.path.insert(0, sys.argv[1] + "/tests")
import oracle, qw38_amd.ops as ops
from _fix import silu_rows
n, k, m = 5120, 17408, 8
g = torch.Generator(device="cuda"); g.manual_seed(321)
x = torch.randn(n, k, generator=g, device="cuda") * 0.02
w = ops.upload_q6k_blocks(ops.quantize_q6k_blocks(x, n, k), n, k)
bf = oracle.fp32_to_bf16(silu_rows(m, k, 322))
q = ops.Q8Input.empty(m, k)
flag = torch.zeros(1, dtype=torch.int32, device="cuda")
ops.pack_q8(torch.from_numpy(bf.view(np.int16)).cuda(), q, flag)
y = torch.empty(m, n, device="cuda")
ops.q4k_q8_project(w, q, y)
torch.cuda.synchronize()
np.save(sys.argv[2], y.cpu().numpy())
"""


def test_q6k_decode_segments_rows_independent_of_m_and_mode(torch_gpu, tmp_path):
    """Q6_K batched decode (M 3..8): fixed K segments, two half-waves each,
    partials added in order. Rows are bitwise the same at every M in 3..8,
    and the whole-tile mode (no scratch; QW38_Q6_DECODE_OWN=1, run in a child
    process since the switch is read once) gives the same bits as the
    spread mode with the cross-block counters."""
    import os
    import subprocess
    import sys
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 5120, 17408
    g = torch.Generator(device="cuda")
    g.manual_seed(321)
    x = torch.randn(n, k, generator=g, device="cuda") * 0.02
    w = ops.upload_q6k_blocks(ops.quantize_q6k_blocks(x, n, k), n, k)
    wl = oracle.Q6K.from_ggml(ops.quantize_q6k_blocks(x, n, k).cpu().numpy(), n, k)
    del x
    q, ob = _q8(torch, ops, silu_rows(8, k, 322))
    ys = {}
    for m in (8, 3, 4, 5, 6, 7):
        print(f"Q6_K decode segments M={m}", flush=True)
        qm = ops.Q8Input.empty(m, k)
        qm.codes.copy_(q.codes[:m]); qm.scales.copy_(q.scales[:m]); qm.sums.copy_(q.sums[:m])
        for rep in range(2):  # the second call reuses the partials of the first one
            y = torch.full((m, n), float("nan"), device="cuda")
            torch.cuda.synchronize()
            before = ops.scratch_stats()
            ops.q4k_q8_project(w, qm, y)
            torch.cuda.synchronize()
            after = ops.scratch_stats()
            assert after[0] == before[0] + 1 and after[1:] == before[1:], \
                f"M={m}: the spread decode did not get the scratch ({before} -> {after})"
            yn = y.cpu().numpy()
            if rep:
                assert np.array_equal(yn.view(np.uint32), ys[m].view(np.uint32)), f"M={m} repeat differs"
            ys[m] = yn
        assert np.array_equal(ys[m].view(np.uint32), ys[8][:m].view(np.uint32)), f"M={m} rows differ from M=8"
    ref, _, _ = oracle.q6k_q8_contract(wl, ob)
    _check(ys[8], ref, "Q6_K decode M=8")
    out = str(tmp_path / "own.npy")
    env = dict(os.environ, QW38_Q6_DECODE_OWN="1")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _OWN_SCRIPT, root, out], env=env, timeout=110,
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    own = np.load(out)
    assert np.array_equal(own.view(np.uint32), ys[8].view(np.uint32)), "whole-tile mode differs from spread mode"


def test_q6k_small_shapes_and_dots(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    for (n, k) in [(37, 512), (64, 1024), (8, 256)]:
        wl = random_q6k(n, k, n + k)
        co, mo = wl.physical()
        w = ops.PrefillWeight.from_bytes(co, mo, oracle.LAYOUT_Q6K_W64, n, k)
        for m in (1, 2, 3, 8, 9, 33, 130):
            q, ob = _q8(torch, ops, normal((m, k), m + 7))
            y = _project(torch, ops, w, q, m, n)
            ref, _, dots = oracle.q6k_q8_contract(wl, ob, want_dots=True)
            _check(y, ref, f"Q6_K n={n} k={k} M={m}")
            if m in (3, 33):
                d = torch.zeros(m * n * (k // 32), dtype=torch.int32, device="cuda")
                ops.group_dots(w, q, d)
                torch.cuda.synchronize()
                assert np.array_equal(d.cpu().numpy().reshape(dots.shape), dots)


_DMA_OFF_SCRIPT = r"""
import sys, numpy as np, torch
sys.path.insert(0, sys.argv[1]); sys.path.insert(0, sys.argv[1] + "/tests")
import oracle, qw38_amd.ops as ops
from _fix import normal
n, k, m = 34816, 5120, 512
g = torch.Generator(device="cuda"); g.manual_seed(331)
x = torch.randn(n, k, generator=g, device="cuda") * 0.02
fail = torch.zeros(1, dtype=torch.int32, device="cuda")
w = ops.upload_q4k_blocks(ops.quantize_q4k_blocks(x, n, k, fail), n, k, layout=oracle.LAYOUT_Q4K_SEQ)
bf = oracle.fp32_to_bf16(normal((m, k), 332))
q = ops.Q8Input.empty(m, k)
flag = torch.zeros(1, dtype=torch.int32, device="cuda")
ops.pack_q8(torch.from_numpy(bf.view(np.int16)).cuda(), q, flag)
y = torch.empty(m, n, device="cuda")
ops.q4k_q8_project(w, q, y)
torch.cuda.synchronize()
np.save(sys.argv[2], y.cpu().numpy())
"""


def test_q4k_mmq_direct_copy_rows_independent_of_m(torch_gpu, tmp_path):
    """Q4_K 0x020D MMQ at config 2's N: the 256 x 128 tiles run the
    direct-copy kernel (q4k_mmq_dma.hip: pre-pass plus global->LDS copies)
    when the library scratch holds its pre-pass, next to the 128 x 32 tail
    split and the smaller tiles of the other M. Every token row must be
    bitwise the same at every M (the reference's schedule invariance,
    tests/q4k_q8_test.cpp:118-120), the launches that take the direct-copy
    kernel must have got the scratch, M = 40 matches the oracle, and the
    same M = 512 call with the kernel switched off (QW38_MMQ_DMA=0) and on its
    int8 form (QW38_MMQ_I8=1; child processes, since the switches are read
    once) must give the same bits."""
    import os
    import subprocess
    import sys
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 34816, 5120
    w, wl = _fit_q4k(torch, ops, n, k, 331, oracle.LAYOUT_Q4K_SEQ)
    q, ob = _q8(torch, ops, normal((512, k), 332))
    full = None
    # 512: direct-copy 256 x 128 tiles + 128 x 32 tail split (the second time
    # with a residual); 130 / 25 / 40 / 64: the other tile picks (25 is the
    # smallest M above the batched-decode passes)
    for m in (512, 512, 130, 25, 40, 64):
        print(f"Q4_K MMQ family M={m}", flush=True)
        qm = ops.Q8Input.empty(m, k)
        qm.codes.copy_(q.codes[:m]); qm.scales.copy_(q.scales[:m]); qm.sums.copy_(q.sums[:m])
        y = torch.full((m, n), float("nan"), device="cuda")
        res = torch.from_numpy(normal((m, n), 333)).cuda() if full is not None and m == 512 else None
        torch.cuda.synchronize()
        before = ops.scratch_stats()
        ops.q4k_q8_project(w, qm, y, residual=res)
        torch.cuda.synchronize()
        after = ops.scratch_stats()
        if m == 512:
            assert after[0] == before[0] + 1 and after[1:] == before[1:], \
                f"M={m}: the direct-copy kernel did not get the scratch ({before} -> {after})"
        yn = y.cpu().numpy()
        if res is not None:  # the residual epilogue adds exactly
            want = (full[:m] + res.cpu().numpy()).astype(np.float32)
            assert np.array_equal(yn.view(np.uint32), want.view(np.uint32)), "residual epilogue, M=512"
        elif full is None:
            full = yn
        else:
            assert np.array_equal(yn.view(np.uint32), full[:m].view(np.uint32)), f"M={m} rows differ from M=512"
        if m == 40:
            rows = np.sort(np.random.Generator(np.random.PCG64(40)).choice(n, 512, replace=False))
            sub = oracle.Q4K(wl.codes[rows], wl.meta[rows], len(rows), k)
            ref, _, _ = oracle.q4k_q8_contract(sub, oracle.Q8(ob.codes[:m], ob.scales[:m], ob.sums[:m], m, k, ob.pk))
            _check(yn[:, rows], ref, "Q4_K MMQ M=40")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    # the same call with the direct-copy kernel off, and on its int8 form
    # (QW38_MMQ_I8=1: v_mfma_i32_16x16x32_i8 on the raw codes, P = f32(s dot))
    for var, val in (("QW38_MMQ_DMA", "0"), ("QW38_MMQ_I8", "1")):
        print(f"Q4_K MMQ M=512 with {var}={val}", flush=True)
        out = str(tmp_path / f"{var}.npy")
        env = dict(os.environ, **{var: val})
        r = subprocess.run([sys.executable, "-c", _DMA_OFF_SCRIPT, root, out], env=env, timeout=110,
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        other = np.load(out)
        assert np.array_equal(other.view(np.uint32), full.view(np.uint32)), f"{var}={val} differs from the direct-copy kernel"


@pytest.mark.parametrize("layout", [oracle.LAYOUT_Q4K_SEQ, oracle.LAYOUT_Q4K_W64], ids=["020D", "0240"])
@pytest.mark.parametrize("n,k,m", [(12288, 5120, 128), (12288, 5120, 512), (12288, 5120, 2048),
                                   (34816, 5120, 128), (34816, 5120, 512), (34816, 5120, 2048)])
def test_config4_mmq_row_sample(torch_gpu, n, k, m, layout):
    """MMQ at the config-4 shapes (the tile shape follows the cost model:
    128x32 at M=128, 256x128 with the tail split at M=512, 256x128 at 2048);
    the oracle checks a seeded sample of 512 rows."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    w, wl = _fit_q4k(torch, ops, n, k, 401 + m, layout)
    q, ob = _q8(torch, ops, normal((m, k), 402 + m))
    y = _project(torch, ops, w, q, m, n)
    rows = np.sort(np.random.Generator(np.random.PCG64(m)).choice(n, 512, replace=False))
    sub = oracle.Q4K(wl.codes[rows], wl.meta[rows], len(rows), k)
    ref, _, _ = oracle.q4k_q8_contract(sub, ob)
    _check(y[:, rows], ref, f"config4 N={n} M={m}")


@pytest.mark.parametrize("m", [128, 512, 2048])
def test_config4_q6k_mmq_row_sample(torch_gpu, m):
    """Config-4 Q6_K down projection (5120x17408) at M = 128, 512, 2048."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 5120, 17408
    w, wl = _fit_q6k(torch, ops, n, k, 501 + m)
    q, ob = _q8(torch, ops, silu_rows(m, k, 502 + m))
    y = _project(torch, ops, w, q, m, n)
    rows = np.sort(np.random.Generator(np.random.PCG64(5 + m)).choice(n, 128, replace=False))
    sub = oracle.Q6K(wl.q[rows], wl.sc[rows], wl.d[rows], len(rows), k)
    ref, _, _ = oracle.q6k_q8_contract(sub, ob)
    _check(y[:, rows], ref, f"config4 Q6_K M={m}")


@pytest.mark.parametrize("layout", [oracle.LAYOUT_Q4K_SEQ, oracle.LAYOUT_Q4K_W64], ids=["020D", "0240"])
@pytest.mark.parametrize("m", [512, 2048])
def test_config4_mmq_outlier_rows(torch_gpu, m, layout):
    """MMQ on config 2's activations (1% of channels x20): the per-token
    power-of-two and FP16 hi+lo split of a*sum is the MMQ's one lossy step,
    and wide ranges of a stress it. Gate+up N=34816, 384 sampled rows."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 34816, 5120
    w, wl = _fit_q4k(torch, ops, n, k, 801 + m, layout)
    q, ob = _q8(torch, ops, outlier_rows(m, k, 802 + m))
    y = _project(torch, ops, w, q, m, n)
    rows = np.sort(np.random.Generator(np.random.PCG64(80 + m)).choice(n, 384, replace=False))
    sub = oracle.Q4K(wl.codes[rows], wl.meta[rows], len(rows), k)
    ref, _, _ = oracle.q4k_q8_contract(sub, ob)
    _check(y[:, rows], ref, f"config4 outlier rows N={n} M={m}")


def test_config5_qkv_decode(torch_gpu, tmp_path):
    """Config-5 QKV/gate projection (12288x5120, Q4_K on 0x020D) at M=1, the
    full output against the oracle."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 12288, 5120
    w, wl = _fit_q4k(torch, ops, n, k, 901, oracle.LAYOUT_Q4K_SEQ)
    q, ob = _q8(torch, ops, normal((1, k), 902))
    y = _project(torch, ops, w, q, 1, n)
    ref, _, _ = oracle.q4k_q8_contract(wl, ob)
    _check(y, ref, "config5 QKV M=1")
    # 1536 strips run one block each (six per CU); the persistent grid of
    # four blocks per CU (QW38_GEMV_STREAM_BLOCKS=1024, child process: the
    # switch is read once) must give the same bits
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    out = str(tmp_path / "persistent.npy")
    env = dict(os.environ, QW38_GEMV_STREAM_BLOCKS="1024")
    r = subprocess.run([sys.executable, "-c", _QKV_SCRIPT, root, out], env=env, timeout=110,
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    assert np.array_equal(np.load(out).view(np.uint32), y.view(np.uint32)), "persistent grid rows differ"


_QKV_SCRIPT = r"""
import sys, numpy as np, torch
sys.path.insert(0, sys.argv[1]); sys.path.insert(0, sys.argv[1] + "/tests")
import oracle, qw38_amd.ops as ops
from _fix import normal
from test_gpu_configs import _fit_q4k, _q8, _project
w, wl = _fit_q4k(torch, ops, 12288, 5120, 901, oracle.LAYOUT_Q4K_SEQ)
q, ob = _q8(torch, ops, normal((1, 5120), 902))
np.save(sys.argv[2], _project(torch, ops, w, q, 1, 12288))
"""


@pytest.mark.parametrize("m", [1, 8, 128, 512])
def test_config5_out_projection(torch_gpu, m):
    """Config-5 out projection (N=5120, K=6144, Q4_K on the reference layout
    0x020D): GEMV at M=1 and 8, MMQ at 128 (128x32 tiles) and 512 (128x64
    tiles); the oracle checks a seeded sample of 256 rows."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 5120, 6144
    w, wl = _fit_q4k(torch, ops, n, k, 601 + m, oracle.LAYOUT_Q4K_SEQ)
    q, ob = _q8(torch, ops, normal((m, k), 602 + m))
    y = _project(torch, ops, w, q, m, n)
    rows = np.sort(np.random.Generator(np.random.PCG64(60 + m)).choice(n, 256, replace=False))
    sub = oracle.Q4K(wl.codes[rows], wl.meta[rows], len(rows), k)
    ref, _, _ = oracle.q4k_q8_contract(sub, ob)
    _check(y[:, rows], ref, f"config5 out M={m}")


def test_config5_q6k_down_m128(torch_gpu):
    """Config-5 down projection at M=128 (Q6_K, the cost model picks 128x32
    tiles); 256 sampled rows against the oracle."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k, m = 5120, 17408, 128
    w, wl = _fit_q6k(torch, ops, n, k, 701)
    q, ob = _q8(torch, ops, normal((m, k), 702))
    y = _project(torch, ops, w, q, m, n)
    rows = np.sort(np.random.Generator(np.random.PCG64(7)).choice(n, 256, replace=False))
    sub = oracle.Q6K(wl.q[rows], wl.sc[rows], wl.d[rows], len(rows), k)
    ref, _, _ = oracle.q6k_q8_contract(sub, ob)
    _check(y[:, rows], ref, "config5 Q6_K down M=128")


@pytest.mark.parametrize("m", [1, 2])
def test_q6k_stream_unaligned_and_residual(torch_gpu, m):
    """Q6_K decode (M <= 2 streams the strip): Q8 codes at a 4-byte offset give
    bitwise the aligned result, the residual is added exactly, and the words
    around a row-tail output span stay untouched (tests/q4k_q8_test.cpp:96-117
    carried over to the Q6_K layout)."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 37, 2560
    wl = random_q6k(n, k, 4242)
    co, mo = wl.physical()
    w = ops.PrefillWeight.from_bytes(co, mo, oracle.LAYOUT_Q6K_W64, n, k)
    q, ob = _q8(torch, ops, normal((m, k), 99 + m))
    y = _project(torch, ops, w, q, m, n)
    ref, _, _ = oracle.q6k_q8_contract(wl, ob)
    _check(y, ref, f"Q6_K stream n={n} k={k} M={m}")
    z = q.codes.cpu().numpy().reshape(-1)
    shifted = np.full(z.size + 8, 99, np.int8)
    shifted[4:4 + z.size] = z
    dshift = _dev(torch, shifted)
    residual = ((np.arange(m * n) % 13).astype(np.float32) - 6) * 0.25
    dres = _dev(torch, residual)
    qv = ops.Q8Input(q.codes, q.scales, q.sums, q.m, q.k, q.padded_k)
    qv.codes = dshift
    qv.codes_ptr = dshift.data_ptr() + 4
    qv.codes_len = z.size
    guards = torch.full((m * n + 2,), -12345.0, device="cuda")
    ops.q4k_q8_project(w, qv, guards, residual=dres, output_ptr=guards.data_ptr() + 4,
                       output_len=m * n)
    torch.cuda.synchronize()
    r = guards.cpu().numpy()
    assert np.array_equal(r[1:-1], (y.reshape(-1) + residual).astype(np.float32))
    assert r[0] == -12345.0 and r[-1] == -12345.0


@pytest.mark.parametrize("m", [1, 512])
def test_config5_pass_graph_replay(torch_gpu, m):
    """The config-5 pass as the bench runs it (every projection of each layer
    captured in one hipGraph; Q4_K on 0x020D, Q6_K on 0x0241), here over two
    layers: after two replays, each projection of the last layer matches the
    oracle on 128 sampled rows (all rows at M=1 for the small shapes)."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    shapes = [(12288, 5120, "q4k"), (5120, 6144, "q4k"), (34816, 5120, "q4k"), (5120, 17408, "q6k")]
    layers = 2
    ws, wl, qs, obs = [], [], [], []
    for l in range(layers):
        for j, (n, k, fmt) in enumerate(shapes):
            seed = 1000 + 16 * l + j
            if fmt == "q4k":
                w, lw = _fit_q4k(torch, ops, n, k, seed, oracle.LAYOUT_Q4K_SEQ)
            else:
                w, lw = _fit_q6k(torch, ops, n, k, seed)
            q, ob = _q8(torch, ops, normal((m, k), seed + 7919))
            ws.append(w), wl.append(lw), qs.append(q), obs.append(ob)
    outs = [torch.full((m, n), float("nan"), device="cuda") for n, _, _ in shapes]

    def run_pass():
        for l in range(layers):
            for j in range(len(shapes)):
                ops.q4k_q8_project(ws[l * len(shapes) + j], qs[l * len(shapes) + j], outs[j])

    run_pass()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run_pass()
    for o in outs:
        o.fill_(float("nan"))
    for _ in range(2):
        g.replay()
        torch.cuda.synchronize()
    for j, (n, k, fmt) in enumerate(shapes):
        i = (layers - 1) * len(shapes) + j
        rows = np.sort(np.random.Generator(np.random.PCG64(j)).choice(n, 128, replace=False))
        y = outs[j].cpu().numpy()[:, rows]
        if fmt == "q4k":
            sub = oracle.Q4K(wl[i].codes[rows], wl[i].meta[rows], len(rows), k)
            ref, _, _ = oracle.q4k_q8_contract(sub, obs[i])
        else:
            sub = oracle.Q6K(wl[i].q[rows], wl[i].sc[rows], wl[i].d[rows], len(rows), k)
            ref, _, _ = oracle.q6k_q8_contract(sub, obs[i])
        _check(y, ref, f"config5 pass graph M={m} projection {j} ({n}x{k} {fmt})")
