"""BF16 prefill projections over Q4_K 0x020D (cuda/prefill.cu:510-779)
through the C-ABI: projections against the oracle (float64 sums of the rebuilt
BF16 operands), epilogues, token-count invariance, the paired SwiGLU, the BF16
RMS producer (bit-exact) and the whole MLP stage by stage."""
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


def _ref(wl, xb, rows=None):
    """float64 reference [tokens][n or len(rows)] from BF16 bits xb [tokens][k]."""
    sub = wl if rows is None else oracle.Q4K(wl.codes[rows], wl.meta[rows], len(rows), wl.k)
    return np.stack([oracle.q4k_bf16_gemv(sub, xb[t]) for t in range(xb.shape[0])])


def _check(y, ref, label):
    ok, ma, mr = oracle.parity_ok(y, ref)
    ok_ref = np.all(np.abs(y - ref) <= 1e-3 + 1e-4 * np.abs(ref))
    print(f"{label}: max_abs/rms={ma:.3g} mean_rel={mr:.3g}", flush=True)
    assert ok and ok_ref, label


@pytest.mark.parametrize("n,k,m", [(136, 256, 1), (136, 512, 17), (1000, 2560, 130),
                                   (5120, 5120, 64)])
def test_project_vs_oracle(torch_gpu, n, k, m):
    torch = torch_gpu
    import qw38_amd.ops as ops
    wl = random_q4k(n, k, n + k + m)
    w = _weight(ops, wl)
    xb = oracle.fp32_to_bf16(normal((m, k), m + 1))
    y = torch.full((m, n), float("nan"), device="cuda")
    ops.prefill_project(w, _dev(torch, xb.view(np.int16)), m, y, ops.DECODE_STORE_FP32)
    got = y.cpu().numpy()
    rows = None if n * k <= 2_600_000 else np.sort(
        np.random.Generator(np.random.PCG64(n)).choice(n, 256, replace=False))
    ref = _ref(wl, xb, rows)
    _check(got if rows is None else got[:, rows], ref, f"prefill n={n} k={k} m={m}")


def test_epilogues_and_token_invariance(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k, m = 264, 1024, 70
    wl = random_q4k(n, k, 9)
    w = _weight(ops, wl)
    xb = oracle.fp32_to_bf16(normal((m, k), 10))
    x = _dev(torch, xb.view(np.int16))
    f32 = torch.empty(m, n, device="cuda")
    ops.prefill_project(w, x, m, f32, ops.DECODE_STORE_FP32)
    base = f32.cpu().numpy()
    b16 = torch.empty(m, n, dtype=torch.int16, device="cuda")
    ops.prefill_project(w, x, m, b16, ops.DECODE_STORE_BF16)
    assert np.array_equal(b16.cpu().numpy().view(np.uint16), oracle.fp32_to_bf16(base))
    res = normal((m, n), 11)
    out = torch.empty(m, n, device="cuda")
    ops.prefill_project(w, x, m, out, ops.DECODE_RESIDUAL_ADD_FP32, residual=_dev(torch, res))
    assert np.array_equal(out.cpu().numpy(), (res + base).astype(np.float32))
    # each token's row is independent of how many tokens share the launch
    one = torch.empty(1, n, device="cuda")
    ops.prefill_project(w, x[37:38].contiguous(), 1, one, ops.DECODE_STORE_FP32)
    assert np.array_equal(one.cpu().numpy()[0], base[37])
    # unaligned (2-byte) input span: same results through the narrow-load path
    xu = torch.empty(m * k + 1, dtype=torch.int16, device="cuda")
    xu[1:] = x.flatten()
    ops.prefill_project(w, xu[1:], m, f32, ops.DECODE_STORE_FP32)
    assert np.array_equal(f32.cpu().numpy(), base)


def test_tail_split_bitwise(torch_gpu):
    """M=512 over 34816 rows makes 272 tiles of 256 x 256: one round of them
    and a 128-row tail (rows 32768 on at 256 CUs). Every row, head or tail,
    equals the 128 x 64 kernel's result for the same token bitwise, and
    sampled rows match the oracle. The BF16 and residual epilogues and the
    2-byte-aligned activation path of the same launch give the same values."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k, m = 34816, 256, 512
    wl = random_q4k(n, k, 77)
    w = _weight(ops, wl)
    xb = oracle.fp32_to_bf16(normal((m, k), 78))
    x = _dev(torch, xb.view(np.int16))
    y = torch.full((m, n), float("nan"), device="cuda")
    ops.prefill_project(w, x, m, y, ops.DECODE_STORE_FP32)
    got = y.cpu().numpy()
    small = torch.full((64, n), float("nan"), device="cuda")
    ops.prefill_project(w, x[448:].contiguous(), 64, small, ops.DECODE_STORE_FP32)
    assert np.array_equal(got[448:], small.cpu().numpy())
    rows = np.concatenate([np.arange(0, 64), np.arange(32700, 32830), np.arange(n - 64, n)])
    _check(got[::16][:, rows], _ref(wl, xb[::16], rows), "prefill split n=34816 m=512")
    # the 256 x 256 tile's other epilogues and its 2-byte-aligned load path
    b16 = torch.empty(m, n, dtype=torch.int16, device="cuda")
    ops.prefill_project(w, x, m, b16, ops.DECODE_STORE_BF16)
    assert np.array_equal(b16.cpu().numpy().view(np.uint16), oracle.fp32_to_bf16(got))
    res = normal((m, n), 79)
    out = torch.empty(m, n, device="cuda")
    ops.prefill_project(w, x, m, out, ops.DECODE_RESIDUAL_ADD_FP32, residual=_dev(torch, res))
    assert np.array_equal(out.cpu().numpy(), (res + got).astype(np.float32))
    xu = torch.empty(m * k + 1, dtype=torch.int16, device="cuda")
    xu[1:] = x.flatten()
    ops.prefill_project(w, xu[1:], m, y, ops.DECODE_STORE_FP32)
    assert np.array_equal(y.cpu().numpy(), got)


def test_paired_swiglu(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k, m = 520, 1536, 33
    gl, ul = random_q4k(n, k, 21), random_q4k(n, k, 22)
    g, u = _weight(ops, gl), _weight(ops, ul)
    x = _dev(torch, oracle.fp32_to_bf16(normal((m, k), 23)).view(np.int16))
    ga, ua = torch.empty(m, n, device="cuda"), torch.empty(m, n, device="cuda")
    ops.prefill_project(g, x, m, ga, ops.DECODE_STORE_FP32)
    ops.prefill_project(u, x, m, ua, ops.DECODE_STORE_FP32)
    sw = torch.empty(m, n, dtype=torch.int16, device="cuda")
    ops.prefill_paired_swiglu(g, u, x, sw, m)
    gd, ud = ga.cpu().numpy().astype(np.float64), ua.cpu().numpy().astype(np.float64)
    ref = oracle.bf16_to_fp32(oracle.fp32_to_bf16((gd / (1 + np.exp(-gd)) * ud).astype(np.float32)))
    got = oracle.bf16_to_fp32(sw.cpu().numpy().view(np.uint16))
    ulp = np.abs(ref.view(np.int32).astype(np.int64) - got.view(np.int32).astype(np.int64))
    assert np.all(ulp <= 65536)


def test_paired_big_tile_bitwise(torch_gpu):
    """17408 features at M=512 run the paired 256 x 256 tile (128 gate + 128
    up rows per block) over whole rounds and a 128 x 64 paired tail: every
    feature equals the 128 x 64 paired kernel's output for the same token
    bitwise, and stays within 1 BF16 ulp of SiLU(g) * u from the separate
    projections."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k, m = 17408, 256, 512
    gl, ul = random_q4k(n, k, 31), random_q4k(n, k, 32)
    g, u = _weight(ops, gl), _weight(ops, ul)
    x = _dev(torch, oracle.fp32_to_bf16(normal((m, k), 33)).view(np.int16))
    sw = torch.full((m, n), -1, dtype=torch.int16, device="cuda")
    ops.prefill_paired_swiglu(g, u, x, sw, m)
    small = torch.full((64, n), -1, dtype=torch.int16, device="cuda")
    ops.prefill_paired_swiglu(g, u, x[448:].contiguous(), small, 64)
    got = sw.cpu().numpy()
    assert np.array_equal(got[448:], small.cpu().numpy())
    ga, ua = torch.empty(m, n, device="cuda"), torch.empty(m, n, device="cuda")
    ops.prefill_project(g, x, m, ga, ops.DECODE_STORE_FP32)
    ops.prefill_project(u, x, m, ua, ops.DECODE_STORE_FP32)
    gd, ud = ga.cpu().numpy().astype(np.float64), ua.cpu().numpy().astype(np.float64)
    ref = oracle.bf16_to_fp32(oracle.fp32_to_bf16((gd / (1 + np.exp(-gd)) * ud).astype(np.float32)))
    val = oracle.bf16_to_fp32(got.view(np.uint16))
    ulp = np.abs(ref.view(np.int32).astype(np.int64) - val.view(np.int32).astype(np.int64))
    assert np.all(ulp <= 65536)


def test_hidden_rms_bf16_bit_exact(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    m = 5
    res = (normal((m, 5120), 31) * 4).astype(np.float32)
    res[2] = 0.0
    gamma = oracle.fp32_to_bf16(normal(5120, 32, 0.1))
    out = torch.empty(m, 5120, dtype=torch.int16, device="cuda")
    ops.hidden_rms_bf16(_dev(torch, res), _dev(torch, gamma.view(np.int16)), 1e-6, m, out)
    _, bf = oracle.rms_q8(res, gamma, 1e-6)
    assert np.array_equal(out.cpu().numpy().view(np.uint16), bf)


def test_prefill_mlp(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    m = 40
    gl, ul, dl = random_q4k(17408, 5120, 41), random_q4k(17408, 5120, 42), random_q4k(5120, 17408, 43)
    g, u, d = _weight(ops, gl), _weight(ops, ul), _weight(ops, dl)
    gamma = oracle.fp32_to_bf16(normal(5120, 44, 0.1))
    h = normal((m, 5120), 45)
    dh, dg = _dev(torch, h), _dev(torch, gamma.view(np.int16))
    ws = torch.zeros(ops.prefill_mlp_workspace_bytes(m), dtype=torch.uint8, device="cuda")
    out = torch.full((m, 5120), float("nan"), device="cuda")
    ops.prefill_mlp(g, u, d, dh, dg, 1e-6, out, m, ws)
    b = ws.cpu().numpy()
    norm = b[:m * 5120 * 2].view(np.uint16).reshape(m, 5120)
    sw = b[m * 5120 * 2:m * 5120 * 2 + m * 17408 * 2].view(np.uint16).reshape(m, 17408)
    _, bf = oracle.rms_q8(h, gamma, 1e-6)
    assert np.array_equal(norm, bf), "RMS -> BF16 stage"
    sw2 = torch.empty(m, 17408, dtype=torch.int16, device="cuda")
    ops.prefill_paired_swiglu(g, u, _dev(torch, norm.view(np.int16)), sw2, m)
    assert np.array_equal(sw, sw2.cpu().numpy().view(np.uint16)), "SwiGLU stage"
    rows = np.sort(np.random.Generator(np.random.PCG64(46)).choice(5120, 128, replace=False))
    ref = _ref(dl, sw, rows)
    _check(out.cpu().numpy()[:, rows] - h[:, rows], ref, "prefill mlp down")
