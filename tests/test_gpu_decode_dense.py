"""decode_mmv over the reference's dense tile layouts through the C-ABI:
Q4G64 (0x0201 / 0x020B), Q8G32 (0x0202 / 0x020C) and BF16 dense tiles (0x0203)
(cuda/decode_mmv.cu:92-180, 406-560). One-hot inputs return every rebuilt BF16
operand exactly (the check of tests/decode_mmv_unit_test.cpp:405-478 applied
to these layouts); random projections against the oracle's float64 sum of the
rebuilt operands within the reference's decode budget; padding, odd tile
counts, the maximum K, every epilogue, paired, ranged and a/b launches."""
import numpy as np
import pytest

import oracle
from _fix import normal

pytestmark = pytest.mark.gpu

LAYOUTS = [0x0201, 0x020B, 0x0202, 0x020C, 0x0203]
IDS = ["q4g64", "q4g64c", "q8g32", "q8g32c", "bf16"]


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _bf16(torch, x):
    return _dev(torch, oracle.fp32_to_bf16(np.asarray(x, np.float32)).view(np.int16))


def _random_dense(layout, n, k, seed):
    """Seeded logical weight of the layout -> (tiled codes, scales or None,
    BF16 operand bits [n][k] from the oracle)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    pn, pk = oracle.pad8(n), oracle.pad256(k)
    if layout == 0x0203:
        w = oracle.fp32_to_bf16((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
        co = oracle.pack_bf16_tile(w, n, k)
        return co, None, oracle.dense_operands(layout, co, None, pn, pk)[:n, :k]
    g = oracle.dense_group(layout)
    q4 = g == 64
    c = rng.integers(-8 if q4 else -127, 8 if q4 else 128, (n, k)).astype(np.int8)
    s = (np.abs(rng.standard_normal((n, k // g))) * 0.02 / (7 if q4 else 127) + 1e-5)
    s = s.astype(np.float16).view(np.uint16)
    co, so = oracle.pack_dense(layout, c, s, n, k)
    return co, so, oracle.dense_operands(layout, co, so, pn, pk)[:n, :k]


def _weight(torch, ops, layout, co, so, n, k):
    return ops.dense_weight(layout, _dev(torch, co), None if so is None else _dev(torch, so), n, k)


def _tol_ok(y, ref):
    """The reference's decode budget (cuda/decode_mmv.hpp:108-112) and the
    north-star tolerance."""
    ok_ref = np.all(np.abs(y - ref) <= 1e-3 + 1e-4 * np.abs(ref))
    ok, ma, mr = oracle.parity_ok(y, ref)
    return ok_ref and ok, ma, mr


@pytest.mark.parametrize("layout", LAYOUTS, ids=IDS)
def test_onehot_exact_operands(torch_gpu, layout):
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 16, 768  # two strips, three K tiles (an odd Q4 tile pair tail)
    co, so, wb = _random_dense(layout, n, k, layout)
    w = _weight(torch, ops, layout, co, so, n, k)
    eye = torch.zeros(k, k, dtype=torch.int16, device="cuda")
    eye.fill_diagonal_(0x3F80)  # BF16 1.0
    y = torch.full((k, n), float("nan"), device="cuda")
    for col in range(k):
        ops.decode_mmv(ops.decode_desc(w, eye[col], y[col], ops.DECODE_STORE_FP32))
    got = y.cpu().numpy()  # got[col][row] = w[row][col]
    want = oracle.bf16_to_fp32(wb).T
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"layout {layout:#x}"


SHAPES = [(20, 192), (136, 768), (2048, 5120), (300, 17408)]


@pytest.mark.parametrize("layout", LAYOUTS, ids=IDS)
@pytest.mark.parametrize("n,k", SHAPES, ids=[f"{n}x{k}" for n, k in SHAPES])
def test_random_projection_vs_oracle(torch_gpu, layout, n, k):
    torch = torch_gpu
    import qw38_amd.ops as ops
    print(f"dense decode layout={layout:#x} n={n} k={k}", flush=True)
    x = normal(k, n + 3 * k)
    y = torch.full((n,), float("nan"), device="cuda")
    if layout == 0x0203 and (n % 8 or k % 256):
        w = _weight(torch, ops, layout, np.zeros(oracle.pad8(n) * oracle.pad256(k) * 2, np.uint8), None, n, k)
        # the reference rejects these shapes before any launch (cuda/decode_mmv.cu:375-380)
        from qw38_amd._lib import QW38_INVALID_ARGUMENT, Qw38Error
        with pytest.raises(Qw38Error) as e:
            ops.decode_mmv(ops.decode_desc(w, _bf16(torch, x), y, ops.DECODE_STORE_FP32))
        assert e.value.status == QW38_INVALID_ARGUMENT and "N%8==0 and K%256==0" in e.value.detail
        torch.cuda.synchronize()
        assert torch.isnan(y).all(), "nothing was written"
        return
    co, so, wb = _random_dense(layout, n, k, n * 7 + k + layout)
    w = _weight(torch, ops, layout, co, so, n, k)
    ops.decode_mmv(ops.decode_desc(w, _bf16(torch, x), y, ops.DECODE_STORE_FP32))
    ref = oracle.bf16_gemv(wb, oracle.fp32_to_bf16(x))
    ok, ma, mr = _tol_ok(y.cpu().numpy(), ref)
    print(f"  max_abs/rms={ma:.3g} mean_rel={mr:.3g}", flush=True)
    assert ok


def test_vocab_head_shape_q8(torch_gpu):
    """The Q8G32 vocabulary head geometry class (N=248320 x 5120 in the
    reference, cuda/decode_mmv.cu:548-553) at N=65536, row-sampled."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 65536, 5120
    co, so, wb = _random_dense(0x0202, n, k, 99)
    w = _weight(torch, ops, 0x0202, co, so, n, k)
    x = normal(k, 98)
    y = torch.empty(n, device="cuda")
    ops.decode_mmv(ops.decode_desc(w, _bf16(torch, x), y, ops.DECODE_STORE_FP32))
    rows = np.sort(np.random.Generator(np.random.PCG64(4)).choice(n, 1024, replace=False))
    ref = oracle.bf16_gemv(wb[rows], oracle.fp32_to_bf16(x))
    ok, ma, mr = _tol_ok(y.cpu().numpy()[rows], ref)
    print(f"q8 head: max_abs/rms={ma:.3g} mean_rel={mr:.3g}", flush=True)
    assert ok


@pytest.mark.parametrize("layout", LAYOUTS, ids=IDS)
def test_epilogues_paired_ranges(torch_gpu, layout):
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 1000, 2560
    print(f"dense epilogues layout={layout:#x}", flush=True)
    (gc, gs_, _), (uc, us_, _) = _random_dense(layout, n, k, 31), _random_dense(layout, n, k, 32)
    g = _weight(torch, ops, layout, gc, gs_, n, k)
    u = _weight(torch, ops, layout, uc, us_, n, k)
    x = _bf16(torch, normal(k, 33))
    ga, ua = torch.empty(n, device="cuda"), torch.empty(n, device="cuda")
    ops.decode_mmv(ops.decode_desc(g, x, ga, ops.DECODE_STORE_FP32))
    ops.decode_mmv(ops.decode_desc(u, x, ua, ops.DECODE_STORE_FP32))
    gsv, usv = ga.cpu().numpy(), ua.cpu().numpy()
    # BF16 store: the FP32 result rounded
    b16 = torch.empty(n, dtype=torch.int16, device="cuda")
    ops.decode_mmv(ops.decode_desc(g, x, b16, ops.DECODE_STORE_BF16))
    assert np.array_equal(b16.cpu().numpy().view(np.uint16), oracle.fp32_to_bf16(gsv))
    # residual: separate output, then in place
    res = normal(n, 34)
    r = _dev(torch, res)
    out = torch.empty(n, device="cuda")
    ops.decode_mmv(ops.decode_desc(g, x, out, ops.DECODE_RESIDUAL_ADD_FP32, residual=r))
    assert np.array_equal(out.cpu().numpy(), (res + gsv).astype(np.float32))
    ops.decode_mmv(ops.decode_desc(g, x, None, ops.DECODE_RESIDUAL_ADD_FP32, residual=r))
    assert np.array_equal(r.cpu().numpy(), (res + gsv).astype(np.float32))
    # paired with separate FP32 outputs: bitwise equal to the single launches
    pa, pb = torch.empty(n, device="cuda"), torch.empty(n, device="cuda")
    ops.decode_mmv_paired(ops.decode_desc(g, x, pa, ops.DECODE_STORE_FP32),
                          ops.decode_desc(u, x, pb, ops.DECODE_STORE_FP32))
    assert np.array_equal(pa.cpu().numpy(), gsv) and np.array_equal(pb.cpu().numpy(), usv)
    # paired SwiGLU -> BF16 into A's output
    sw = torch.empty(n, dtype=torch.int16, device="cuda")
    ops.decode_mmv_paired(ops.decode_desc(g, x, sw, ops.DECODE_SWIGLU_BF16),
                          ops.decode_desc(u, x, None, ops.DECODE_SWIGLU_BF16))
    gd, ud = gsv.astype(np.float64), usv.astype(np.float64)
    ref = oracle.bf16_to_fp32(oracle.fp32_to_bf16((gd / (1 + np.exp(-gd)) * ud).astype(np.float32)))
    got = oracle.bf16_to_fp32(sw.cpu().numpy().view(np.uint16))
    ulp = np.abs(ref.view(np.int32).astype(np.int64) - got.view(np.int32).astype(np.int64))
    assert np.all(ulp <= 65536), "SwiGLU within one BF16 ulp of the float64 formula"
    # ranges: BF16 stores equal to the single launches
    outs = [torch.empty(n, dtype=torch.int16, device="cuda") for _ in range(2)]
    ops.decode_mmv_ranges([ops.decode_desc(g, x, outs[0], ops.DECODE_STORE_BF16),
                           ops.decode_desc(u, x, outs[1], ops.DECODE_STORE_BF16)])
    assert np.array_equal(outs[0].cpu().numpy().view(np.uint16), oracle.fp32_to_bf16(gsv))
    assert np.array_equal(outs[1].cpu().numpy().view(np.uint16), oracle.fp32_to_bf16(usv))
    if layout == 0x0203:
        # GDN a/b contraction (cuda/decode_mmv.cu:781-800): FP32 outputs, one launch
        aa, ab = torch.empty(n, device="cuda"), torch.empty(n, device="cuda")
        ops.decode_ab_bf16(ops.decode_desc(g, x, aa, ops.DECODE_STORE_FP32),
                           ops.decode_desc(u, x, ab, ops.DECODE_STORE_FP32))
        assert np.array_equal(aa.cpu().numpy(), gsv) and np.array_equal(ab.cpu().numpy(), usv)
    else:
        with pytest.raises(Exception, match="cuda_bf16_dense_tile_v0"):
            ops.decode_ab_bf16(ops.decode_desc(g, x, pa, ops.DECODE_STORE_FP32),
                               ops.decode_desc(u, x, pb, ops.DECODE_STORE_FP32))
