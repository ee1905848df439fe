"""CPU pins of the oracle (test infrastructure) before it is trusted as the
checker: golden fixtures from the reference's pinned llama.cpp header,
the compiled header itself (oracle/_ref) where present, and closed forms /
invariants chosen so that a dropped term, sign or index fails."""
import os

import numpy as np
import pytest

import oracle
from _fix import REF_K, REF_N, ggml_q6k_coord, ggml_q6k_decode, normal, random_q4k, random_q6k, ref_fixture_input, ref_fixture_weight

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
L = oracle.lib()


def _golden(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


# ---- scalar conversions ------------------------------------------------------
def test_fp16_decode_exhaustive_closed_form():
    """Every finite FP16 pattern against the IEEE definition evaluated in numpy
    (np.float16 -> float32 is exact), including all subnormals."""
    bits = np.arange(65536, dtype=np.uint16)
    finite = (bits & 0x7C00) != 0x7C00
    want = bits[finite].view(np.float16).astype(np.float32)
    got = np.array([L.orc_fp16_to_fp32(int(b)) for b in bits[finite]], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_fp16_encode_matches_pinned_llama_fixture():
    g = _golden("fp16_ref.npz")
    got = np.array([L.orc_fp32_to_fp16(float(v)) for v in g["f32"]], np.uint16)
    assert np.array_equal(got, g["f16"])
    # and IEEE RNE as numpy implements it (NaN payloads aside)
    fin = np.isfinite(g["f32"])
    with np.errstate(over="ignore"):  # finite values beyond FP16's range round to inf
        want = g["f32"][fin].astype(np.float16).view(np.uint16)
    assert np.array_equal(got[fin], want)


def test_nearest_int_matches_pinned_fixture_and_rint():
    g = _golden("fp16_ref.npz")
    got = np.array([L.orc_nearest_int(float(v)) for v in g["ni_in"]], np.int32)
    assert np.array_equal(got, g["ni"])
    assert np.array_equal(got, np.rint(g["ni_in"]).astype(np.int32))


def test_bf16_rne_ties_and_nan():
    x = np.array([1.0, 1.00390625, 1.01171875, -1.00390625, 3.3895314e38, np.inf], np.float32)
    # 1 + 2^-8 is a tie -> even (1.0); 1 + 3*2^-8 -> up
    b = oracle.fp32_to_bf16(x)
    assert list(b[:4]) == [0x3F80, 0x3F80, 0x3F82, 0xBF80]
    assert b[5] == 0x7F80
    nan = oracle.fp32_to_bf16(np.array([np.float32("nan")]))[0]
    assert nan & 0x7F80 == 0x7F80 and nan & 0x7F
    for v in x[:5]:
        assert L.orc_fp32_to_bf16_rne(float(v)) == oracle.fp32_to_bf16(np.array([v]))[0]


def test_expf_within_one_ulp():
    xs = np.linspace(-87.0, 88.0, 20001).astype(np.float32)
    got = np.array([L.orc_expf(float(v)) for v in xs], np.float32)
    ref = np.exp(xs.astype(np.float64)).astype(np.float32)
    ulp = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert ulp.max() <= 1
    assert np.isnan(L.orc_expf(float("nan")))
    assert L.orc_expf(100.0) == float("inf") and L.orc_expf(-200.0) == 0.0


# ---- Q4_K fitter ---------------------------------------------------------------
def test_q4k_fitter_bytes_equal_pinned_llama_fixture():
    g = _golden("q4k_ref_blocks.npz")
    saw_sub_d = saw_sub_m = False
    for x, want, deq in zip(g["x"], g["blocks"], g["dequant"]):
        rc, codes, meta = oracle.quantize_q4k_block(x)
        assert rc == 0
        q = oracle.Q4K(codes.reshape(1, 256), meta.reshape(1, 1, 16), 1, 256)
        assert np.array_equal(q.ggml(), want)
        d = int(want[0]) | int(want[1]) << 8
        dm = int(want[2]) | int(want[3]) << 8
        saw_sub_d |= 0 < d < 0x400
        saw_sub_m |= 0 < dm < 0x400
        # dequantized operand (reference.hpp:253-275) from the oracle's own decode
        mine = np.array([L.orc_fp16_to_fp32(d) * _sm(meta, j // 32)[0] * codes[j]
                         - L.orc_fp16_to_fp32(dm) * _sm(meta, j // 32)[1] for j in range(256)],
                        np.float32)
        assert np.array_equal(mine.view(np.uint32), deq.view(np.uint32))
    assert saw_sub_d and saw_sub_m, "FP16 subnormal d and dmin are exercised"


def _sm(meta, g):
    p = meta[4:]
    if g < 4:
        return np.float32(p[g] & 63), np.float32(p[g + 4] & 63)
    return (np.float32((p[g + 4] & 15) | ((p[g - 4] >> 6) << 4)),
            np.float32((p[g + 4] >> 4) | ((p[g] >> 6) << 4)))


def test_q4k_fitter_against_compiled_pinned_header():
    R = oracle.ref()
    if R is None:
        pytest.skip("oracle/_ref not built (reference tree absent); golden fixture covers this")
    w = normal((64, 5120), 77, 0.02)
    blk = np.zeros(64 * 20 * 144, np.uint8)
    R.ref_quantize_row_q4_K(w.ctypes.data, blk.ctypes.data, w.size)
    assert np.array_equal(oracle.quantize_q4k(w).ggml(), blk)


def test_q4k_fitter_rejections():
    x = np.zeros(256, np.float32)
    x[0] = np.inf
    assert oracle.quantize_q4k_block(x)[0] == 1
    x[0] = np.nan
    assert oracle.quantize_q4k_block(x)[0] == 1
    x[0] = np.finfo(np.float32).max
    assert oracle.quantize_q4k_block(x)[0] == 2
    for tiny in (2.0 ** -126, -(2.0 ** -126), 2.0 ** -133):
        assert oracle.quantize_q4k_block(np.full(256, tiny, np.float32))[0] == 2


# ---- Q8 pack ----------------------------------------------------------------------
def test_q8_pack_reference_fixture_closed_form():
    for m in (1, 5):
        x = ref_fixture_input(m)
        q = oracle.pack_q8(x, m, REF_K)
        assert not q.failed
        pk = oracle.pad256(REF_K)
        v = np.zeros((m, pk), np.float32)
        v[:, :REF_K] = oracle.bf16_to_fp32(x).reshape(m, REF_K)
        g = v.reshape(m, pk // 32, 32)
        peak = np.abs(g).max(axis=2)
        a = np.where(peak == 0, np.float32(1), peak / np.float32(127)).astype(np.float32)
        z = np.clip(np.rint(g / a[:, :, None]), -127, 127).astype(np.int32)
        assert np.array_equal(q.codes.astype(np.int32), z.reshape(m, pk))
        assert np.array_equal(q.scales.view(np.uint32), a.view(np.uint32))
        assert np.array_equal(q.sums, z.sum(axis=2))
        assert list(q.codes[0, :5]) == [127, 0, 2, 0, -2]  # ties to even + saturation
        assert q.sums[0, 2] < 0
    q = oracle.pack_q8(ref_fixture_input(3), 3, REF_K)
    assert np.all(q.codes[2] == 0) and np.all(q.scales[2] == 1.0), "whole zero token -> scale 1"
    assert np.all(q.codes[:, REF_K:] == 0), "padding packs as zeros"


def test_q8_pack_nonfinite_flags():
    x = ref_fixture_input(2)
    for bits in (0x7F80, 0xFF80, 0x7FC0):
        xb = x.copy()
        xb[1, 40] = bits
        q = oracle.pack_q8(xb, 2, REF_K)
        assert q.failed and np.isnan(q.scales[1, 1]) and np.all(q.codes[1, 32:64] == 0)
        assert np.isfinite(q.scales[0]).all()


# ---- layouts ------------------------------------------------------------------------
def test_layout_020d_golden_coordinates():
    """tests/pack_layout_test.cpp:197-245 restated: byte j of a tile row holds
    code[2j] | code[2j+1] << 4; metadata at ((row/8*blocks + block)*8 + row%8)*16."""
    w = ref_fixture_weight()
    co, mo = w.physical(oracle.LAYOUT_Q4K_SEQ)
    kbs = w.pk // 256
    for row in (0, 7, 8, 136):
        for kb in range(kbs):
            tr = ((row // 8) * kbs + kb) * 8 + row % 8
            assert np.array_equal(mo[tr * 16:(tr + 1) * 16], w.meta[row, kb])
            cb = co[tr * 128:(tr + 1) * 128]
            c = w.codes[row, kb * 256:(kb + 1) * 256]
            assert np.array_equal(cb, (c[0::2] | (c[1::2] << 4)).astype(np.uint8))
    assert co.size == oracle.pad8(REF_N) * w.pk // 2


def test_layout_0240_coordinates_and_roundtrip():
    n, k = 40, 768 * 4  # 12 super-blocks: one full chunk of 8 + a short chunk of 4
    w = random_q4k(n, k, 5)
    co, mo = w.physical(oracle.LAYOUT_Q4K_W64)
    strips, kbs = oracle.pad8(n) // 8, k // 256
    row, kb, g = 13, 9, 5            # strip 1, chunk 1 (nk = 4), kq = 1
    nk = 4
    off = strips * 8192 * 1 + 1 * nk * 1024 + g * nk * 128 + (1 * 8 + 5) * 16
    c = w.codes[row, kb * 256 + g * 32: kb * 256 + g * 32 + 32]
    want = np.array([c[8 * (j // 4) + j % 4] | (c[8 * (j // 4) + 4 + j % 4] << 4) for j in range(16)],
                    np.uint8)
    assert np.array_equal(co[off:off + 16], want)
    moff = strips * 1024 * 1 + 1 * nk * 128 + (1 * 8 + 5) * 16
    assert np.array_equal(mo[moff:moff + 16], w.meta[row, kb])
    w2 = oracle.Q4K.from_physical(oracle.LAYOUT_Q4K_W64, co, mo, n, k)
    assert np.array_equal(w2.codes, w.codes) and np.array_equal(w2.meta, w.meta)


def test_layout_0241_chunk_planes():
    """Q6_K 0x0241: an 8-row tile (strip, kb) is 1536 code bytes at
    (strip*kbs + kb)*1536, a low-nibble plane of 16 B chunks then a high-pair
    plane of 8 B chunks, chunk c = (g/2)*16 + 2r + g%2 for row r of the tile
    and K32 group g; scales per tile row, then the fp16 d array."""
    n, k = 20, 768  # three strips (the last padded), three super-blocks
    q6 = random_q6k(n, k, 17)
    co, mo = q6.physical()
    kbs, pn = k // 256, oracle.pad8(n)
    assert co.size == pn * kbs * 192 and mo.size == pn * kbs * 18
    for row, kb, g in [(0, 0, 0), (13, 2, 5), (7, 1, 7), (19, 0, 3)]:
        r, tile = row % 8, (row // 8) * kbs + kb
        c = (g // 2) * 16 + 2 * r + g % 2
        q = q6.q[row, kb * 256 + g * 32: kb * 256 + g * 32 + 32].astype(np.uint32)
        lo = np.array([(q[8 * (j // 4) + j % 4] & 15) | ((q[8 * (j // 4) + 4 + j % 4] & 15) << 4)
                       for j in range(16)], np.uint8)
        assert np.array_equal(co[tile * 1536 + c * 16: tile * 1536 + c * 16 + 16], lo)
        hi = np.array([sum(((q[16 * (b // 4) + 4 * s + b % 4] >> 4) & 3) << (2 * s) for s in range(4))
                       for b in range(8)], np.uint8)
        assert np.array_equal(co[tile * 1536 + 1024 + c * 8: tile * 1536 + 1024 + c * 8 + 8], hi)
        tr = tile * 8 + r
        assert np.array_equal(mo[tr * 16: tr * 16 + 16].view(np.int8), q6.sc[row, kb * 16: kb * 16 + 16])
        d = int(mo[pn * kbs * 16 + tr * 2]) | (int(mo[pn * kbs * 16 + tr * 2 + 1]) << 8)
        assert d == int(q6.d[row, kb])
    # padding rows of the last strip stay zero
    tile = 2 * kbs
    for r in range(n % 8, 8):
        for g in range(8):
            c = (g // 2) * 16 + 2 * r + g % 2
            assert not co[tile * 1536 + c * 16: tile * 1536 + c * 16 + 16].any()


def _sm_all(meta):
    """Vectorised 6-bit scale/min unpack (get_scale_min_k4) of [..., 16] metadata."""
    p = meta[..., 4:].astype(np.int32)
    s = np.empty(meta.shape[:-1] + (8,), np.float32)
    m = np.empty_like(s)
    for g in range(8):
        if g < 4:
            s[..., g], m[..., g] = p[..., g] & 63, p[..., g + 4] & 63
        else:
            s[..., g] = (p[..., g + 4] & 15) | ((p[..., g - 4] >> 6) << 4)
            m[..., g] = (p[..., g + 4] >> 4) | ((p[..., g] >> 6) << 4)
    return s, m


def test_q4k_ggml_roundtrip_and_dequant_equals_compiled_header():
    """The GGML Q4_K byte order: logical -> GGML -> logical is lossless, and the
    compiled pinned header's dequantize_row_q4_K of the oracle's GGML bytes
    equals, bit for bit, fp16(d)*s*c - fp16(dmin)*m formed in FP32 from the
    oracle's logical codes and metadata (reference.hpp:253-275)."""
    w = random_q4k(9, 512, 11)
    assert np.array_equal(oracle.Q4K.from_ggml(w.ggml(), 9, 512).codes, w.codes)
    R = oracle.ref()
    if R is None:
        pytest.skip("oracle/_ref not built (reference tree absent); the golden fixture test covers this")
    blk = w.ggml()
    deq = np.zeros(9 * 512, np.float32)
    R.ref_dequantize_row_q4_K(blk.ctypes.data, deq.ctypes.data, 9 * 512)
    d = _fp16_bits_to_f32(w.meta[..., 0].astype(np.uint16) | (w.meta[..., 1].astype(np.uint16) << 8))
    dm = _fp16_bits_to_f32(w.meta[..., 2].astype(np.uint16) | (w.meta[..., 3].astype(np.uint16) << 8))
    s, m = _sm_all(w.meta)
    d1 = (d[..., None] * s).astype(np.float32)          # [n][kb][8]
    m1 = (dm[..., None] * m).astype(np.float32)
    c = w.codes.reshape(9, 2, 8, 32).astype(np.float32)
    mine = (d1[..., None] * c).astype(np.float32) - m1[..., None]
    assert np.array_equal(mine.astype(np.float32).reshape(-1).view(np.uint32), deq.view(np.uint32))


def test_q6k_ggml_byte_order_single_bit_coordinates():
    """Each of the 210*8 source bits of a GGML Q6_K block, flipped alone, moves
    exactly the weight bit, scale byte or d bit that ggml's dequantize_row_q6_K
    index expressions name (tests/_fix.py ggml_q6k_coord, restated from the
    published format, not from the oracle); and each logical bit, set alone,
    lands on exactly that source bit. A swapped ql/qh interleave, a wrong qh
    shift or a misplaced scales/d offset fails here."""
    where = {}
    for i in range(256):
        ql, nib, qh, sh, _ = ggml_q6k_coord(i)
        for b in range(4):
            where[(ql, nib + b)] = ("q", i, b)
        for b in range(2):
            where[(qh, sh + b)] = ("q", i, 4 + b)
    for j in range(16):
        for b in range(8):
            where[(192 + j, b)] = ("sc", j, b)
    for b in range(16):
        where[(208 + b // 8, b % 8)] = ("d", 0, b)
    assert len(where) == 210 * 8, "every source bit has exactly one destination"
    for (byte, bit), (kind, idx, vb) in where.items():
        blk = np.zeros(210, np.uint8)
        blk[byte] = 1 << bit
        w = oracle.Q6K.from_ggml(blk, 1, 256)
        q = np.zeros(256, np.uint8)
        sc = np.zeros(16, np.uint8)
        d = 0
        if kind == "q":
            q[idx] = 1 << vb
        elif kind == "sc":
            sc[idx] = 1 << vb
        else:
            d = 1 << vb
        assert np.array_equal(w.q[0], q), (byte, bit)
        assert np.array_equal(w.sc[0].view(np.uint8), sc), (byte, bit)
        assert int(w.d[0, 0]) == d, (byte, bit)
        # and the other direction: the logical bit alone lands on (byte, bit)
        back = oracle.Q6K(q.reshape(1, 256), sc.view(np.int8).reshape(1, 16),
                          np.array([[d]], np.uint16), 1, 256).ggml()
        assert np.array_equal(back, blk), (byte, bit)


def test_q6k_ggml_random_blocks_against_published_decode():
    """Random GGML bytes decode the same through the oracle and through the
    published expressions; logical -> GGML -> logical is lossless."""
    rng = np.random.Generator(np.random.PCG64(31))
    blk = rng.integers(0, 256, size=(37, 210), dtype=np.uint8)
    q, sc, d = ggml_q6k_decode(blk)
    w = oracle.Q6K.from_ggml(blk.reshape(-1), 37, 256)
    assert np.array_equal(w.q, q) and np.array_equal(w.sc, sc) and np.array_equal(w.d[:, 0], d)
    assert np.array_equal(w.ggml(), blk.reshape(-1))
    q6 = random_q6k(7, 512, 3)
    back = oracle.Q6K.from_ggml(q6.ggml(), 7, 512)
    assert np.array_equal(back.q, q6.q) and np.array_equal(back.sc, q6.sc) and np.array_equal(back.d, q6.d)
    co, mo = q6.physical()
    back = oracle.Q6K.from_physical(co, mo, 7, 512)
    assert np.array_equal(back.q, q6.q) and np.array_equal(back.sc, q6.sc)


# ---- contractions ---------------------------------------------------------------------
def test_q4k_contract_brute_force_dots_and_closed_form():
    w = ref_fixture_weight()
    m = 3
    q = oracle.pack_q8(ref_fixture_input(m), m, REF_K)
    out64, out32, dots = oracle.q4k_q8_contract(w, q, want_dots=True)
    brute = np.einsum("rgk,tgk->trg", w.codes.reshape(REF_N, -1, 32).astype(np.int64),
                      q.codes.reshape(m, -1, 32).astype(np.int64))
    assert np.array_equal(dots, brute)
    assert np.abs(dots).max() <= 32 * 15 * 127
    # closed form in float64 from an independent numpy decode of the metadata
    d = np.array([[L.orc_fp16_to_fp32(int(mb[0]) | int(mb[1]) << 8) for mb in row] for row in w.meta])
    dm = np.array([[L.orc_fp16_to_fp32(int(mb[2]) | int(mb[3]) << 8) for mb in row] for row in w.meta])
    s = np.array([[_sm(mb, g)[0] for mb in row for g in range(8)] for row in w.meta], np.float64)
    mn = np.array([[_sm(mb, g)[1] for mb in row for g in range(8)] for row in w.meta], np.float64)
    ds = (np.repeat(d, 8, axis=1) * s)
    dmm = (np.repeat(dm, 8, axis=1) * mn)
    ref = np.einsum("tg,trg->tr", q.scales.astype(np.float64),
                    ds[None] * dots - dmm[None] * q.sums.astype(np.float64)[:, None, :])
    assert np.allclose(out64, ref, rtol=1e-6, atol=1e-6)
    assert np.allclose(out32, out64, rtol=1e-4, atol=1e-3)


def test_q6k_contract_equals_dequantized_dot():
    w = random_q6k(21, 512, 1)
    x = oracle.fp32_to_bf16(normal((3, 512), 2))
    q = oracle.pack_q8(x, 3, 512)
    out64, _, dots = oracle.q6k_q8_contract(w, q, want_dots=True)
    z = q.codes.astype(np.float64) * np.repeat(q.scales.astype(np.float64), 32, axis=1)
    ref = z @ w.dequantize().T
    assert np.allclose(out64, ref, rtol=1e-6, atol=1e-5)
    # integer form of the per-group value
    qq = w.q.astype(np.int64) - 32
    s = w.sc.astype(np.int64)
    zz = q.codes.astype(np.int64)
    brute = np.einsum("rgk,tgk->trg", (qq * np.repeat(s, 16, axis=1)).reshape(21, -1, 32),
                      zz.reshape(3, -1, 32))
    assert np.array_equal(dots, brute)


def test_q6k_fitter_invariants():
    x = normal((16, 512), 5, 0.02)
    q = oracle.quantize_q6k(x)
    assert q.q.max() <= 63
    err = np.abs(q.dequantize() - x)
    assert err.max() < 0.01 and err.mean() < 1e-3
    z = oracle.quantize_q6k(np.zeros((1, 256), np.float32))
    assert np.all(z.d == 0) and np.all(z.sc == 0) and np.all(z.q == 0)


# ---- Q6_K fitter pins ------------------------------------------------------
# The fitter restates llama.cpp quantize_row_q6_K_ref at e6ab7c1a4 (MIT), which
# the reference does not vendor (third_party/llama.cpp-q4k/README.md:27-54):
# per 16-element sub-block, make_qx_quants(n=16, nmax=32, rmse_type=1,
# weights x^2) picks the signed scale whose extreme element maps to -32
# (iscale = -32/max, then 18 perturbed iscales -(32 + 0.1 i)/max refined by
# weighted least squares); the block's largest-magnitude sub-block scale maps to
# -128 (iscale = -128/max_scale, d = fp16(1/iscale)); sc = min(127,
# nearest(iscale * scale)); finally q = clamp(nearest(x / (d sc)), -32, 31) + 32.
# nearest() rounds half to even (the 1.5 * 2^23 bias trick). The checks below
# pin each step with a property a plausible mistake breaks.


def _fp16_bits_to_f32(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def _exact_q6k_blocks(nblocks, seed):
    """Blocks that are exactly d * sc_j * (q - 32): d a normal fp16, sc_j
    nonzero with exactly one sub-block at -128 (the largest magnitude), every
    sub-block holding a q = 0 element (its extreme value, -32 d sc_j)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    d = rng.integers(0x1000, 0x2400, size=nblocks).astype(np.uint16)
    sc = rng.integers(-127, 128, size=(nblocks, 16))
    sc[sc == 0] = 1
    sc[np.arange(nblocks), rng.integers(0, 16, size=nblocks)] = -128
    q = rng.integers(1, 64, size=(nblocks, 16, 16))
    q[np.arange(nblocks)[:, None], np.arange(16)[None, :], rng.integers(0, 16, size=(nblocks, 16))] = 0
    dd = _fp16_bits_to_f32(d)[:, None] * sc.astype(np.float32)  # exact: 11-bit x 8-bit
    x = (dd[:, :, None] * (q - 32).astype(np.float32)).astype(np.float32)  # exact
    return x.reshape(nblocks, 256), d, sc.astype(np.int8), q.reshape(nblocks, 256).astype(np.uint8)


def test_q6k_fitter_recovers_exact_blocks():
    """A block built exactly from (d, sc, q) comes back byte-exact: pins the
    sign convention (extreme -> -32), the -128 mapping of the largest scale,
    the fp16 rounding of d, the sc rounding and the final code mapping
    (an off-by-one in the -32 offset or a dropped clamp fails here)."""
    x, d, sc, q = _exact_q6k_blocks(512, 77)
    got = oracle.quantize_q6k(x.reshape(-1, 256))
    assert np.array_equal(got.d.reshape(-1), d)
    assert np.array_equal(got.sc.reshape(-1, 16), sc)
    assert np.array_equal(got.q.reshape(-1, 256), q)
    assert np.array_equal(got.dequantize().astype(np.float32).reshape(-1, 256), x)


def test_q6k_fitter_final_step_and_scale_map():
    """On random N(0, 0.02) rows: every code is the clamped round-half-even
    nearest of x / (d sc) (llama.cpp's last pass), restated here in float32
    numpy; the largest-magnitude sub-block scale of each block is -128; and the
    per-sub-block reconstruction error is at most d |sc| / 2 except where the
    clamp at +31 applies."""
    x = normal((64, 1024), 9, 0.02).reshape(-1, 256)
    w = oracle.quantize_q6k(x)
    d = _fp16_bits_to_f32(w.d.reshape(-1))
    sc = w.sc.reshape(-1, 16).astype(np.float32)
    q = w.q.reshape(-1, 16, 16).astype(np.int32)
    dd = (d[:, None] * sc).astype(np.float32)
    xs = x.reshape(-1, 16, 16)
    with np.errstate(divide="ignore", invalid="ignore"):
        l = np.rint((xs / dd[:, :, None]).astype(np.float32))
    expect = np.clip(l, -32, 31) + 32
    live = dd != 0
    assert np.array_equal(q[live], expect[live].astype(np.int32))
    assert np.all(np.abs(w.sc.reshape(-1, 16).astype(np.int32)).max(axis=1) == 128)
    assert np.all(w.sc.reshape(-1, 16).min(axis=1) == -128)
    rec = dd[:, :, None] * (q - 32).astype(np.float32)
    err = np.abs(rec - xs)
    unclamped = (l > -32.5) & (l < 31.5)
    tol = np.abs(dd)[:, :, None] / 2 * (1 + 2 ** -20)
    assert np.all((err <= tol) | ~unclamped)


def _qx_candidates(x, weighted=True, n_perturb=9):
    """Every candidate of make_qx_quants(n=16, nmax=32): iscale = -32/max and
    -(32 + 0.1 i)/max for i = +-1..+-n_perturb, in the float32 arithmetic of
    the C source; codes clamped to [-32, 31]; the weighted (w = x^2, or 1)
    least-squares fit of each evaluated in float64."""
    x = x.astype(np.float32)
    mx = x[np.argmax(np.abs(x))]
    out = []
    for i in [0] + [j for j in range(-n_perturb, n_perturb + 1) if j]:
        iscale = np.float32(-(np.float32(32) + np.float32(0.1) * np.float32(i))) / mx
        l = np.clip(np.rint((iscale * x).astype(np.float32)), -32, 31).astype(np.float64)
        w = x.astype(np.float64) ** 2 if weighted else np.ones(16)
        sumlx, suml2 = float((w * x * l).sum()), float((w * l * l).sum())
        out.append((sumlx * sumlx / suml2 if suml2 > 0 else -1.0, l, sumlx / suml2 if suml2 else 0.0))
    return out


def _qx_best(x, **kw):
    c = _qx_candidates(x, **kw)
    merit = np.array([m for m, _, _ in c])
    best = int(np.argmax(merit))  # first maximum, as the strict '>' of the C loop keeps it
    # relative margin to the best candidate whose codes differ (equal codes tie exactly)
    other = [m for m, l, _ in c if not np.array_equal(l, c[best][1])]
    top = merit[best]
    gap = (top - max(other)) / top if other and top > 0 else 1.0
    return c[best], gap


def test_q6k_subblock_search_against_brute_force():
    """The sub-block search of the Q6_K fitter (llama.cpp make_qx_quants with
    rmse_type=1 at e6ab7c1a4) against an independent float64 brute force of its
    19 candidates: the chosen codes are the candidate with the largest
    x^2-weighted sumlx^2/suml2 and the scale is that candidate's sumlx/suml2.
    The same brute force, unweighted or with only 9 candidates, disagrees with
    the oracle on some sub-blocks, so a plausible slip in either is caught."""
    rng = np.random.Generator(np.random.PCG64(2024))
    xs = (rng.standard_normal((4000, 16)) * 0.02).astype(np.float32)
    xs[::7] *= rng.uniform(0.1, 10, size=(len(xs[::7]), 1)).astype(np.float32)
    checked = unweighted_differs = short_differs = 0
    for x in xs:
        L_ = np.zeros(16, np.uint8)
        scale = L.orc_q6k_fit_subblock(x.ctypes.data, L_.ctypes.data)
        (merit, l, s64), gap = _qx_best(x)
        if gap < 2e-6:   # float32 accumulation in the C code may order near-ties differently
            continue
        checked += 1
        assert np.array_equal(L_.astype(np.int64) - 32, l.astype(np.int64))
        assert abs(scale - s64) <= 2e-5 * abs(s64)
        (_, lu, _), _ = _qx_best(x, weighted=False)
        (_, ls, _), _ = _qx_best(x, n_perturb=4)
        unweighted_differs += not np.array_equal(lu, l)
        short_differs += not np.array_equal(ls, l)
    assert checked > 2400
    assert unweighted_differs > 50 and short_differs > 50
    # sign convention: the extreme element maps to -32 before refinement
    x = np.linspace(-1, 0.5, 16).astype(np.float32)
    L_ = np.zeros(16, np.uint8)
    L.orc_q6k_fit_subblock(x.ctypes.data, L_.ctypes.data)
    assert L_[0] == 0 and L.orc_q6k_fit_subblock(np.zeros(16, np.float32).ctypes.data, L_.ctypes.data) == 0


def test_linearity_of_contraction_in_activation_scale():
    """Doubling every activation scale doubles every output exactly (a dropped
    or misplaced scale factor breaks this)."""
    w = random_q4k(24, 512, 8)
    q = oracle.pack_q8(oracle.fp32_to_bf16(normal((2, 512), 9)), 2, 512)
    o1, _, _ = oracle.q4k_q8_contract(w, q)
    q.scales = q.scales * np.float32(2)
    o2, _, _ = oracle.q4k_q8_contract(w, q)
    assert np.array_equal(o2, 2 * o1)


# ---- producers -------------------------------------------------------------------------
def test_rms_q8_closed_form():
    rng = np.random.Generator(np.random.PCG64(3))
    res = (rng.standard_normal((3, 5120)) * 3).astype(np.float32)
    gamma = oracle.fp32_to_bf16((rng.standard_normal(5120) * 0.1).astype(np.float32))
    q, bf = oracle.rms_q8(res, gamma, 1e-6)
    assert not q.failed
    g = oracle.bf16_to_fp32(gamma).astype(np.float64)
    r64 = res.astype(np.float64)
    want = (1 + g) * r64 / np.sqrt(np.mean(r64 * r64, axis=1, keepdims=True) + 1e-6)
    got = oracle.bf16_to_fp32(bf).astype(np.float64)
    assert np.all(np.abs(got - want) <= np.abs(want) * 2 ** -7 + 1e-30)  # within 1 bf16 ulp
    q2 = oracle.pack_q8(bf, 3, 5120)
    assert np.array_equal(q2.codes, q.codes) and np.array_equal(q2.sums, q.sums)
    res[1, 77] = np.nan
    qn, _ = oracle.rms_q8(res, gamma, 1e-6)
    assert qn.failed


def test_swiglu_q8_closed_form():
    rng = np.random.Generator(np.random.PCG64(4))
    g = (rng.standard_normal((2, 512)) * 4).astype(np.float32)
    u = rng.standard_normal((2, 512)).astype(np.float32)
    q, bf = oracle.swiglu_q8(g, u)
    want = (g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))) * u
    got = oracle.bf16_to_fp32(bf).astype(np.float64)
    assert np.all(np.abs(got - want) <= np.abs(want) * 2 ** -7 + 1e-30)
    g[0, 3] = np.inf
    qn, _ = oracle.swiglu_q8(g, u)
    assert qn.failed


# ---- decode_mmv dense layouts (Q4G64, Q8G32, BF16 dense tile) ----------------
def _le16(a, i):
    return int(a[i]) | (int(a[i + 1]) << 8)


def _dense_logical(layout, n, k):
    g = oracle.dense_group(layout)
    return np.zeros((n, k), np.int8), np.zeros((n, k // g), np.uint16)


def test_dense_q4_golden_bytes():
    """tests/pack_layout_test.cpp:329-351: nibble order, signed nibbles, scale LE."""
    c, s = _dense_logical(0x0201, 8, 256)
    c[0, :6] = [1, 2, 3, 4, -1, 7]
    s[0, 0] = 0x3C00
    co, so = oracle.pack_dense(0x0201, c, s, 8, 256)
    assert co.size == 8 * 128 and so.size == 8 * 4 * 2
    assert (co[0], co[1], co[2]) == (0x21, 0x43, 0x7F)
    assert _le16(so, 0) == 0x3C00


def test_dense_q4_tile_coordinates_and_padding():
    """tests/pack_layout_test.cpp:353-400: (row 9, col 300) of 16x512 lands at
    byte 3222 (tn=1, tk=1, r=1, c=44), scale index [N/8, K/256, row, group];
    a 5x192 matrix pads to 8x256 with zero codes and zero padded-group scales."""
    c, s = _dense_logical(0x0201, 16, 512)
    c[9, 300] = 5
    s[9, 300 // 64] = 0x4200
    co, so = oracle.pack_dense(0x0201, c, s, 16, 512)
    assert co.size == 2 * 2 * 8 * 128
    assert co[3222] & 0x0F == 5 and np.count_nonzero(co) == 1
    si = ((1 * 2 + 1) * 8 + 1) * 4 + (44 // 64)
    assert _le16(so, 2 * si) == 0x4200
    c, s = _dense_logical(0x0201, 5, 192)
    c[0, 0], s[0, 0] = 3, 0x4000
    co, so = oracle.pack_dense(0x0201, c, s, 5, 192)
    assert co.size == 8 * 128 and so.size == 8 * 4 * 2
    assert co[0] == 3 and np.count_nonzero(co) == 1
    assert so[2] == 0 and so[3] == 0  # padded K group scale


def test_dense_q8_golden_bytes_and_coordinates():
    """tests/pack_layout_test.cpp:399-460: two's complement codes, eight scales
    per tile row, four-tile 16x512 placement."""
    c, s = _dense_logical(0x0202, 8, 256)
    c[0, :3] = [1, -1, -127]
    s[0, 0] = 0x3C00
    co, so = oracle.pack_dense(0x0202, c, s, 8, 256)
    assert co.size == 8 * 256 and so.size == 8 * 8 * 2
    assert (co[0], co[1], co[2]) == (1, 0xFF, 0x81)
    c, s = _dense_logical(0x0202, 16, 512)
    c[9, 300], c[15, 511] = -127, 126
    s[9, 300 // 32], s[15, 511 // 32] = 0x4200, 0x3555
    co, so = oracle.pack_dense(0x0202, c, s, 16, 512)
    tr = lambda row, col: ((row // 8) * 2 + col // 256) * 8 + row % 8
    assert co[tr(9, 300) * 256 + 300 % 256] == 0x81
    assert co[tr(15, 511) * 256 + 511 % 256] == 126
    i = tr(15, 511) * 8 + (511 % 256) // 32
    assert _le16(so, 2 * i) == 0x3555
    assert np.count_nonzero(co) == 2


@pytest.mark.parametrize("layout", [0x0201, 0x020B, 0x0202, 0x020C])
def test_dense_operands_equal_scaled_codes(layout):
    """Packer and decoder are restated independently; composing them must give
    BF16_RNE(code * scale) in logical order (0 for a zero scale), including
    padding (zero) and ragged shapes."""
    rng = np.random.Generator(np.random.PCG64(layout))
    g = oracle.dense_group(layout)
    n, k = 21, 5 * 64 if g == 64 else 7 * 32
    q4 = g == 64
    c = rng.integers(-8 if q4 else -127, 8 if q4 else 128, (n, k)).astype(np.int8)
    s = (rng.random((n, k // g)) * 2 - 1).astype(np.float16).view(np.uint16)
    s[0, 0] = 0  # zero scale
    s[1, 0] = 0x8000  # negative zero
    s[2, 0] = 0x0001  # subnormal scale
    co, so = oracle.pack_dense(layout, c, s, n, k)
    pn, pk = oracle.pad8(n), oracle.pad256(k)
    w = oracle.dense_operands(layout, co, so, pn, pk)
    scale = np.repeat(s.view(np.float16).astype(np.float32), g, axis=1)
    want = oracle.fp32_to_bf16(np.where(scale != 0, c.astype(np.float32) * scale, 0).astype(np.float32))
    assert np.array_equal(w[:n, :k], want)
    assert not w[n:].any() and not w[:, k:].any()


def test_dense_extreme_and_zero_cases():
    """tests/decode_mmv_unit_test.cpp:335-400: all-zero codes/scales give zero
    operands; code 127 with the largest FP16 scale 0x7BFF is BF16(127 * 65504)."""
    c, s = _dense_logical(0x0201, 8, 256)
    co, so = oracle.pack_dense(0x0201, c, s, 8, 256)
    assert not oracle.dense_operands(0x0201, co, so, 8, 256).any()
    c, s = _dense_logical(0x0202, 8, 256)
    c[:], s[:] = 127, 0x7BFF
    co, so = oracle.pack_dense(0x0202, c, s, 8, 256)
    w = oracle.dense_operands(0x0202, co, so, 8, 256)
    assert np.all(w == oracle.fp32_to_bf16(np.array([127.0 * 65504.0], np.float32))[0])


def test_bf16_tile_coordinates_roundtrip():
    """src/format/pack.cpp:247-290: element (row, col) at tile row
    ((row/8)*K/256 + col/256)*8 + row%8, offset 2*(col%256); the operand decoder
    inverts it exactly."""
    rng = np.random.Generator(np.random.PCG64(7))
    n, k = 16, 768
    w = rng.integers(0, 65536, (n, k)).astype(np.uint16)
    co = oracle.pack_bf16_tile(w, n, k)
    row, col = 11, 600
    tr = ((row // 8) * 3 + col // 256) * 8 + row % 8
    assert _le16(co, tr * 512 + 2 * (col % 256)) == w[row, col]
    assert np.array_equal(oracle.dense_operands(0x0203, co, None, n, k), w)


# ---- FP8 (OCP E4M3FN) ---------------------------------------------------------
def _value(code):
    """tests/fp8_test.cpp:34-38: independent E4M3 decode."""
    mag = code & 127
    e, f = mag >> 3, mag & 7
    v = np.ldexp(1.0 + f / 8.0, e - 7) if e else f / 512.0
    return -v if code & 128 else v


def _nearest(x):
    """tests/fp8_test.cpp:39-43: nearest code 0..126 by brute force, ties to
    the even code, sign from x."""
    best, err = 0, abs(x)
    for c in range(1, 127):
        e = abs(abs(x) - _value(c))
        if e < err or (e == err and not (c & 1)):
            err, best = e, c
    return best | (128 if np.signbit(x) else 0)


def test_e4m3_decode_all_codes():
    got = oracle.e4m3_to_fp32(np.arange(256))
    for c in range(256):
        if c & 127 == 127:
            assert np.isnan(got[c])
        else:
            assert got[c] == np.float32(_value(c)), c
    torch = pytest.importorskip("torch")
    t = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(t), np.isnan(got))
    fin = ~np.isnan(got)
    assert np.array_equal(t[fin].view(np.uint32), got[fin].view(np.uint32))


def test_e4m3_encode_rne_saturating():
    """Every code value, every midpoint between neighbours (ties), values just
    either side of them, subnormals, saturation and NaN."""
    vals = oracle.e4m3_to_fp32(np.arange(127)).astype(np.float64)
    mids = (vals[:-1] + vals[1:]) / 2
    xs = np.concatenate([vals, mids, np.nextafter(mids, 0), np.nextafter(mids, 1e9),
                         [448.0, 449.0, 464.0, 500.0, 1e30, 2.0 ** -10, 2.0 ** -11, 3 * 2.0 ** -11]])
    xs = np.concatenate([xs, -xs]).astype(np.float32)
    got = oracle.fp32_to_e4m3(xs)
    for x, g in zip(xs, got):
        assert g == _nearest(float(x)), (float(x), g)
    assert oracle.fp32_to_e4m3(np.array([np.nan], np.float32))[0] & 127 == 127
    torch = pytest.importorskip("torch")
    inr = np.abs(xs) <= 448
    t = torch.from_numpy(xs[inr]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(t, got[inr])


def test_pack_fp8_blocks():
    """tests/fp8_test.cpp:55-92 checks restated: per (row, 128-block) scale
    absmax/448 floored at the smallest normal, 1 for zero blocks; codes the RNE
    code of x/scale; zero tails; rows independent of each other; a nonfinite
    value makes its block's scale NaN."""
    m, k = 130, 387
    r = np.arange(m)[:, None]
    c = np.arange(k)[None, :]
    x = (((r * 23 + c * 17) % 97) - 48) * 0.03125 * (1 + r // 128 + c // 128)
    xb = oracle.fp32_to_bf16(x.astype(np.float32))
    xb[3, 5] = oracle.fp32_to_bf16(np.array([80.0], np.float32))[0]
    xb[7, :] = 0
    xb[9, 200] = 0x7F80  # +inf
    codes, scales = oracle.pack_fp8(xb, m, k)
    pm, pk = 256, 512
    assert codes.shape == (pm, pk) and scales.shape == (pk // 128, pm)
    xf = oracle.bf16_to_fp32(xb)
    for row in [0, 3, 7, 9, 100, 129]:
        for b in range(pk // 128):
            blk = xf[row, b * 128:min(k, b * 128 + 128)]
            if not np.all(np.isfinite(blk)):
                assert np.isnan(scales[b, row])
                continue
            peak = float(np.abs(blk).max()) if blk.size else 0.0
            want = 1.0 if peak == 0 else max(np.float32(peak) / np.float32(448), np.float32(2.0 ** -126))
            assert scales[b, row] == np.float32(want)
            for col in range(b * 128, min(k, b * 128 + 128), 37):
                assert codes[row, col] == _nearest(float(np.float32(xf[row, col]) / scales[b, row]))
    assert not codes[m:].any() and not codes[:, k:].any()
    one, s1 = oracle.pack_fp8(xb[3:4], 1, k)
    assert np.array_equal(one[0], codes[3]) and np.array_equal(s1[:, 0], scales[:, 3])


def test_fp8_contractions_closed_form():
    """The double closed forms agree with a dense numpy evaluation of the
    decoded operands (gemv and gemm, including the scale indexing)."""
    rng = np.random.Generator(np.random.PCG64(8))
    n, k, m = 256, 384, 5
    wc = rng.integers(0, 256, (n, k)).astype(np.uint8)
    wc[(wc & 127) == 127] = 0
    ws = rng.random((k // 128, n // 128)).astype(np.float32) + 0.5
    x = oracle.fp32_to_bf16(rng.standard_normal(k).astype(np.float32))
    y, _ = oracle.fp8_gemv(wc, ws, n, k, x)
    wd = oracle.e4m3_to_fp32(wc).astype(np.float64) * np.repeat(np.repeat(ws.T, 128, 0), 128, 1)
    assert np.allclose(y, wd @ oracle.bf16_to_fp32(x).astype(np.float64), rtol=1e-12, atol=1e-12)
    xc = rng.integers(0, 256, (m, k)).astype(np.uint8)
    xc[(xc & 127) == 127] = 1
    xs = rng.random((k // 128, m)).astype(np.float32)
    g, _ = oracle.fp8_gemm(wc, ws, n, k, xc, xs, m)
    xd = oracle.e4m3_to_fp32(xc).astype(np.float64) * np.repeat(xs.T, 128, 1)
    assert np.allclose(g, xd @ wd.T, rtol=1e-12, atol=1e-12)


# ---- NVFP4 (src/format/nvfp4.cpp, cuda/nvfp4_device.cuh) ---------------------
def _np_nvfp4_block(v):
    """Numpy restatement of one block, written independently of the oracle's
    exhaustive search: the scale through E4M3 RNE (orc_fp32_to_e4m3 on a
    nonnegative value), elements through the E2M1 tie table."""
    v = np.asarray(v, np.float32)
    if not np.all(np.isfinite(v)):
        return 127, np.zeros(16, np.uint8)
    peak = np.float32(np.abs(v).max())
    s = int(oracle.fp32_to_e4m3(np.array([peak / np.float32(6)], np.float32))[0])
    if peak != 0 and s == 0:
        s = 1
    scale = oracle.ue4m3_value(s)
    out = np.zeros(16, np.uint8)
    for i, x in enumerate(v):
        if x == 0:
            continue
        q = np.float32(x / scale)
        a = abs(float(q))
        mag = (0 if a <= .25 else 1 if a < .75 else 2 if a <= 1.25 else 3 if a < 1.75 else
               4 if a <= 2.5 else 5 if a < 3.5 else 6 if a <= 5 else 7)
        out[i] = mag | (8 if np.signbit(q) else 0)
    return s, out


def test_nvfp4_values_and_encoders():
    # nvfp4_e2m1 / nvfp4_e4m3 (src/format/nvfp4.cpp:8-16)
    assert list(oracle.e2m1_value(np.arange(8))) == [0, .5, 1, 1.5, 2, 3, 4, 6]
    assert list(oracle.e2m1_value(np.arange(8, 16))) == [-0.0, -.5, -1, -1.5, -2, -3, -4, -6]
    assert oracle.ue4m3_value(1) == 2.0 ** -9 and oracle.ue4m3_value(8) == 2.0 ** -6
    assert oracle.ue4m3_value(126) == 448.0
    # E2M1 ties to the even code (tests/nvfp4_test.cpp:139-140 tie set)
    ties = [.25, .75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0]
    want = [0, 2, 2, 4, 4, 6, 6, 7]
    assert [oracle.nvfp4_nearest(t, False) for t in ties] == want
    assert [oracle.nvfp4_nearest(-t, False) for t in ties] == [w | 8 for w in want]
    assert oracle.nvfp4_nearest(100.0, False) == 7 and oracle.nvfp4_nearest(-1e-3, False) == 8
    # the exhaustive UE4M3 search equals E4M3 RNE on nonnegative values:
    # every midpoint, both neighbours of it, and a log-uniform sample
    vals = [oracle.ue4m3_value(c) for c in range(127)]
    mids = [(a + b) / 2 for a, b in zip(vals, vals[1:])]
    rng = np.random.Generator(np.random.PCG64(5))
    probe = np.concatenate([np.array(mids, np.float32),
                            np.nextafter(np.array(mids, np.float32), np.float32(0)),
                            np.nextafter(np.array(mids, np.float32), np.float32(1e9)),
                            np.exp2(rng.uniform(-12, 10, 4000)).astype(np.float32),
                            np.array([0, 448, 460, 1e6], np.float32)])
    got = np.array([oracle.nvfp4_nearest(float(p), True) for p in probe])
    assert np.array_equal(got, oracle.fp32_to_e4m3(probe))


def test_nvfp4_scale_swizzle_bijection():
    # src/format/nvfp4.hpp:14-17: a bijection of (row, block) over pad128 rows,
    # 128-row stripes of pk/16 bytes, 512-byte chunks of four blocks
    pk, rows = 512, 256
    idx = np.array([[oracle.nvfp4_sf_index(r, b, pk) for b in range(pk // 16)] for r in range(rows)])
    assert np.array_equal(np.sort(idx.ravel()), np.arange(rows * pk // 16))
    assert np.all(idx[:128].max() < 128 * pk // 16) and np.all(idx[128:].min() >= 128 * pk // 16)
    # one chunk = rows 0..127 x blocks 0..3: contiguous 512 bytes
    assert sorted(idx[:128, :4].ravel()) == list(range(512))
    assert oracle.nvfp4_sf_index(33, 5, 512) == 512 + 16 + 4 + 1


def test_nvfp4_pack_blocks_and_fixtures():
    rng = np.random.Generator(np.random.PCG64(6))
    m, k = 5, 387   # ragged K (pk 512), rows padded to 128 in the scales
    x = oracle.fp32_to_bf16((rng.standard_normal((m, k)) * 3).astype(np.float32))
    x[1, :] = 0
    x[2, 40] = 0x7F80                       # +inf: block 2 of row 2 gets scale 127
    # tests/nvfp4_test.cpp:133-140: midpoints of consecutive scales x 6, ties
    for b in range(1, 8):
        x[3, 16 * b:16 * b + 16] = oracle.fp32_to_bf16(
            np.float32((oracle.ue4m3_value(b) + oracle.ue4m3_value(b + 1)) * 3))
    t = np.array([.25, .75, 1.25, 1.75, 2.5, 3.5, 5., 6.], np.float32)
    x[4, 256:272] = oracle.fp32_to_bf16(np.concatenate([t, -t]))
    codes, scales = oracle.pack_nvfp4(x, m, k)
    pk = 512
    xf = np.zeros((m, pk), np.float32)
    xf[:, :k] = oracle.bf16_to_fp32(x)
    for r in range(128):
        for b in range(pk // 16):
            si = oracle.nvfp4_sf_index(r, b, pk)
            if r >= m:
                assert scales[si] == 0
                continue
            s, c = _np_nvfp4_block(xf[r, 16 * b:16 * b + 16])
            assert scales[si] == s, (r, b)
            got = np.zeros(16, np.uint8)
            got[0::2] = codes[r, 8 * b:8 * b + 8] & 15
            got[1::2] = codes[r, 8 * b:8 * b + 8] >> 4
            assert np.array_equal(got, c), (r, b)
    assert scales[oracle.nvfp4_sf_index(2, 2, pk)] == 127
    assert np.all(codes[2, 16:24] == 0)


def test_nvfp4_quantizer_invariants():
    rng = np.random.Generator(np.random.PCG64(7))
    n, k = 13, 300
    w = oracle.fp32_to_bf16((rng.standard_normal((n, k)) * 0.05).astype(np.float32))
    codes, scales = oracle.quantize_nvfp4(w, n, k)
    pk, pn = 512, 16
    factor = scales[:4].view(np.float32)[0]
    peak = np.abs(oracle.bf16_to_fp32(w)).max()
    # power-of-two factor with peak / factor in (1344, 2688] (src/compiler/quantization/nvfp4.cpp:25-28)
    assert np.frexp(factor)[0] == 0.5 and 1344 < peak / factor <= 2688
    assert np.all(scales[4:256] == 0)
    # padding rows and columns carry zero codes and zero scales
    assert np.all(codes[n:] == 0) and np.all(codes[:, (k + 1) // 2 + 8:] == 0)
    for r in range(pn, 128):
        assert scales[256 + oracle.nvfp4_sf_index(r, 0, pk)] == 0
    # reconstruction error: at most half an E2M1 step of the block scale
    wf = oracle.bf16_to_fp32(w)
    for r in range(n):
        for c in range(0, k, 7):
            sf = scales[256 + oracle.nvfp4_sf_index(r, c // 16, pk)]
            code = (codes[r, c // 2] >> (4 * (c & 1))) & 15
            rec = factor * oracle.ue4m3_value(sf) * oracle.e2m1_value(code)
            assert abs(rec - wf[r, c]) <= factor * oracle.ue4m3_value(sf) * 1.0 + 1e-30
    with pytest.raises(ValueError):
        bad = w.copy()
        bad[0, 0] = 0x7FC0
        oracle.quantize_nvfp4(bad, n, k)


def _nvfp4_dense(codes, scales, rows, pk, header):
    """Dequantize in float64 from the layout definition."""
    nib = np.zeros((rows, pk), np.uint8)
    nib[:, 0::2] = codes[:rows] & 15
    nib[:, 1::2] = codes[:rows] >> 4
    sf = np.array([[scales[header + oracle.nvfp4_sf_index(r, b, pk)] for b in range(pk // 16)]
                   for r in range(rows)])
    return oracle.e2m1_value(nib).astype(np.float64) * np.repeat(oracle.ue4m3_value(sf), 16, axis=1)


def test_nvfp4_contractions_closed_form():
    rng = np.random.Generator(np.random.PCG64(8))
    n, k, m = 24, 512, 5
    wc, ws = oracle.quantize_nvfp4(oracle.fp32_to_bf16(rng.standard_normal((n, k)).astype(np.float32)), n, k)
    x = oracle.fp32_to_bf16(rng.standard_normal((m, k)).astype(np.float32))
    xc, xs = oracle.pack_nvfp4(x, m, k)
    factor = float(ws[:4].view(np.float32)[0])
    W = _nvfp4_dense(wc, ws, n, k, 256)
    A = _nvfp4_dense(xc, xs, m, k, 0)
    y, l1 = oracle.nvfp4_gemm(wc, ws, n, k, xc, xs, m)
    assert np.allclose(y, factor * (A @ W.T), rtol=1e-12, atol=1e-12)
    assert np.all(l1 >= np.abs(y) - 1e-9)
    # decode: FP32 element RN(RN(scale * factor) * value), times BF16 x
    sf = np.array([[ws[256 + oracle.nvfp4_sf_index(r, b, k)] for b in range(k // 16)] for r in range(n)])
    sc = (oracle.ue4m3_value(sf) * np.float32(factor)).astype(np.float32)
    nib = np.zeros((n, k), np.uint8)
    nib[:, 0::2] = wc[:n] & 15
    nib[:, 1::2] = wc[:n] >> 4
    wf = (np.repeat(sc, 16, axis=1) * oracle.e2m1_value(nib)).astype(np.float32)
    yd, _ = oracle.nvfp4_gemv(wc, ws, n, k, x[0], k)
    assert np.allclose(yd, wf.astype(np.float64) @ oracle.bf16_to_fp32(x[0]).astype(np.float64),
                       rtol=1e-12, atol=1e-12)
