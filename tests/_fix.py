"""Shared fixtures: the reference tests' deterministic inputs restated as data
formulas, plus seeded synthetic weights/activations for the BASELINE shapes."""
from __future__ import annotations

import numpy as np

import oracle

# ---- tests/q4k_q8_test.cpp:36-60 (N=137, K=259 odd-shape fixture) -----------
REF_N, REF_K = 137, 259


def ref_fixture_weight() -> oracle.Q4K:
    n, k = REF_N, REF_K
    pk = oracle.pad256(k)
    codes = np.zeros((n, pk), np.uint8)
    meta = np.zeros((n, pk // 256, 16), np.uint8)
    c = np.arange(k)
    for r in range(n):
        codes[r, :k] = (r * 7 + c * 11) % 16
        for b in range(2):
            dh = 1 if r == 0 else [0x1400, 0x1800, 0x1A00][r % 3]
            mh = 2 if r == 0 else (0x1000 if b == 0 else 0x1400)
            m = meta[r, b]
            m[0], m[1], m[2], m[3] = dh & 255, dh >> 8, mh & 255, mh >> 8
            p = m[4:]
            for g in range(8):
                s = (r * 13 + g * 17 + 3) % 64
                mn = (r * 11 + g * 7 + 5) % 64
                if g < 4:
                    p[g] |= s
                    p[g + 4] |= mn
                else:
                    p[g + 4] |= (s & 15) | ((mn & 15) << 4)
                    p[g - 4] |= (s >> 4) << 6
                    p[g] |= (mn >> 4) << 6
    return oracle.Q4K(codes, meta, n, k)


def ref_fixture_input(m: int) -> np.ndarray:
    """BF16 bits [m][259] of the reference fixture rows."""
    k = REF_K
    x = np.zeros((m, k), np.float32)
    c = np.arange(k)
    head = np.array([127.0, 0.5, 1.5, -0.5, -1.5], np.float32)
    for r in range(m):
        v = (((r * 23 + c * 19) % 67).astype(np.int64) - 44) * 0.125 * (1 + r % 5)
        v = v.astype(np.float32)
        v[32:64] = 0
        v[:5] = head
        if r == 2:
            v[:] = 0
        x[r] = v
    return oracle.fp32_to_bf16(x)


# ---- seeded synthetic data -------------------------
def normal(shape, seed, scale=1.0):
    rng = np.random.Generator(np.random.PCG64(seed))
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float32)


def outlier_rows(m, k, seed, frac=0.01, factor=20.0):
    """~N(0,1) rows with a fixed seeded 1% of channels scaled by 20 (config 2)."""
    x = normal((m, k), seed)
    rng = np.random.Generator(np.random.PCG64(seed + 7))
    ch = rng.choice(k, size=max(1, int(round(frac * k))), replace=False)
    x[:, ch] *= np.float32(factor)
    return x


def silu_rows(m, k, seed):
    """SiLU(a) * b with a, b ~N(0,1) (config 3 down-projection input)."""
    a = normal((m, k), seed)
    b = normal((m, k), seed + 1)
    return (a / (1 + np.exp(-a)) * b).astype(np.float32)


def random_q4k(n, k, seed) -> oracle.Q4K:
    """Random but valid logical Q4_K (fast; skips the fitter): codes 0..15,
    6-bit scales/mins, fp16 d ~ 2^-9..2^-7, dmin ~ 2^-9..2^-8."""
    rng = np.random.Generator(np.random.PCG64(seed))
    pk = oracle.pad256(k)
    codes = rng.integers(0, 16, size=(n, pk), dtype=np.uint8)
    codes[:, k:] = 0
    meta = rng.integers(0, 256, size=(n, pk // 256, 16), dtype=np.uint8)
    d = rng.integers(0x1800, 0x2000, size=(n, pk // 256), dtype=np.uint16)
    dm = rng.integers(0x1800, 0x1C00, size=(n, pk // 256), dtype=np.uint16)
    meta[..., 0] = d & 255
    meta[..., 1] = d >> 8
    meta[..., 2] = dm & 255
    meta[..., 3] = dm >> 8
    return oracle.Q4K(codes, meta, n, k)


def random_q6k(n, k, seed) -> oracle.Q6K:
    rng = np.random.Generator(np.random.PCG64(seed))
    q = rng.integers(0, 64, size=(n, k), dtype=np.uint8)
    sc = rng.integers(-128, 128, size=(n, k // 16), dtype=np.int8)
    d = rng.integers(0x0C00, 0x1400, size=(n, k // 256), dtype=np.uint16)
    return oracle.Q6K(q, sc, d, n, k)


def quantized_q4k(n, k, seed) -> oracle.Q4K:
    return oracle.quantize_q4k(normal((n, k), seed, 0.02))


def quantized_q6k(n, k, seed) -> oracle.Q6K:
    return oracle.quantize_q6k(normal((n, k), seed, 0.02))


# ---- published GGML Q6_K block (ggml-common.h block_q6_K) -------------------
# struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; ggml_half d; }
# = 210 bytes. ggml's dequantize_row_q6_K walks the block in two halves of
# 128 weights (ql += 64, qh += 32, sc += 8 per half) and, for l in 0..31 and
# is = l/16, reads
#   y[l +  0] = d*sc[is+0]*((ql[l   ] & 0xF) | ((qh[l] >> 0) & 3) << 4) - 32)
#   y[l + 32] = d*sc[is+2]*((ql[l+32] & 0xF) | ((qh[l] >> 2) & 3) << 4) - 32)
#   y[l + 64] = d*sc[is+4]*((ql[l   ] >>  4) | ((qh[l] >> 4) & 3) << 4) - 32)
#   y[l + 96] = d*sc[is+6]*((ql[l+32] >>  4) | ((qh[l] >> 6) & 3) << 4) - 32)
# The coordinates below are those expressions, written out per weight index.
def ggml_q6k_coord(i: int):
    """(ql byte, nibble shift 0/4, qh byte, qh shift, scale byte) that weight i
    of a 256-weight block reads, as byte offsets into the 210-byte block."""
    half, j = divmod(i, 128)
    quarter, l = divmod(j, 32)
    ql = 64 * half + l + (32 if quarter in (1, 3) else 0)
    nib = 0 if quarter in (0, 1) else 4
    qh = 128 + 32 * half + l
    return ql, nib, qh, 2 * quarter, 192 + 8 * half + l // 16 + 2 * quarter


def ggml_q6k_decode(blocks: np.ndarray):
    """Unsigned 6-bit codes q [blocks][256], int8 scales [blocks][16] and fp16
    d bits [blocks] of GGML Q6_K bytes, by the published index expressions."""
    b = np.asarray(blocks, np.uint8).reshape(-1, 210)
    q = np.zeros((b.shape[0], 256), np.uint8)
    for i in range(256):
        ql, nib, qh, sh, _ = ggml_q6k_coord(i)
        q[:, i] = ((b[:, ql] >> nib) & 15) | (((b[:, qh] >> sh) & 3) << 4)
    sc = b[:, 192:208].view(np.int8).copy()
    d = (b[:, 208].astype(np.uint16) | (b[:, 209].astype(np.uint16) << 8))
    return q, sc, d
