/*
 * CPU oracle for the Q4_K / Q6_K x Q8 projection path -- TEST INFRASTRUCTURE.
 *
 * Loaded only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg, as the checker or as the timed CPU baseline; never by the product.
 *
 * Restated reference algorithms and how each is pinned:
 *   orc_fp16_to_fp32      src/format/floatcvt.hpp:17-41. Pinned: exhaustive
 *                         65536-pattern equality against the pinned llama.cpp
 *                         header (oracle/_ref) and fixtures.
 *   orc_fp32_to_fp16      third_party/llama.cpp-q4k/reference.hpp:58-82 (IEEE
 *                         round-to-nearest-even). Pinned: random + edge sweep vs
 *                         oracle/_ref; fixture.
 *   orc_fp32_to_bf16_rne  src/format/floatcvt.hpp:82-95. Pinned: closed form
 *                         (ties, NaN quieting) in tests.
 *   orc_nearest_int       reference.hpp:86-91. Pinned vs oracle/_ref and rint().
 *   orc_pack_q8           cuda/q8_device.cuh:6-25, cuda/q4k_q8.cu:44-50.
 *                         Pinned: the reference test's independent equation
 *                         tests/q4k_q8_test.cpp:83-94 (ties, saturation, zero
 *                         token, padding, NaN/Inf) as golden vectors.
 *   orc_rms_q8            cuda/activation.cu:134-190 (block 256, warp-32 tree
 *                         reductions, FMA contraction where nvcc contracts).
 *                         Pinned: closed-form RMS in double within 1 bf16 ulp,
 *                         invariants (scale invariance) -- exact tree order is
 *                         this restatement's own claim.
 *   orc_swiglu_q8         cuda/q4k_q8.cu:52-61 with orc_expf (Cody-Waite range
 *                         reduction + degree-7 Taylor polynomial) in place of
 *                         CUDA's expf. Pinned: orc_expf within 2 ulp of libm
 *                         over a sweep; NaN propagation.
 *   orc_quantize_q4k_*    src/compiler/quantization/q4k.cpp:186-278 and
 *                         reference.hpp:93-252. Pinned: byte equality with the
 *                         compiled pinned llama.cpp header (oracle/_ref) on the
 *                         reference test's blocks (tests/q4k_reference_test.cpp
 *                         :126-165) and committed fixtures.
 *   orc_q4k_*ggml*        reference.hpp:244-248, tests/q4k_reference_test.cpp:
 *                         55-59. Pinned: round trip + _ref dequantize equality.
 *   orc_pack_q4k_layout   src/format/pack.cpp:216-262 (0x020D). Pinned: golden
 *                         tile coordinates of tests/pack_layout_test.cpp:197-245
 *                         and lossless round trip. 0x0240 (this build's plane
 *                         order) pinned by round trip + explicit coordinates.
 *   orc_quantize_q6k_*    llama.cpp quantize_row_q6_K_ref / make_qx_quants
 *                         (ggml-quants.c at e6ab7c1a4, MIT, not vendored in the
 *                         reference; no reference vectors exist). Pinned by
 *                         the mathematics: blocks built exactly as
 *                         d*sc*(q-32) (one sub-block at sc=-128) come back
 *                         byte-exact; on random data every code is the clamped
 *                         round-half-even nearest of x/(d*sc) (restated in
 *                         numpy), the largest sub-block scale is -128, and the
 *                         error is <= d|sc|/2 off the clamp. The sub-block
 *                         search (orc_q6k_fit_subblock: 19 iscales, x^2-
 *                         weighted least squares) is pinned against an
 *                         independent float64 brute force that maximises
 *                         sumlx^2/suml2 over the candidates; unweighted and
 *                         9-candidate variants are shown to disagree with it.
 *   orc_q6k_*ggml*        ggml block_q6_K byte order (ggml-common.h:
 *                         ql[128], qh[64], scales[16], d). Pinned: every
 *                         source bit of a block is flipped alone and must move
 *                         exactly the weight that ggml's dequantize_row_q6_K
 *                         index expressions name (restated independently in
 *                         the test), for both conversion directions.
 *   orc_q4k_q8_contract   tests/q4k_q8_test.cpp:121-131 (double closed form),
 *                         cuda/q4k_q8.cu:97,140 (FP32 K32 order). Pinned: brute
 *                         force integer dots, closed form on the reference
 *                         test's hash fixture, linearity.
 *   orc_q6k_q8_contract   new (no reference code); closed form from the GGML
 *                         Q6_K dequantization. Pinned: equals a dequantize-then-
 *                         dot in double on random data.
 *   orc_q4k_bf16_*        cuda/decode_mmv.cu:121-140 (BF16 operand rebuild).
 *                         Pinned: one-hot operand fixture of
 *                         tests/decode_mmv_unit_test.cpp:405-478 restated.
 *   orc_pack_dense_layout src/format/pack.cpp:143-215 (Q4G64 / Q8G32 tiles).
 *                         Pinned: the golden bytes and coordinates of
 *                         tests/pack_layout_test.cpp:313-460 (nibble order,
 *                         two's complement, tile/row/group order, padding).
 *   orc_pack_bf16_tile    src/format/pack.cpp:247-290. Pinned: explicit
 *                         coordinates and lossless inverse via the operands.
 *   orc_dense_operands    cuda/decode_mmv.cu:92-180 (decode8 Q4 / Q8 / BF16).
 *                         Pinned: equals BF16_RNE(code * scale) computed from
 *                         the logical codes (packer and decoder restated
 *                         independently), zero and max-FP16 cases of
 *                         tests/decode_mmv_unit_test.cpp:335-400.
 *   orc_e4m3_*            OCP E4M3FN (cutlass::float_e4m3_t, cuda/fp8.cu:79).
 *                         Pinned: decode of all 256 codes and encode (RNE,
 *                         ties to the even code, saturation at 448) against
 *                         the independent value()/nearest() search of
 *                         tests/fp8_test.cpp:34-43 and torch.float8_e4m3fn.
 *   orc_pack_fp8          cuda/fp8.cu:64-81. Pinned: per-block absmax/448
 *                         closed form, zero tails, row independence and the
 *                         nonfinite rule, as tests/fp8_test.cpp:55-92 checks.
 *   orc_fp8_gemv/_gemm    cuda/fp8.cu:82-160 contraction in double; pinned as
 *                         the reference test's own closed form
 *                         (tests/fp8_test.cpp:105-116).
 *   orc_nvfp4_*           src/format/nvfp4.{hpp,cpp}, cuda/nvfp4_device.cuh,
 *                         src/compiler/quantization/nvfp4.cpp. Element/scale
 *                         values restate nvfp4_e2m1 / nvfp4_e4m3; the encoders
 *                         are the exhaustive nearest-value search the reference
 *                         test uses as its own oracle (tests/nvfp4_test.cpp:
 *                         47-56). Pinned: the UE4M3 search equals E4M3 RNE on
 *                         nonnegative values, the midpoint and tie fixtures of
 *                         tests/nvfp4_test.cpp:127-147, the scale swizzle is a
 *                         bijection with the documented stripe/chunk layout,
 *                         and the contraction is the reference test's double
 *                         closed form (tests/nvfp4_test.cpp:181-196).
 *
 * Build with -ffp-contract=off -fno-fast-math: every FMA here is explicit.
 */
#include "oracle.h"

#include <math.h>
#include <string.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ---- scalar conversions ------------------------------------------------ */
float orc_fp16_to_fp32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 31u, mant = h & 1023u;
  if (e == 0) {
    if (mant == 0) return u2f(sign);
    /* subnormal: value = mant * 2^-24 exactly representable in FP32 */
    float v = (float)mant * 0x1p-24f;
    return u2f(sign | f2u(v));
  }
  if (e == 31) return u2f(sign | 0x7f800000u | (mant << 13));
  return u2f(sign | ((e + 112u) << 23) | (mant << 13));
}

uint16_t orc_fp32_to_fp16(float f) {
  uint32_t u = f2u(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  uint32_t au = u & 0x7fffffffu;
  if (au > 0x7f800000u) return sign | 0x7e00u; /* NaN */
  if (au >= 0x477ff000u) return sign | 0x7c00u; /* rounds to >= 65520: Inf */
  if (au < 0x38800000u) {
    /* result is FP16 subnormal or zero: quantum 2^-24, RNE */
    float a = u2f(au);
    double q = (double)a * 16777216.0; /* exact */
    double r = nearbyint(q);           /* RNE in default mode */
    return sign | (uint16_t)r;
  }
  /* normal: keep 10 mantissa bits, RNE on the dropped 13 */
  uint32_t exp = (au >> 23) - 112u;
  uint32_t mant = au & 0x7fffffu;
  uint32_t h = (exp << 10) | (mant >> 13);
  uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
  return sign | (uint16_t)h;
}

float orc_bf16_to_fp32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t orc_fp32_to_bf16_rne(float x) {
  uint32_t b = f2u(x);
  if (((b >> 23) & 0xffu) == 0xffu) {
    uint16_t h = (uint16_t)(b >> 16);
    if (b & 0x7fffffu) h |= 0x40u;
    return h;
  }
  return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

/* Magic-number rounding: adding 1.5*2^23 leaves the RNE integer in the low
 * mantissa bits for |x| < 2^22. */
int orc_nearest_int(float x) {
  float v = x + 12582912.f;
  int32_t i;
  memcpy(&i, &v, 4);
  return (i & 0x007fffff) - 0x00400000;
}

/* exp by Cody-Waite reduction x = n*ln2 + r, |r| <= ln2/2, and a degree-7
 * Taylor polynomial in Horner form with explicit FMAs (Cephes constants for
 * the two-part ln2). The device SwiGLU producer evaluates the same steps. */
float orc_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return INFINITY;
  if (x < -103.972084045410f) return 0.0f;
  float n = rintf(x * 1.44269502162933349609375f);
  float r = fmaf(n, -0.693145751953125f, x);
  r = fmaf(n, -1.428606765330187045e-06f, r);
  float p = 1.98412698412698412698e-4f;        /* 1/5040 */
  p = fmaf(p, r, 1.38888888888888888889e-3f);  /* 1/720 */
  p = fmaf(p, r, 8.33333333333333333333e-3f);  /* 1/120 */
  p = fmaf(p, r, 4.16666666666666666667e-2f);  /* 1/24 */
  p = fmaf(p, r, 1.66666666666666666667e-1f);  /* 1/6 */
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)n);
}

/* ---- Q8 activation producers ------------------------------------------- */
static int pack_group(const float* x /*32*/, int8_t* z, float* a_out, int32_t* s_out) {
  float peak = 0.f;
  int finite = 1;
  for (int t = 0; t < 32; ++t) {
    if (isfinite(x[t])) { float v = fabsf(x[t]); if (v > peak) peak = v; }
    else finite = 0;
  }
  float a = peak == 0.f ? 1.f : peak / 127.f;
  int valid = finite && isfinite(a) && a > 0.f;
  int32_t sum = 0;
  for (int t = 0; t < 32; ++t) {
    int code = 0;
    if (valid) {
      float q = rintf(x[t] / a);
      code = q > 127.f ? 127 : q < -127.f ? -127 : (int)q;
    }
    z[t] = (int8_t)code;
    sum += code;
  }
  *a_out = valid ? a : u2f(0x7fc00000u);
  *s_out = sum;
  return !valid;
}

int orc_pack_q8_f32(const float* x, uint32_t m, uint32_t k, uint32_t pk,
                    int8_t* codes, float* scales, int32_t* sums) {
  int fail = 0;
  float buf[32];
  for (uint32_t r = 0; r < m; ++r)
    for (uint32_t g = 0; g < pk / 32; ++g) {
      for (int t = 0; t < 32; ++t) {
        uint32_t c = g * 32 + t;
        buf[t] = c < k ? x[(size_t)r * k + c] : 0.f;
      }
      size_t gi = (size_t)r * (pk / 32) + g;
      fail |= pack_group(buf, codes + gi * 32, scales + gi, sums + gi);
    }
  return fail;
}

int orc_pack_q8(const uint16_t* bf16, uint32_t m, uint32_t k, uint32_t pk,
                int8_t* codes, float* scales, int32_t* sums) {
  int fail = 0;
  float buf[32];
  for (uint32_t r = 0; r < m; ++r)
    for (uint32_t g = 0; g < pk / 32; ++g) {
      for (int t = 0; t < 32; ++t) {
        uint32_t c = g * 32 + t;
        buf[t] = c < k ? orc_bf16_to_fp32(bf16[(size_t)r * k + c]) : 0.f;
      }
      size_t gi = (size_t)r * (pk / 32) + g;
      fail |= pack_group(buf, codes + gi * 32, scales + gi, sums + gi);
    }
  return fail;
}

/* 32-lane shuffle-down tree: lane i adds lane i+off for off = 16..1. */
static float tree32_sum(float* v) {
  for (int off = 16; off; off >>= 1)
    for (int i = 0; i < off; ++i) v[i] = v[i] + v[i + off];
  return v[0];
}
static float tree32_max(float* v) {
  for (int off = 16; off; off >>= 1)
    for (int i = 0; i < off; ++i) v[i] = fmaxf(v[i], v[i + off]);
  return v[0];
}
/* 256-thread block reduction: per-warp tree, then warp 0 over 8 partials
 * padded with zeros to 32 lanes. */
static float block256(float* per_thread, int is_max) {
  float part[32];
  for (int w = 0; w < 8; ++w) {
    float lane[32];
    memcpy(lane, per_thread + 32 * w, sizeof lane);
    part[w] = is_max ? tree32_max(lane) : tree32_sum(lane);
  }
  for (int i = 8; i < 32; ++i) part[i] = 0.f;
  return is_max ? tree32_max(part) : tree32_sum(part);
}

int orc_rms_q8(const float* residual, const uint16_t* gamma, float eps,
               uint32_t m, int8_t* codes, float* scales, int32_t* sums,
               uint16_t* bf16_out) {
  enum { H = 5120, T = 256 };
  int fail = 0;
  float th[T];
  float y[H];
  for (uint32_t tok = 0; tok < m; ++tok) {
    const float* x = residual + (size_t)tok * H;
    for (int t = 0; t < T; ++t) {
      float s = 0.f;
      for (int i = t; i < H; i += T) s = fmaxf(s, fabsf(x[i]));
      th[t] = s;
    }
    float scale = block256(th, 1);
    float safe = scale == 0.f ? 1.f : scale;
    for (int t = 0; t < T; ++t) {
      float s = 0.f;
      for (int i = t; i < H; i += T) { float q = x[i] / safe; s = fmaf(q, q, s); }
      th[t] = s;
    }
    float sumsq = block256(th, 0);
    float se = sqrtf(eps) / safe;
    float inv = 1.0f / sqrtf(fmaf(se, se, sumsq / (float)H));
    for (int i = 0; i < H; ++i) {
      float g = orc_bf16_to_fp32(gamma[i]);
      float v = (1.0f + g) * ((x[i] / safe) * inv);
      uint16_t b = orc_fp32_to_bf16_rne(v);
      y[i] = orc_bf16_to_fp32(b);
      if (bf16_out) bf16_out[(size_t)tok * H + i] = b;
    }
    for (int g = 0; g < H / 32; ++g) {
      size_t gi = (size_t)tok * (H / 32) + g;
      fail |= pack_group(y + 32 * g, codes + gi * 32, scales + gi, sums + gi);
    }
  }
  return fail;
}

int orc_swiglu_q8(const float* gate, const float* up, uint32_t m, uint32_t n,
                  int8_t* codes, float* scales, int32_t* sums, uint16_t* bf16_out) {
  int fail = 0;
  float buf[32];
  for (size_t gi = 0; gi < (size_t)m * n / 32; ++gi) {
    for (int t = 0; t < 32; ++t) {
      size_t i = gi * 32 + t;
      float g = gate[i], u = up[i];
      float v = (g / (1.f + orc_expf(-g))) * u;
      if (!isfinite(g) || !isfinite(u)) v = u2f(0x7fc00000u);
      uint16_t b = orc_fp32_to_bf16_rne(v);
      if (bf16_out) bf16_out[i] = b;
      buf[t] = orc_bf16_to_fp32(b);
    }
    fail |= pack_group(buf, codes + gi * 32, scales + gi, sums + gi);
  }
  return fail;
}

/* ---- Q4_K quantizer ----------------------------------------------------- */
/* Weighted min/max affine fit over 32 values with a 21-step scale search
 * (reference.hpp:93-172). Updates of the running minimum feed later search
 * steps, exactly as the published routine does. */
static float fit_qkx2(const float* x, const float* w, uint8_t* L, float* the_min,
                      uint8_t* Laux) {
  const int n = 32, nmax = 15, nstep = 20;
  const float rmin = -1.f, rdelta = 0.1f;
  float mn = x[0], mx = x[0];
  float sum_w = w[0];
  float sum_x = sum_w * x[0];
  for (int i = 1; i < n; ++i) {
    if (x[i] < mn) mn = x[i];
    if (x[i] > mx) mx = x[i];
    float wi = w[i];
    sum_w += wi;
    sum_x += wi * x[i];
  }
  if (mn > 0) mn = 0;
  if (mx == mn) {
    for (int i = 0; i < n; ++i) L[i] = 0;
    *the_min = -mn;
    return 0.f;
  }
  float iscale = nmax / (mx - mn);
  float scale = 1 / iscale;
  float best = 0;
  for (int i = 0; i < n; ++i) {
    int l = orc_nearest_int(iscale * (x[i] - mn));
    L[i] = (uint8_t)(l < 0 ? 0 : l > nmax ? nmax : l);
    float diff = scale * L[i] + mn - x[i];
    diff = diff * diff;
    best += w[i] * diff;
  }
  for (int is = 0; is <= nstep; ++is) {
    iscale = (rmin + rdelta * is + nmax) / (mx - mn);
    float sl = 0, sl2 = 0, sxl = 0;
    for (int i = 0; i < n; ++i) {
      int l = orc_nearest_int(iscale * (x[i] - mn));
      l = l < 0 ? 0 : l > nmax ? nmax : l;
      Laux[i] = (uint8_t)l;
      float wi = w[i];
      sl += wi * l;
      sl2 += wi * l * l;
      sxl += wi * l * x[i];
    }
    float D = sum_w * sl2 - sl * sl;
    if (D > 0) {
      float ts = (sum_w * sxl - sum_x * sl) / D;
      float tm = (sl2 * sum_x - sl * sxl) / D;
      if (tm > 0) { tm = 0; ts = sxl / sl2; }
      float cur = 0;
      for (int i = 0; i < n; ++i) {
        float diff = ts * Laux[i] + tm - x[i];
        diff = diff * diff;
        cur += w[i] * diff;
      }
      if (cur < best) {
        for (int i = 0; i < n; ++i) L[i] = Laux[i];
        best = cur;
        scale = ts;
        mn = tm;
      }
    }
  }
  *the_min = -mn;
  return scale;
}

void orc_q4k_scale_min(const uint8_t* meta, unsigned g, unsigned* s, unsigned* m) {
  const uint8_t* p = meta + 4;
  if (g < 4) { *s = p[g] & 63u; *m = p[g + 4] & 63u; }
  else {
    *s = (p[g + 4] & 15u) | ((unsigned)(p[g - 4] >> 6) << 4);
    *m = (unsigned)(p[g + 4] >> 4) | ((unsigned)(p[g] >> 6) << 4);
  }
}

int orc_quantize_q4k_block(const float* x, uint8_t* codes, uint8_t* meta) {
  for (int i = 0; i < 256; ++i) {
    if (!isfinite(x[i])) return 1;
    if (fabsf(x[i]) > 1.0e10f) return 2;
  }
  uint8_t L[256], aux[32];
  float w[32], mins[8], scl[8];
  float max_scale = 0, max_min = 0;
  for (int j = 0; j < 8; ++j) {
    const float* xj = x + 32 * j;
    float lo = 0, hi = xj[0];
    for (int i = 0; i < 32; ++i) { lo = fminf(lo, xj[i]); hi = fmaxf(hi, xj[i]); }
    if (hi != lo && !isfinite(16.f / (hi - lo))) return 2;
    float sx2 = 0;
    for (int i = 0; i < 32; ++i) sx2 += xj[i] * xj[i];
    float av = sqrtf(sx2 / 32);
    for (int i = 0; i < 32; ++i) w[i] = av + fabsf(xj[i]);
    scl[j] = fit_qkx2(xj, w, L + 32 * j, &mins[j], aux);
    if (scl[j] > max_scale) max_scale = scl[j];
    if (mins[j] > max_min) max_min = mins[j];
  }
  float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
  float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
  if (!isfinite(inv_scale) || !isfinite(inv_min)) return 2;
  uint8_t* p = meta + 4;
  memset(p, 0, 12);
  for (int j = 0; j < 8; ++j) {
    uint8_t ls = (uint8_t)orc_nearest_int(inv_scale * scl[j]);
    uint8_t lm = (uint8_t)orc_nearest_int(inv_min * mins[j]);
    if (ls > 63) ls = 63;
    if (lm > 63) lm = 63;
    if (j < 4) { p[j] = ls; p[j + 4] = lm; }
    else {
      p[j + 4] = (uint8_t)((ls & 15) | ((lm & 15) << 4));
      p[j - 4] |= (uint8_t)((ls >> 4) << 6);
      p[j] |= (uint8_t)((lm >> 4) << 6);
    }
  }
  uint16_t d = orc_fp32_to_fp16(max_scale / 63.f);
  uint16_t dmin = orc_fp32_to_fp16(max_min / 63.f);
  if ((d & 0x7c00u) == 0x7c00u || (dmin & 0x7c00u) == 0x7c00u) return 2;
  meta[0] = d & 255; meta[1] = d >> 8; meta[2] = dmin & 255; meta[3] = dmin >> 8;
  for (int j = 0; j < 8; ++j) {
    unsigned sc, mm;
    orc_q4k_scale_min(meta, j, &sc, &mm);
    float step = orc_fp16_to_fp32(d) * sc;
    if (!step) continue;
    float off = orc_fp16_to_fp32(dmin) * mm;
    for (int i = 0; i < 32; ++i) {
      int l = orc_nearest_int((x[32 * j + i] + off) / step);
      L[32 * j + i] = (uint8_t)(l < 0 ? 0 : l > 15 ? 15 : l);
    }
  }
  memcpy(codes, L, 256);
  return 0;
}

int orc_quantize_q4k_rows(const float* x, uint64_t n, uint64_t k, uint8_t* codes,
                          uint8_t* meta, int threads) {
  if (k % 256) return 3;
  int64_t blocks = (int64_t)(n * (k / 256));
  int err = 0;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static) reduction(| : err)
#endif
  for (int64_t b = 0; b < blocks; ++b)
    err |= orc_quantize_q4k_block(x + b * 256, codes + b * 256, meta + b * 16);
  (void)threads;
  return err;
}

void orc_q4k_logical_to_ggml(const uint8_t* codes, const uint8_t* meta,
                             uint64_t blocks, uint8_t* ggml) {
  for (uint64_t b = 0; b < blocks; ++b) {
    uint8_t* y = ggml + b * 144;
    memcpy(y, meta + b * 16, 16);
    const uint8_t* c = codes + b * 256;
    for (int j = 0; j < 4; ++j)
      for (int l = 0; l < 32; ++l)
        y[16 + 32 * j + l] = (uint8_t)(c[64 * j + l] | (c[64 * j + 32 + l] << 4));
  }
}

void orc_q4k_ggml_to_logical(const uint8_t* ggml, uint64_t blocks, uint8_t* codes,
                             uint8_t* meta) {
  for (uint64_t b = 0; b < blocks; ++b) {
    const uint8_t* y = ggml + b * 144;
    memcpy(meta + b * 16, y, 16);
    uint8_t* c = codes + b * 256;
    for (int j = 0; j < 4; ++j)
      for (int l = 0; l < 32; ++l) {
        c[64 * j + l] = y[16 + 32 * j + l] & 15;
        c[64 * j + 32 + l] = y[16 + 32 * j + l] >> 4;
      }
  }
}

/* ---- layouts ------------------------------------------------------------ */
static inline uint64_t tile_row(uint32_t row, uint32_t kb, uint32_t kbs) {
  return ((uint64_t)(row / 8) * kbs + kb) * 8 + row % 8;
}
static inline uint32_t pad8(uint32_t n) { return (n + 7u) & ~7u; }

/* Byte j (0..15) of K32 group chunk -> the two logical code offsets it holds.
 * 0x020D: sequential pairs. 0x0240: word t holds codes 8t..8t+3 in its low
 * nibbles and 8t+4..8t+7 in its high nibbles. */
static inline void nib_map(uint16_t layout, int j, int* lo, int* hi) {
  if (layout == 0x020D) { *lo = 2 * j; *hi = 2 * j + 1; }
  else { int t = j / 4, i = j % 4; *lo = 8 * t + i; *hi = 8 * t + 4 + i; }
}

/* Byte offsets of the 16-byte code word of (row, super-block kb, K32 group g)
 * and of the 16-byte metadata row of (row, kb), for `strips` 8-row strips.
 * 0x020D: tile row ((row/8)*kbs + kb)*8 + row%8: 128 code bytes (group g at
 *   g*16) and 16 metadata bytes per tile row.
 * 0x0240: chunk-major. Super-blocks form chunks of nk <= 8 (only the last is
 *   short); chunk c of every strip is contiguous, strip after strip. Within
 *   (chunk, strip) the codes are eight planes of nk*128 B, one per group, with
 *   16-byte entries ordered (kb%8)*8 + row%8; the metadata is one such plane. */
static inline uint64_t code_word(uint16_t layout, uint32_t row, uint32_t kb, uint32_t g,
                                 uint32_t kbs, uint32_t strips) {
  if (layout == 0x020D) return tile_row(row, kb, kbs) * 128 + g * 16;
  uint32_t c = kb / 8, kq = kb % 8;
  uint32_t nk = kbs - 8 * c < 8 ? kbs - 8 * c : 8;
  return (uint64_t)strips * 8192 * c + (uint64_t)(row / 8) * nk * 1024 +
         (uint64_t)g * nk * 128 + (kq * 8 + row % 8) * 16;
}
static inline uint64_t meta_row(uint16_t layout, uint32_t row, uint32_t kb, uint32_t kbs,
                                uint32_t strips) {
  if (layout == 0x020D) return tile_row(row, kb, kbs) * 16;
  uint32_t c = kb / 8, kq = kb % 8;
  uint32_t nk = kbs - 8 * c < 8 ? kbs - 8 * c : 8;
  return (uint64_t)strips * 1024 * c + (uint64_t)(row / 8) * nk * 128 + (kq * 8 + row % 8) * 16;
}

int orc_pack_q4k_layout(uint16_t layout, const uint8_t* codes, const uint8_t* meta,
                        uint32_t n, uint32_t pk, uint8_t* co, uint8_t* mo) {
  if ((layout != 0x020D && layout != 0x0240) || pk % 256) return 1;
  uint32_t kbs = pk / 256, pn = pad8(n);
  memset(co, 0, (size_t)pn * pk / 2);
  memset(mo, 0, (size_t)pn * kbs * 16);
  for (uint32_t r = 0; r < n; ++r)
    for (uint32_t kb = 0; kb < kbs; ++kb) {
      memcpy(mo + meta_row(layout, r, kb, kbs, pn / 8), meta + ((size_t)r * kbs + kb) * 16, 16);
      const uint8_t* c = codes + (size_t)r * pk + kb * 256;
      for (int g = 0; g < 8; ++g)
        for (int j = 0; j < 16; ++j) {
          int lo, hi;
          nib_map(layout, j, &lo, &hi);
          co[code_word(layout, r, kb, g, kbs, pn / 8) + j] =
              (uint8_t)(c[32 * g + lo] | (c[32 * g + hi] << 4));
        }
    }
  return 0;
}

int orc_unpack_q4k_layout(uint16_t layout, const uint8_t* ci, const uint8_t* mi,
                          uint32_t n, uint32_t pk, uint8_t* codes, uint8_t* meta) {
  if ((layout != 0x020D && layout != 0x0240) || pk % 256) return 1;
  uint32_t kbs = pk / 256;
  for (uint32_t r = 0; r < n; ++r)
    for (uint32_t kb = 0; kb < kbs; ++kb) {
      memcpy(meta + ((size_t)r * kbs + kb) * 16, mi + meta_row(layout, r, kb, kbs, pad8(n) / 8), 16);
      uint8_t* c = codes + (size_t)r * pk + kb * 256;
      for (int g = 0; g < 8; ++g)
        for (int j = 0; j < 16; ++j) {
          int lo, hi;
          nib_map(layout, j, &lo, &hi);
          uint8_t b = ci[code_word(layout, r, kb, g, kbs, pad8(n) / 8) + j];
          c[32 * g + lo] = b & 15;
          c[32 * g + hi] = b >> 4;
        }
    }
  return 0;
}

/* ---- Q6_K quantizer (llama.cpp quantize_row_q6_K_ref, published algorithm) */
#define Q6_GROUP_MAX_EPS 1e-15f
static float fit_qx(int n, int nmax, const float* x, uint8_t* L) {
  float max = 0, amax = 0;
  for (int i = 0; i < n; ++i) {
    float ax = fabsf(x[i]);
    if (ax > amax) { amax = ax; max = x[i]; }
  }
  if (amax < Q6_GROUP_MAX_EPS) {
    for (int i = 0; i < n; ++i) L[i] = 0;
    return 0.f;
  }
  float iscale = -nmax / max;
  float sumlx = 0, suml2 = 0;
  for (int i = 0; i < n; ++i) {
    int l = orc_nearest_int(iscale * x[i]);
    l = l < -nmax ? -nmax : l > nmax - 1 ? nmax - 1 : l;
    L[i] = (uint8_t)(l + nmax);
    float w = x[i] * x[i];
    sumlx += w * x[i] * l;
    suml2 += w * l * l;
  }
  float scale = suml2 ? sumlx / suml2 : 0.0f;
  float best = scale * sumlx;
  for (int is = -9; is <= 9; ++is) {
    if (is == 0) continue;
    iscale = -(nmax + 0.1f * is) / max;
    sumlx = suml2 = 0;
    for (int i = 0; i < n; ++i) {
      int l = orc_nearest_int(iscale * x[i]);
      l = l < -nmax ? -nmax : l > nmax - 1 ? nmax - 1 : l;
      float w = x[i] * x[i];
      sumlx += w * x[i] * l;
      suml2 += w * l * l;
    }
    if (suml2 > 0 && sumlx * sumlx > best * suml2) {
      for (int i = 0; i < n; ++i) {
        int l = orc_nearest_int(iscale * x[i]);
        l = l < -nmax ? -nmax : l > nmax - 1 ? nmax - 1 : l;
        L[i] = (uint8_t)(nmax + l);
      }
      scale = sumlx / suml2;
      best = scale * sumlx;
    }
  }
  return scale;
}

/* One 16-element sub-block's search, exposed so the tests can pin it against
 * an independent brute force of the 19 candidates. */
float orc_q6k_fit_subblock(const float* x, uint8_t* L) { return fit_qx(16, 32, x, L); }

void orc_quantize_q6k_block(const float* x, uint8_t* q, int8_t* sc, uint16_t* d) {
  uint8_t L[256];
  float scales[16];
  float max_scale = 0, max_abs = 0;
  for (int ib = 0; ib < 16; ++ib) {
    float s = fit_qx(16, 32, x + 16 * ib, L + 16 * ib);
    scales[ib] = s;
    float as = fabsf(s);
    if (as > max_abs) { max_abs = as; max_scale = s; }
  }
  if (max_abs < Q6_GROUP_MAX_EPS) {
    memset(q, 0, 256);
    memset(sc, 0, 16);
    *d = 0;
    return;
  }
  float iscale = -128.f / max_scale;
  *d = orc_fp32_to_fp16(1 / iscale);
  for (int ib = 0; ib < 16; ++ib) {
    int l = orc_nearest_int(iscale * scales[ib]);
    sc[ib] = (int8_t)(l < 127 ? l : 127);
  }
  for (int j = 0; j < 16; ++j) {
    float dd = orc_fp16_to_fp32(*d) * sc[j];
    if (!dd) continue;
    for (int i = 0; i < 16; ++i) {
      int l = orc_nearest_int(x[16 * j + i] / dd);
      l = l < -32 ? -32 : l > 31 ? 31 : l;
      L[16 * j + i] = (uint8_t)(l + 32);
    }
  }
  memcpy(q, L, 256);
}

int orc_quantize_q6k_rows(const float* x, uint64_t n, uint64_t k, uint8_t* q,
                          int8_t* sc, uint16_t* d, int threads) {
  if (k % 256) return 3;
  int64_t blocks = (int64_t)(n * (k / 256));
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
#endif
  for (int64_t b = 0; b < blocks; ++b)
    orc_quantize_q6k_block(x + b * 256, q + b * 256, sc + b * 16, d + b);
  (void)threads;
  return 0;
}

void orc_q6k_logical_to_ggml(const uint8_t* q, const int8_t* sc, const uint16_t* d,
                             uint64_t blocks, uint8_t* ggml) {
  for (uint64_t b = 0; b < blocks; ++b) {
    uint8_t* y = ggml + b * 210;
    const uint8_t* L = q + b * 256;
    uint8_t* ql = y;
    uint8_t* qh = y + 128;
    for (int half = 0; half < 2; ++half) {
      const uint8_t* Lh = L + 128 * half;
      uint8_t* qlh = ql + 64 * half;
      uint8_t* qhh = qh + 32 * half;
      for (int l = 0; l < 32; ++l) {
        qlh[l] = (uint8_t)((Lh[l] & 15) | ((Lh[l + 64] & 15) << 4));
        qlh[l + 32] = (uint8_t)((Lh[l + 32] & 15) | ((Lh[l + 96] & 15) << 4));
        qhh[l] = (uint8_t)((Lh[l] >> 4) | ((Lh[l + 32] >> 4) << 2) |
                           ((Lh[l + 64] >> 4) << 4) | ((Lh[l + 96] >> 4) << 6));
      }
    }
    memcpy(y + 192, sc + b * 16, 16);
    y[208] = d[b] & 255;
    y[209] = d[b] >> 8;
  }
}

void orc_q6k_ggml_to_logical(const uint8_t* ggml, uint64_t blocks, uint8_t* q,
                             int8_t* sc, uint16_t* d) {
  for (uint64_t b = 0; b < blocks; ++b) {
    const uint8_t* y = ggml + b * 210;
    uint8_t* L = q + b * 256;
    for (int half = 0; half < 2; ++half) {
      const uint8_t* qlh = y + 64 * half;
      const uint8_t* qhh = y + 128 + 32 * half;
      uint8_t* Lh = L + 128 * half;
      for (int l = 0; l < 32; ++l) {
        Lh[l] = (uint8_t)((qlh[l] & 15) | (((qhh[l] >> 0) & 3) << 4));
        Lh[l + 32] = (uint8_t)((qlh[l + 32] & 15) | (((qhh[l] >> 2) & 3) << 4));
        Lh[l + 64] = (uint8_t)((qlh[l] >> 4) | (((qhh[l] >> 4) & 3) << 4));
        Lh[l + 96] = (uint8_t)((qlh[l + 32] >> 4) | (((qhh[l] >> 6) & 3) << 4));
      }
    }
    memcpy(sc + b * 16, y + 192, 16);
    d[b] = (uint16_t)(y[208] | (y[209] << 8));
  }
}

/* Q6_K wave64 layout 0x0241. An 8-row x K256 tile (strip, kb) is 1536
 * contiguous code bytes at (strip*kbs + kb)*1536: the 1024 B low-nibble plane
 * (chunk c of 16 B per (row r, K32 group g), nibble order as 0x0240), then the
 * 512 B high-pair plane (chunk c of 8 B: word u, byte i, bits 2s..2s+1 hold
 * code 16u+4s+i), with c = (g/2)*16 + 2r + g%2, so the two groups of a pair
 * are adjacent for each row and one chunk per lane covers a plane.
 * Metadata: 16 int8 scales at tile_row*16, then the fp16 d array at
 * padded_n*kbs*16 + tile_row*2. */
static uint64_t q6_chunk(uint32_t r, uint32_t kb, uint32_t kbs, int g) {
  return ((uint64_t)(r / 8) * kbs + kb) * 64 + (uint64_t)((g / 2) * 16 + 2 * (r % 8) + g % 2);
}
int orc_pack_q6k_layout(const uint8_t* q, const int8_t* sc, const uint16_t* d,
                        uint32_t n, uint32_t pk, uint8_t* co, uint8_t* mo) {
  if (pk % 256) return 1;
  uint32_t kbs = pk / 256, pn = pad8(n);
  uint64_t rows = (uint64_t)pn * kbs;
  memset(co, 0, rows * 192);
  memset(mo, 0, rows * 18);
  for (uint32_t r = 0; r < n; ++r)
    for (uint32_t kb = 0; kb < kbs; ++kb) {
      uint64_t tr = tile_row(r, kb, kbs);
      size_t blk = (size_t)r * kbs + kb;
      memcpy(mo + tr * 16, sc + blk * 16, 16);
      mo[rows * 16 + tr * 2] = d[blk] & 255;
      mo[rows * 16 + tr * 2 + 1] = d[blk] >> 8;
      const uint8_t* c = q + (size_t)r * pk + kb * 256;
      for (int g = 0; g < 8; ++g) {
        const uint64_t ch = q6_chunk(r, kb, kbs, g);
        uint8_t* lo = co + (ch / 64) * 1536 + (ch % 64) * 16;
        uint8_t* hi = co + (ch / 64) * 1536 + 1024 + (ch % 64) * 8;
        const uint8_t* cg = c + 32 * g;
        for (int j = 0; j < 16; ++j) {
          int t = j / 4, i = j % 4;
          lo[j] = (uint8_t)((cg[8 * t + i] & 15) | ((cg[8 * t + 4 + i] & 15) << 4));
        }
        for (int u = 0; u < 2; ++u)
          for (int i = 0; i < 4; ++i) {
            uint8_t b = 0;
            for (int s = 0; s < 4; ++s) b |= (uint8_t)(((cg[16 * u + 4 * s + i] >> 4) & 3) << (2 * s));
            hi[4 * u + i] = b;
          }
      }
    }
  return 0;
}

int orc_unpack_q6k_layout(const uint8_t* ci, const uint8_t* mi, uint32_t n, uint32_t pk,
                          uint8_t* q, int8_t* sc, uint16_t* d) {
  if (pk % 256) return 1;
  uint32_t kbs = pk / 256, pn = pad8(n);
  uint64_t rows = (uint64_t)pn * kbs;
  for (uint32_t r = 0; r < n; ++r)
    for (uint32_t kb = 0; kb < kbs; ++kb) {
      uint64_t tr = tile_row(r, kb, kbs);
      size_t blk = (size_t)r * kbs + kb;
      memcpy(sc + blk * 16, mi + tr * 16, 16);
      d[blk] = (uint16_t)(mi[rows * 16 + tr * 2] | (mi[rows * 16 + tr * 2 + 1] << 8));
      uint8_t* c = q + (size_t)r * pk + kb * 256;
      for (int g = 0; g < 8; ++g) {
        const uint64_t ch = q6_chunk(r, kb, kbs, g);
        const uint8_t* lo = ci + (ch / 64) * 1536 + (ch % 64) * 16;
        const uint8_t* hi = ci + (ch / 64) * 1536 + 1024 + (ch % 64) * 8;
        uint8_t* cg = c + 32 * g;
        for (int j = 0; j < 16; ++j) {
          int t = j / 4, i = j % 4;
          cg[8 * t + i] = lo[j] & 15;
          cg[8 * t + 4 + i] = lo[j] >> 4;
        }
        for (int u = 0; u < 2; ++u)
          for (int i = 0; i < 4; ++i)
            for (int s = 0; s < 4; ++s)
              cg[16 * u + 4 * s + i] |= (uint8_t)(((hi[4 * u + i] >> (2 * s)) & 3) << 4);
      }
    }
  return 0;
}

/* ---- contractions ------------------------------------------------------- */
void orc_q4k_q8_contract(const uint8_t* codes, const uint8_t* meta, uint32_t n,
                         uint32_t pk, const int8_t* z, const float* a,
                         const int32_t* sums, uint32_t m, double* out64,
                         float* out32, int32_t* dots, int threads) {
  uint32_t groups = pk / 32, kbs = pk / 256;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic, 16)
#endif
  for (int64_t r = 0; r < (int64_t)n; ++r) {
    for (uint32_t t = 0; t < m; ++t) {
      double acc64 = 0;
      float acc32 = 0;
      for (uint32_t g = 0; g < groups; ++g) {
        const uint8_t* mb = meta + ((size_t)r * kbs + g / 8) * 16;
        unsigned s, mm;
        orc_q4k_scale_min(mb, g % 8, &s, &mm);
        float d = orc_fp16_to_fp32((uint16_t)(mb[0] | (mb[1] << 8)));
        float dmin = orc_fp16_to_fp32((uint16_t)(mb[2] | (mb[3] << 8)));
        const uint8_t* c = codes + (size_t)r * pk + g * 32;
        const int8_t* zz = z + (size_t)t * pk + g * 32;
        int32_t dot = 0;
        for (int j = 0; j < 32; ++j) dot += (int32_t)c[j] * zz[j];
        if (dots) dots[((size_t)t * n + r) * groups + g] = dot;
        float ds = d * (float)s, dm = dmin * (float)mm;
        size_t gi = (size_t)t * groups + g;
        float term = a[gi] * (ds * (float)dot - dm * (float)sums[gi]);
        acc64 += term;
        acc32 += term;
      }
      if (out64) out64[(size_t)t * n + r] = acc64;
      if (out32) out32[(size_t)t * n + r] = acc32;
    }
  }
  (void)threads;
}

void orc_q6k_q8_contract(const uint8_t* q, const int8_t* sc, const uint16_t* d,
                         uint32_t n, uint32_t pk, const int8_t* z, const float* a,
                         const int32_t* sums, uint32_t m, double* out64,
                         float* out32, int32_t* dots, int threads) {
  uint32_t groups = pk / 32, kbs = pk / 256;
  (void)sums;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic, 16)
#endif
  for (int64_t r = 0; r < (int64_t)n; ++r) {
    for (uint32_t t = 0; t < m; ++t) {
      double acc64 = 0;
      float acc32 = 0;
      for (uint32_t g = 0; g < groups; ++g) {
        size_t blk = (size_t)r * kbs + g / 8;
        float dd = orc_fp16_to_fp32(d[blk]);
        const int8_t* s = sc + (size_t)r * (pk / 16) + 2 * g;
        const uint8_t* c = q + (size_t)r * pk + g * 32;
        const int8_t* zz = z + (size_t)t * pk + g * 32;
        int32_t d0 = 0, d1 = 0;
        for (int j = 0; j < 16; ++j) d0 += ((int32_t)c[j] - 32) * zz[j];
        for (int j = 16; j < 32; ++j) d1 += ((int32_t)c[j] - 32) * zz[j];
        int32_t I = s[0] * d0 + s[1] * d1;
        if (dots) dots[((size_t)t * n + r) * groups + g] = I;
        size_t gi = (size_t)t * groups + g;
        float term = a[gi] * (dd * (float)I);
        acc64 += term;
        acc32 += term;
      }
      if (out64) out64[(size_t)t * n + r] = acc64;
      if (out32) out32[(size_t)t * n + r] = acc32;
    }
  }
  (void)threads;
}

/* ---- BF16-activation decode reference ----------------------------------- */
float orc_q4k_bf16_weight(const uint8_t* mb, unsigned code, unsigned g) {
  unsigned s, m;
  orc_q4k_scale_min(mb, g, &s, &m);
  float d = orc_fp16_to_fp32((uint16_t)(mb[0] | (mb[1] << 8))) * (float)s;
  float mm = orc_fp16_to_fp32((uint16_t)(mb[2] | (mb[3] << 8))) * (float)m;
  float v = d * (float)code - mm;
  return orc_bf16_to_fp32(orc_fp32_to_bf16_rne(v));
}

void orc_q4k_bf16_gemv(const uint8_t* codes, const uint8_t* meta, uint32_t n,
                       uint32_t pk, uint32_t k, const uint16_t* x, double* out64,
                       int threads) {
  uint32_t kbs = pk / 256;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic, 16)
#endif
  for (int64_t r = 0; r < (int64_t)n; ++r) {
    double acc = 0;
    for (uint32_t c = 0; c < k; ++c) {
      const uint8_t* mb = meta + ((size_t)r * kbs + c / 256) * 16;
      float w = orc_q4k_bf16_weight(mb, codes[(size_t)r * pk + c], (c % 256) / 32);
      acc += (double)w * (double)orc_bf16_to_fp32(x[c]);
    }
    out64[r] = acc;
  }
  (void)threads;
}

/* ---- decode_mmv dense layouts: Q4G64, Q8G32, BF16 dense tile ------------- */
static int dense_q4(uint16_t layout) { return layout == 0x0201 || layout == 0x020B; }
static int dense_q8(uint16_t layout) { return layout == 0x0202 || layout == 0x020C; }

/* src/format/pack.cpp:143-215: tile_row = ((row/8)*tiles_k + kb)*8 + row%8;
 * Q4: 128 B per tile row, byte c/2 = nibble(code c) | nibble(code c+1) << 4;
 * Q8: 256 B per tile row, one two's-complement byte per code; FP16 scale bits
 * per group (Q4: 4, Q8: 8 per tile row). Padded rows / K are zero. */
int orc_pack_dense_layout(uint16_t layout, const int8_t* codes, const uint16_t* scales,
                          uint32_t n, uint32_t k, uint8_t* co, uint8_t* so) {
  if (!dense_q4(layout) && !dense_q8(layout)) return 1;
  const uint32_t group = dense_q4(layout) ? 64 : 32;
  if (k % group) return 1;
  const uint32_t pn = pad8(n), pk = (k + 255) / 256 * 256, tiles_k = pk / 256;
  const uint32_t row_bytes = dense_q4(layout) ? 128 : 256, gpt = 256 / group;
  memset(co, 0, (size_t)pn * tiles_k * row_bytes);
  memset(so, 0, (size_t)pn * tiles_k * gpt * 2);
  for (uint32_t row = 0; row < n; ++row)
    for (uint32_t kb = 0; kb < tiles_k; ++kb) {
      const size_t tr = ((size_t)(row / 8) * tiles_k + kb) * 8 + row % 8;
      for (uint32_t g = 0; g < gpt; ++g) {
        const uint32_t c0 = kb * 256 + g * group;
        if (c0 < k) {
          const uint16_t b = scales[(size_t)row * (k / group) + c0 / group];
          so[(tr * gpt + g) * 2] = (uint8_t)(b & 0xff);
          so[(tr * gpt + g) * 2 + 1] = (uint8_t)(b >> 8);
        }
      }
      for (uint32_t c = 0; c < 256; ++c) {
        const uint32_t col = kb * 256 + c;
        const uint8_t v = col < k ? (uint8_t)codes[(size_t)row * k + col] : 0;
        if (dense_q4(layout))
          co[tr * 128 + c / 2] |= (uint8_t)((v & 0x0f) << (4 * (c & 1)));
        else
          co[tr * 256 + c] = v;
      }
    }
  return 0;
}

/* src/format/pack.cpp:247-290: row-major BF16 [n][k] (n%8 == 0, k%256 == 0)
 * to 512 B tile rows. */
int orc_pack_bf16_tile(const uint16_t* w, uint32_t n, uint32_t k, uint8_t* co) {
  if (n % 8 || k % 256) return 1;
  const uint32_t tiles_k = k / 256;
  for (uint32_t row = 0; row < n; ++row)
    for (uint32_t kb = 0; kb < tiles_k; ++kb) {
      const size_t tr = ((size_t)(row / 8) * tiles_k + kb) * 8 + row % 8;
      memcpy(co + tr * 512, w + (size_t)row * k + kb * 256, 512);
    }
  return 0;
}

/* cuda/decode_mmv.cu:92-180 (decode8): the BF16 operand of every padded
 * element, out[pn][pk]: Q4 sign-extended nibble or Q8 int8 times the group's
 * FP16 scale (0 when the scale is 0), rounded to BF16; BF16 tiles as stored. */
void orc_dense_operands(uint16_t layout, const uint8_t* co, const uint8_t* so, uint32_t pn,
                        uint32_t pk, uint16_t* out) {
  const uint32_t tiles_k = pk / 256;
  for (uint32_t row = 0; row < pn; ++row)
    for (uint32_t col = 0; col < pk; ++col) {
      const size_t tr = ((size_t)(row / 8) * tiles_k + col / 256) * 8 + row % 8;
      const uint32_t c = col % 256;
      uint16_t w;
      if (dense_q4(layout) || dense_q8(layout)) {
        int code;
        uint16_t sb;
        if (dense_q4(layout)) {
          const uint8_t b = co[tr * 128 + c / 2];
          const int nib = (c & 1) ? (b >> 4) : (b & 15);
          code = nib >= 8 ? nib - 16 : nib;
          sb = (uint16_t)(so[(tr * 4 + c / 64) * 2] | (so[(tr * 4 + c / 64) * 2 + 1] << 8));
        } else {
          code = (int8_t)co[tr * 256 + c];
          sb = (uint16_t)(so[(tr * 8 + c / 32) * 2] | (so[(tr * 8 + c / 32) * 2 + 1] << 8));
        }
        const float scale = orc_fp16_to_fp32(sb);
        const float v = scale != 0.0f ? (float)code * scale : 0.0f;
        w = orc_fp32_to_bf16_rne(v);
      } else {
        w = (uint16_t)(co[tr * 512 + 2 * c] | (co[tr * 512 + 2 * c + 1] << 8));
      }
      out[(size_t)row * pk + col] = w;
    }
}

/* ---- FP8 (OCP E4M3FN) path: cuda/fp8.cu -------------------------------- */
/* E4M3FN value of a code: 1.mmm * 2^(e-7), subnormal m * 2^-9, 0x7F/0xFF NaN. */
float orc_e4m3_to_fp32(uint8_t c) {
  const unsigned mag = c & 0x7Fu, e = mag >> 3, m = mag & 7u;
  float v;
  if (mag == 0x7Fu) v = NAN;
  else if (e == 0) v = ldexpf((float)m, -9);
  else v = ldexpf(1.0f + (float)m / 8.0f, (int)e - 7);
  return (c & 0x80u) ? -v : v;
}

/* Round to nearest even E4M3FN, finite values saturating at +-448, NaN to
 * 0x7F (the conversion cutlass::float_e4m3_t performs in cuda/fp8.cu:79). */
uint8_t orc_fp32_to_e4m3(float x) {
  if (x != x) return 0x7F;
  const uint8_t s = signbit(x) ? 0x80 : 0x00;
  const float a = fabsf(x);
  if (a >= 448.0f) return s | 0x7E;
  if (a < 0.015625f) {  /* below the smallest normal 2^-6: multiples of 2^-9 */
    const float q = rintf(a * 512.0f);  /* exact scaling; rintf rounds half to even */
    return s | (uint8_t)q;              /* q == 8 is the smallest normal, code 0x08 */
  }
  int e;
  const float f = frexpf(a, &e);        /* a = f * 2^e, f in [0.5, 1) */
  const float q = rintf((f * 2.0f - 1.0f) * 8.0f);  /* 3-bit mantissa, half to even */
  int ee = e - 1, mm = (int)q;
  if (mm == 8) { mm = 0; ++ee; }
  if (ee > 8 || (ee == 8 && mm == 7)) return s | 0x7E;
  return s | (uint8_t)(((ee + 7) << 3) | mm);
}

/* pack_fp8 (cuda/fp8.cu:64-81): BF16 [m][k] -> E4M3 codes [pm][pk] and FP32
 * scales [pk/128][pm], pm, pk padded to 128. Scale per (row, 128-column block):
 * absmax/448 floored at 2^-126, 1 for an all-zero block, NaN when the block holds
 * a nonfinite value; padding is zero. */
void orc_pack_fp8(const uint16_t* x, uint32_t m, uint32_t k, uint8_t* codes, float* scales) {
  const uint32_t pm = (m + 127) / 128 * 128, pk = (k + 127) / 128 * 128;
  for (uint32_t r = 0; r < pm; ++r)
    for (uint32_t b = 0; b < pk / 128; ++b) {
      float peak = 0.0f;
      int finite = 1;
      for (uint32_t c = b * 128; c < b * 128 + 128; ++c) {
        const float v = (r < m && c < k) ? orc_bf16_to_fp32(x[(size_t)r * k + c]) : 0.0f;
        if (!isfinite(v)) finite = 0;
        else if (fabsf(v) > peak) peak = fabsf(v);
      }
      const float scale = !finite ? NAN : (peak == 0.0f ? 1.0f : fmaxf(peak / 448.0f, 0x1p-126f));
      scales[(size_t)b * pm + r] = scale;
      for (uint32_t c = b * 128; c < b * 128 + 128; ++c) {
        const float v = (r < m && c < k) ? orc_bf16_to_fp32(x[(size_t)r * k + c]) : 0.0f;
        codes[(size_t)r * pk + c] = orc_fp32_to_e4m3(v / scale);
      }
    }
}

/* y[r] = sum_c value(code[r][c]) * wscale[(c/128)*(n/128) + r/128] * x[c] in
 * double (cuda/fp8.cu:82-112); l1 = sum of the absolute products. */
void orc_fp8_gemv(const uint8_t* codes, const float* wscales, uint32_t n, uint32_t k,
                  const uint16_t* x, double* out, double* l1) {
  for (uint32_t r = 0; r < n; ++r) {
    double acc = 0, s1 = 0;
    for (uint32_t c = 0; c < k; ++c) {
      const double z = (double)orc_e4m3_to_fp32(codes[(size_t)r * k + c]) *
                       (double)wscales[(size_t)(c / 128) * (n / 128) + r / 128] *
                       (double)orc_bf16_to_fp32(x[c]);
      acc += z;
      s1 += fabs(z);
    }
    out[r] = acc;
    if (l1) l1[r] = s1;
  }
}

/* y[t][r] = sum_c (value(xc[t][c]) xs[c/128][t]) (value(wc[r][c]) ws[(c/128)*(n/128) + r/128])
 * in double (the contraction fp8_gemm performs, cuda/fp8.cu:137-160). */
void orc_fp8_gemm(const uint8_t* wc, const float* ws, uint32_t n, uint32_t k, const uint8_t* xc,
                  const float* xs, uint32_t m, double* out, double* l1) {
  for (uint32_t t = 0; t < m; ++t)
    for (uint32_t r = 0; r < n; ++r) {
      double acc = 0, s1 = 0;
      for (uint32_t c = 0; c < k; ++c) {
        const double a = (double)orc_e4m3_to_fp32(xc[(size_t)t * k + c]) * (double)xs[(size_t)(c / 128) * m + t];
        const double b = (double)orc_e4m3_to_fp32(wc[(size_t)r * k + c]) *
                         (double)ws[(size_t)(c / 128) * (n / 128) + r / 128];
        acc += a * b;
        s1 += fabs(a * b);
      }
      out[(size_t)t * n + r] = acc;
      if (l1) l1[(size_t)t * n + r] = s1;
    }
}

/* ---- NVFP4 (src/format/nvfp4.cpp, cuda/nvfp4_device.cuh) ------------------ */
float orc_e2m1_value(uint8_t c) {
  static const float v[8] = {0.f, .5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};
  return (c & 8u) ? -v[c & 7u] : v[c & 7u];
}

float orc_ue4m3_value(uint8_t c) {
  return (c >> 3) == 0 ? ldexpf((float)(c & 7u), -9) : ldexpf(1.f + (float)(c & 7u) / 8.f, (int)(c >> 3) - 7);
}

/* Nearest code by exhaustive search, ties to the even code
 * (tests/nvfp4_test.cpp:47-56): scale codes 0..126, element codes 0..7 with
 * the sign of a nonzero v in bit 3. */
uint8_t orc_nvfp4_nearest(float v, int scale) {
  float error = INFINITY;
  unsigned best = 0;
  for (unsigned c = 0; c < (scale ? 127u : 8u); ++c) {
    const float value = scale ? orc_ue4m3_value((uint8_t)c) : orc_e2m1_value((uint8_t)c);
    const float e = fabsf(fabsf(v) - value);
    if (e < error || (e == error && !(c & 1u))) { error = e; best = c; }
  }
  return (uint8_t)(best | (!scale && signbit(v) && v != 0 ? 8u : 0u));
}

/* src/format/nvfp4.hpp:14-17 */
uint64_t orc_nvfp4_sf_index(uint64_t row, uint64_t block, uint64_t pk) {
  return (row / 128) * 128 * (pk / 16) + (block / 4) * 512 + (row % 32) * 16 + ((row % 128) / 32) * 4 +
         block % 4;
}

/* One 16-element block (cuda/nvfp4_device.cuh:20-48): returns the scale code,
 * writes the 8 code bytes (element 2j in the low nibble of byte j). */
static uint8_t nvfp4_block(const float v[16], uint8_t out[8]) {
  float peak = 0.f;
  int finite = 1;
  for (int i = 0; i < 16; ++i) {
    if (!isfinite(v[i])) finite = 0;
    else if (fabsf(v[i]) > peak) peak = fabsf(v[i]);
  }
  uint8_t s = finite ? orc_nvfp4_nearest(peak / 6.f, 1) : 127;
  if (finite && peak != 0.f && s == 0) s = 1;
  const float scale = orc_ue4m3_value(s);
  for (int i = 0; i < 8; ++i) {
    const float a = v[2 * i], b = v[2 * i + 1];
    const unsigned lo = (a == 0.f || !finite) ? 0u : orc_nvfp4_nearest(a / scale, 0);
    const unsigned hi = (b == 0.f || !finite) ? 0u : orc_nvfp4_nearest(b / scale, 0);
    out[i] = (uint8_t)(lo | (hi << 4));
  }
  return s;
}

/* launch_pack_nvfp4 (cuda/nvfp4.cu:72-82): BF16 [m][k] -> codes [m][pk/2],
 * scales of pad128(m) rows (padding rows 0; padding rows' codes absent). */
void orc_pack_nvfp4(const uint16_t* x, uint32_t m, uint32_t k, uint8_t* codes, uint8_t* scales) {
  const uint32_t pk = (k + 255) / 256 * 256, pm = (m + 127) / 128 * 128;
  for (uint32_t r = 0; r < pm; ++r)
    for (uint32_t b = 0; b < pk / 16; ++b) {
      float v[16];
      for (uint32_t i = 0; i < 16; ++i) {
        const uint32_t c = b * 16 + i;
        v[i] = (r < m && c < k) ? orc_bf16_to_fp32(x[(size_t)r * k + c]) : 0.f;
      }
      uint8_t out[8];
      scales[orc_nvfp4_sf_index(r, b, pk)] = nvfp4_block(v, out);
      if (r < m) memcpy(codes + ((size_t)r * pk + b * 16) / 2, out, 8);
    }
}

/* quantize_nvfp4 (src/compiler/quantization/nvfp4.cpp:12-61): the weight
 * payload of BF16 [n][k]: codes [pn][pk/2], scales 256-byte header (FP32
 * factor = 2^ceil(log2(peak / 2688)), at least FLT_MIN) + swizzled scales of
 * pad128(pn) rows. pn = n rounded up to 8. Returns 0, or -1 for a nonfinite
 * weight. */
int orc_quantize_nvfp4(const uint16_t* w, uint32_t n, uint32_t k, uint8_t* codes, uint8_t* scales) {
  const uint32_t pk = (k + 255) / 256 * 256, pn = (n + 7) / 8 * 8;
  float peak = 0.f;
  for (size_t i = 0; i < (size_t)n * k; ++i) {
    const float v = orc_bf16_to_fp32(w[i]);
    if (!isfinite(v)) return -1;
    if (fabsf(v) > peak) peak = fabsf(v);
  }
  float factor = peak == 0.f ? 1.f : (float)exp2(ceil(log2((double)peak / 2688.)));
  if (factor < 0x1p-126f) factor = 0x1p-126f;
  memset(codes, 0, (size_t)pn * pk / 2);
  memset(scales, 0, 256 + (size_t)(pn + 127) / 128 * 128 * (pk / 16));
  memcpy(scales, &factor, 4);
  for (uint32_t r = 0; r < n; ++r)
    for (uint32_t b = 0; b < (k + 15) / 16; ++b) {
      float v[16] = {0};
      for (uint32_t i = 0; i < 16 && b * 16 + i < k; ++i)
        v[i] = orc_bf16_to_fp32(w[(size_t)r * k + b * 16 + i]) / factor;
      uint8_t out[8];
      scales[256 + orc_nvfp4_sf_index(r, b, pk)] = nvfp4_block(v, out);
      memcpy(codes + ((size_t)r * pk + b * 16) / 2, out, 8);
    }
  return 0;
}

static inline unsigned nib(const uint8_t* codes, uint64_t i) { return (codes[i / 2] >> (4 * (i & 1))) & 15u; }

/* decode_mmv NVFP4 (cuda/decode_mmv.cu:94-102, 223-239): weight element
 * RN(RN(ue4m3(sf) * factor) * e2m1(code)) in FP32, times BF16 x, summed in
 * double; l1 = sum of |products|. */
void orc_nvfp4_gemv(const uint8_t* codes, const uint8_t* scales, uint32_t n, uint32_t pk,
                    const uint16_t* x, uint32_t k, double* out, double* l1) {
  float factor;
  memcpy(&factor, scales, 4);
  for (uint32_t r = 0; r < n; ++r) {
    double acc = 0, s1 = 0;
    for (uint32_t c = 0; c < k; ++c) {
      const float sc = orc_ue4m3_value(scales[256 + orc_nvfp4_sf_index(r, c / 16, pk)]) * factor;
      const float wv = sc * orc_e2m1_value((uint8_t)nib(codes, (uint64_t)r * pk + c));
      const double z = (double)wv * (double)orc_bf16_to_fp32(x[c]);
      acc += z;
      s1 += fabs(z);
    }
    out[r] = acc;
    if (l1) l1[r] = s1;
  }
}

/* W4A4 (cuda/nvfp4.cu:83-116): y[t][r] = factor * sum_c (sa*a)(sw*w) in double. */
void orc_nvfp4_gemm(const uint8_t* wc, const uint8_t* ws, uint32_t n, uint32_t pk, const uint8_t* xc,
                    const uint8_t* xs, uint32_t m, double* out, double* l1) {
  float factor;
  memcpy(&factor, ws, 4);
  for (uint32_t t = 0; t < m; ++t)
    for (uint32_t r = 0; r < n; ++r) {
      double acc = 0, s1 = 0;
      for (uint32_t c = 0; c < pk; ++c) {
        const double a = (double)orc_ue4m3_value(xs[orc_nvfp4_sf_index(t, c / 16, pk)]) *
                         orc_e2m1_value((uint8_t)nib(xc, (uint64_t)t * pk + c));
        const double b = (double)orc_ue4m3_value(ws[256 + orc_nvfp4_sf_index(r, c / 16, pk)]) *
                         orc_e2m1_value((uint8_t)nib(wc, (uint64_t)r * pk + c));
        acc += a * b;
        s1 += fabs(a * b);
      }
      out[(size_t)t * n + r] = (double)factor * acc;
      if (l1) l1[(size_t)t * n + r] = (double)factor * s1;
    }
}
