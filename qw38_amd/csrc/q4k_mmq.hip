// Prefill MMQ (M > 8) on gfx950 matrix cores (v_mfma_f32_16x16x32_f16).
//
// Exactness. For Q4_K row r and K32 group g the reference contraction
// (cuda/q4k_q8.cu:140,245) is a_tg (d_r s_rg dot_rtg - dmin_r m_rg sum_tg)
// with an exact int32 dot. The A tile holds the integers s_rg * w_rk (<= 945)
// and the B tile the int8 codes z_tk, both exact in FP16; one MFMA covers
// exactly one K32 group and every partial sum of its products is an integer
// below 2^24, so its FP32 result P = s_rg * dot_rtg is exact whatever the
// accumulation order inside the matrix core. Per super-block kb:
//   X_rt  = sum_{g in kb} a_tg P_rtg                 (one VALU FMA per output)
//   Y_rt  = sum_{g in kb} m_rg (a_tg sum_tg)          (two 16x16x16 MFMAs with
//           the FP32 products a*sum, scaled per token by a power of two,
//           split into FP16 hi + lo; K zero-padded from 8 to 16)
//   acc  += d_r X_rt - dmin_r Y_rt
// which is the reference's per-group expression reassociated. Every M-tiling
// runs the same per-(row, token) operation sequence, so all tile shapes give
// bitwise-identical outputs (the reference's J32 == J128 property,
// tests/q4k_q8_test.cpp:118-120).
//
// Q6_K (layout 0x0241): the A tile holds v = sc_sub (q - 32) (|v| <= 4096),
// split exactly into FP16 hi = RN(v) and lo = v - hi; two MFMAs per group give
// P_hi + P_lo = the exact integer I_rtg, and acc += d_r sum_g a_tg I_rtg.
//
// Tiles are converted to FP16 while staging: bytes become FP16 1024 + b by a
// v_perm with 0x64 high bytes, then one packed FP16 FMA/add recovers the exact
// integer value (scaled by s for Q4_K weights). Rows of the LDS tiles are
// 64 halfs + 8 pad; all stores are 16 B.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <type_traits>

#include "common.hpp"

namespace qw38hip {
uint64_t mmq_dma_scratch_bytes(uint32_t m, uint32_t pk);
hipError_t launch_mmq_dma(const WeightView& w, const Q8View& x, float* out, const float* residual,
                          hipStream_t s, uint32_t rows, uint32_t tail_end, void* scratch, const WeightView* up = nullptr,
                          int8_t* qc = nullptr, float* qa = nullptr, int32_t* qs = nullptr,
                          int* failure = nullptr, int tail_nj = 2);
namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

// Halfs per LDS tile row: 2 groups x 32 + 16 pad. A 40-dword stride (an odd
// multiple of 8) keeps the b128 fragment reads free of bank conflicts on the
// 64-bank LDS; a 36-dword stride (+8 pad) halves the read rate.
constexpr int kStride = 80;
// Half offset of the second K32 group in an A-tile row: 40 (20 dwords, an odd
// multiple of 4) instead of 32, so a store phase of lanes holding (row, group)
// pairs of four rows hits eight distinct 4-bank groups (with 32 the groups of
// rows r and r + 2 coincide); the fragment reads stay conflict-free.
constexpr int kG1 = 40;

__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }

// bytes b0, b1 of v -> half2(1024 + b0, 1024 + b1); bytes b2, b3 likewise
__device__ __forceinline__ h2 lo_pair(uint32_t v) { return as_h2(perm(0x64646464u, v, 0x04010400u)); }
__device__ __forceinline__ h2 hi_pair(uint32_t v) { return as_h2(perm(0x64646464u, v, 0x04030402u)); }

// Logical-order code vectors (vector j = codes 4j..4j+3) of one Q4_K group.
template <uint16_t Layout, int NW>
__device__ __forceinline__ void q4_vectors(const uint32_t w[NW], uint32_t v[2 * NW]) {
#pragma unroll
  for (int t = 0; t < NW; ++t) {
    const uint32_t lo = w[t] & 0x0f0f0f0fu;
    const uint32_t hi = (w[t] >> 4) & 0x0f0f0f0fu;
    if constexpr (Layout == QW38_LAYOUT_Q4K_CANDIDATE_V2) {
      v[2 * t] = perm(hi, lo, 0x05010400u);
      v[2 * t + 1] = perm(hi, lo, 0x07030602u);
    } else {
      v[2 * t] = lo;
      v[2 * t + 1] = hi;
    }
  }
}

template <int WR, int WT, int NI, int NJ>
struct Cfg {
  static constexpr int BR = WR * NI * 16;  // weight rows per block
  static constexpr int BT = WT * NJ * 16;  // tokens per block
};

// Block-to-tile order: hardware places block b on XCD b % 8; each XCD gets a
// contiguous range of tiles so the token blocks of one weight-row block share
// that XCD's L2 (a bijection when the tile count is a multiple of 8).
__device__ __forceinline__ uint32_t xcd_tile(uint32_t b, uint32_t nblk) {
  return (nblk % 8 == 0) ? (b % 8) * (nblk / 8) + b / 8 : b;
}

// Global operands of one K step (two K32 groups), loaded into registers one
// or two steps ahead of their LDS store so the loads overlap the matrix-core
// work. Loads of rows past the padded weight and of tokens past m read a clamped
// (valid) row or token instead: every output element depends only on its own
// row and token, and those rows and tokens are never stored.
template <int ZW, int GPT, int AW>
struct Fetch {
  uint32_t w[AW];    // A: this thread's share (16 B or 8 B) of the codes of (row, group)
  uint32_t x[4];     // A: Q4_K metadata row | Q6_K: qh words 0-1, scale pair, d
  uint32_t z[ZW];    // B: this thread's share of a (token, group) code row
  float a[GPT];      // super-block token data (first step of a super-block
  int32_t su[GPT];   // only): this thread's GPT groups of token kt
};

// Fused gate + up (Glu): the up projection's weight and the down
// projection's Q8 operand, written by the SwiGLU -> Q8 epilogue.
struct GluOut {
  const uint8_t* codes2;  // up weight codes / metadata (same geometry as gate)
  const uint8_t* meta2;
  int8_t* qc;             // [m][n] codes
  float* qa;              // [m][n / 32] scales
  int32_t* qs;            // [m][n / 32] code sums
  int* failure;           // sticky nonfinite-producer flag
};

// Glu: a tile's first BR / 2 rows are gate rows and its last BR / 2 the up rows
// of the same BR / 2 features (row_begin and the tile height in features); the
// gate waves hand their outputs to the up waves through LDS, which apply
// SwiGLU -> BF16 -> Q8 per K32 feature group in the up waves' registers. The
// per-(row, token) arithmetic is that of the unfused kernel, so the fused
// codes equal swiglu_q8 of the two separate projections bit for bit.
template <uint16_t Layout, bool Vec, int WR, int WT, int NI, int NJ, bool Glu = false>
__global__ __launch_bounds__(WR * WT * 64, (WR * WT * NI * NJ >= 64) ? 1 : 2) void mmq_kernel(
    const uint8_t* __restrict__ codes, const uint8_t* __restrict__ meta, uint32_t n,
    uint32_t pn, uint32_t kbs, const int8_t* __restrict__ xc, const float* __restrict__ xa,
    const int32_t* __restrict__ xs, uint32_t m, uint32_t pk, float* __restrict__ out,
    const float* __restrict__ residual, uint32_t row_begin, uint32_t row_blocks, uint32_t tok_blocks,
    GluOut glu, uint32_t seg_kb, uint32_t split, float* __restrict__ part) {
  constexpr bool kQ6 = Layout == QW38_LAYOUT_Q6K_WAVE64;
  using C = Cfg<WR, WT, NI, NJ>;
  constexpr int BR = C::BR, BT = C::BT, NT = WR * WT * 64;
  constexpr int HR = Glu ? BR / 2 : BR;  // features (output rows) per tile
  static_assert(!Glu || (!kQ6 && WR % 2 == 0 && NI % 2 == 0), "Glu tiles: Q4_K, gate / up wave halves");
  // A staging: APT threads per (row, group), AW code words each. Tiles with
  // fewer (row, group) items than threads (80 rows) leave the last threads
  // out of A staging: they load a duplicate item and store nothing.
  constexpr int APT0 = NT / (2 * BR);
  constexpr int APT = (APT0 == 1 || (APT0 == 2 && NT == 4 * BR && !kQ6)) ? APT0 : 1, AW = 4 / APT;
  static_assert((APT * 2 * BR == NT || (APT == 1 && 2 * BR < NT)) && (APT == 1 || (APT == 2 && !kQ6)),
                "A staging share");
  constexpr int BB = BT * 64 / NT;  // B bytes staged per thread per step
  static_assert(BB == 4 || BB == 8 || BB == 16 || BB == 32, "B staging share");
  constexpr int ZW = BB / 4, PARTS = 32 / BB;
  // super-block token data: TPT threads per token (at most 8, one group each;
  // threads past BT * TPT have no token-data role)
  constexpr int TPT = NT / BT > 8 ? 8 : NT / BT, GPT = 8 / TPT;
  static_assert(TPT >= 1 && GPT * TPT == 8, "token-data share");
  constexpr int kPlanes = kQ6 ? 2 : 1;  // Q6_K stages hi and lo FP16 planes
  constexpr int kMinR = kQ6 ? 1 : BR * 8, kMinT = kQ6 ? 1 : BT * 8;
  __shared__ __align__(16) _Float16 As[2][kPlanes][BR * kStride];
  __shared__ __align__(16) _Float16 Bs[2][BT * kStride];
  __shared__ __align__(16) _Float16 Mq[2][kMinR];  // m of groups 0..7 per row
  __shared__ __align__(16) _Float16 Uh[2][kMinT];  // scaled a*sum hi per token
  __shared__ __align__(16) _Float16 Ul[2][kMinT];  // scaled a*sum lo per token
  __shared__ float Ti[BT];                         // inverse of the per-token scale
  __shared__ float Aa[2][BT * 8];
  __shared__ float2 Dd[2][BR];                     // (d, -dmin) | (d, 0)

  // Q6_K accumulates K in fixed segments of seg_kb super-blocks (a function
  // of K alone): each segment's sum starts from zero and the segment sums are
  // added in ascending order. With split > 1 each block runs one or two
  // consecutive segments (split = segments or segments / 2 runs) of one tile
  // and, after its loop, writes each segment's sum to part[segment];
  // mmq_seg_reduce_kernel adds them in the same order, so split and unsplit
  // launches give the same bits. (Q4_K has neither: its accumulation order and
  // registers are unchanged.)
  const bool splitk = kQ6 && split > 1;
  const uint32_t tiles_n = row_blocks * tok_blocks;
  const uint32_t run = splitk ? blockIdx.x / tiles_n : 0u;
  const uint32_t tile = xcd_tile(splitk ? blockIdx.x % tiles_n : blockIdx.x, tiles_n);
  const uint32_t spr = splitk ? ((kbs + seg_kb - 1) / seg_kb) / split : 0u;  // segments per run
  const uint32_t kb_lo = splitk ? run * spr * seg_kb : 0u;
  const uint32_t kb_hi = splitk ? min(kbs, kb_lo + spr * seg_kb) : kbs;
  float* part_first = nullptr;  // split runs of two segments: the first one's sum
  if (splitk) {
    part_first = part + size_t(kb_lo / seg_kb) * m * n;
    out = part + size_t((kb_hi - 1) / seg_kb) * m * n;
    residual = nullptr;
  }
  const uint32_t row0 = row_begin + (tile / tok_blocks) * HR, tok0 = (tile % tok_blocks) * BT;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t wr = wave / WT, wt = wave % WT;
  const uint32_t lr = lane & 15u, lk = lane >> 4;
  const uint32_t groups = pk / 32, strips = pn / 8;
  const uint64_t tiles = uint64_t(pn) * kbs;
  const uint32_t steps = kbs * 4;

  // A staging role: row ar, group-in-step asel (clamped row for the loads)
  // Layout 0x0240: consecutive lanes take consecutive rows of one group, so
  // their 16-byte global loads read one contiguous run of a group plane
  // (3% faster at config 2, M=512). 0x020D and Q6_K: lane pairs take the two
  // groups of one row, whose bytes are adjacent in the tile row.
  constexpr bool kRowMajorA = Layout == QW38_LAYOUT_Q4K_WAVE64;
  const uint32_t ah = tid % APT;
  const uint32_t aslot = (tid / APT) % (2 * BR);
  const bool a_on = tid / APT < uint32_t(2 * BR);
  const uint32_t ar = kRowMajorA ? aslot % BR : aslot >> 1;
  const uint32_t asel = kRowMajorA ? aslot / BR : aslot & 1u;
  const uint32_t arow = min(row0 + (Glu ? ar % HR : ar), pn - 1);
  if constexpr (Glu) {  // the tile's up half reads the up weight
    // A wave's staging rows lie in one aligned run of 16..64 rows and the
    // gate / up boundary HR is a multiple of 64, so the choice is the same in
    // every lane: taken from the first lane, the pointers stay scalar.
    if (__builtin_amdgcn_readfirstlane(ar >= uint32_t(HR) ? 1 : 0)) {
      codes = glu.codes2;
      meta = glu.meta2;
    }
  }
  // B staging role: token bt, group-in-step bsel, byte part bpart of BB bytes
  const uint32_t bpart = tid % PARTS, bsel = (tid / PARTS) & 1u, bt = tid / (2 * PARTS);
  const uint32_t btok = min(tok0 + bt, m - 1);
  const uint32_t kt = tid / TPT, kg = (tid % TPT) * GPT;  // token kt, groups kg..kg+GPT-1
  const bool k_on = kt < uint32_t(BT);
  const uint32_t ktok = min(tok0 + kt, m - 1);
  const bool xc_vec = (reinterpret_cast<uintptr_t>(xc) % BB) == 0;

  // Per-thread address parts (the per-step parts are wave-uniform).
  const int8_t* const zrow = xc + (size_t(btok) * groups + bsel) * 32 + bpart * BB;
  const size_t krow = size_t(ktok) * groups + kg;
  uint64_t a_base = 0, m_base = 0;
  uint32_t a_r1 = 0, a_r2 = 0, m_r1 = 0;
  if constexpr (Layout == QW38_LAYOUT_Q4K_WAVE64) {
    a_r1 = (arow / 8) * 1024 + asel * 128;  // scaled by the chunk's super-block count
    a_r2 = (arow % 8) * 16;
    m_r1 = (arow / 8) * 128;
  } else {  // 0x020D and Q6_K: tile row ((row/8)*kbs + kb)*8 + row%8
    const uint64_t tr0 = uint64_t(arow / 8) * kbs * 8 + arow % 8;
    a_base = kQ6 ? tr0 : tr0 * 128 + asel * 16;
    m_base = tr0 * 16;
  }

  // ---- Q4_K per-token scale: ts_t = 2^e with max_g |a_tg| * 2^12 * ts_t in
  // [2^13, 2^14). |sum_tg| <= 32 * 127 < 2^12, so every min-term operand
  // u = a * sum * ts fits FP16 with 22-bit hi + lo precision, and a * ts stays
  // small. ts is fixed over all of K, so the accumulator is kept scaled by ts
  // (acc' = ts * acc, exact: a power of two) and unscaled once at the store. ----
  float ts = 1.f;
  if constexpr (!kQ6) {
    float mx = 0.f;
    const float* ap = xa + size_t(ktok) * groups;
#pragma unroll 4
    for (uint32_t g = tid % TPT; g < kbs * 8; g += TPT) mx = fmaxf(mx, fabsf(ap[g]));
#pragma unroll
    for (int w = 1; w < TPT; w *= 2) mx = fmaxf(mx, __shfl_xor(mx, w));  // the token's lanes
    const int ex = int(__float_as_uint(mx) >> 23);  // 0 for zero/subnormal, 255 for NaN/inf
    const int se = min(max(255 - ex, 1), 253);
    ts = __uint_as_float(uint32_t(se) << 23);
    if (tid % TPT == 0 && k_on) Ti[kt] = __uint_as_float(uint32_t(254 - se) << 23);
  }

  // Step s = 4 kb + q stages K groups 2q, 2q+1 of super-block kb. q is a
  // compile-time constant everywhere below, so a super-block is one branch-free
  // block the scheduler can interleave (staging VALU beside the MFMAs).
  auto fetch = [&](auto qc, uint32_t kb_in, Fetch<ZW, GPT, AW>& F) __attribute__((always_inline)) {
    constexpr uint32_t q = decltype(qc)::value;
    const uint32_t kb = min(kb_in, kb_hi - 1);  // past the end: a harmless re-read
    if constexpr (Layout == QW38_LAYOUT_Q4K_WAVE64) {
      const uint32_t c = kb / 8, kq = kb % 8;
      const uint32_t nk = min(kbs - 8 * c, 8u);
      const uint8_t* cp = codes + uint64_t(strips) * 8192 * c +
                          (nk * a_r1 + a_r2 + (2 * q * nk + kq) * 128) + ah * 4 * AW;
      const uint8_t* mp = meta + uint64_t(strips) * 1024 * c + (nk * m_r1 + a_r2 + kq * 128);
      if constexpr (AW == 4) {
        const uint4 cw = *reinterpret_cast<const uint4*>(cp);
        F.w[0] = cw.x; F.w[1] = cw.y; F.w[2] = cw.z; F.w[3] = cw.w;
      } else {
        const uint2 cw = *reinterpret_cast<const uint2*>(cp);
        F.w[0] = cw.x; F.w[1] = cw.y;
      }
      const uint4 mw = *reinterpret_cast<const uint4*>(mp);
      F.x[0] = mw.x; F.x[1] = mw.y; F.x[2] = mw.z; F.x[3] = mw.w;
    } else if constexpr (Layout == QW38_LAYOUT_Q4K_CANDIDATE_V2) {
      const uint8_t* cp = codes + a_base + kb * 1024 + q * 32;
      const uint8_t* mp = meta + m_base + kb * 128;
      if constexpr (Vec) {  // 16-byte aligned spans: one wide load each
        if constexpr (AW == 4) {
          const uint4 cw = reinterpret_cast<const uint4*>(cp)[ah];
          F.w[0] = cw.x; F.w[1] = cw.y; F.w[2] = cw.z; F.w[3] = cw.w;
        } else {
          const uint2 cw = reinterpret_cast<const uint2*>(cp)[ah];
          F.w[0] = cw.x; F.w[1] = cw.y;
        }
        const uint4 mw = *reinterpret_cast<const uint4*>(mp);
        F.x[0] = mw.x; F.x[1] = mw.y; F.x[2] = mw.z; F.x[3] = mw.w;
      } else {  // 4-byte aligned codes, 2-byte aligned metadata
        const uint32_t* c4 = reinterpret_cast<const uint32_t*>(cp);
        const uint16_t* m2 = reinterpret_cast<const uint16_t*>(mp);
#pragma unroll
        for (int i = 0; i < AW; ++i) F.w[i] = c4[ah * AW + i];
#pragma unroll
        for (int i = 0; i < 4; ++i) F.x[i] = uint32_t(m2[2 * i]) | (uint32_t(m2[2 * i + 1]) << 16);
      }
    } else {
      const uint32_t g = 2 * q + asel;
      const uint64_t tr = a_base + kb * 8;
      const uint8_t* tp = codes + (tr - arow % 8) * kQ6CodeBytes;  // the tile's first byte
      const uint32_t ch = q6_chunk(arow % 8, g);
      const uint4 cw = *reinterpret_cast<const uint4*>(tp + ch * 16);
      const uint2 hw = *reinterpret_cast<const uint2*>(tp + kQ6HiPlane + ch * 8);
      F.w[0] = cw.x; F.w[1] = cw.y; F.w[2] = cw.z; F.w[3] = cw.w;
      F.x[0] = hw.x; F.x[1] = hw.y;
      F.x[2] = *reinterpret_cast<const uint16_t*>(meta + tr * 16 + g * 2);
      F.x[3] = *reinterpret_cast<const uint16_t*>(meta + tiles * 16 + tr * 2);
    }
    const int8_t* zp = zrow + (kb * 8 + 2 * q) * 32;
    if (xc_vec) {
      if constexpr (BB == 4) {
        F.z[0] = *reinterpret_cast<const uint32_t*>(zp);
      } else if constexpr (BB == 8) {
        const uint2 v = *reinterpret_cast<const uint2*>(zp);
        F.z[0] = v.x; F.z[1] = v.y;
      } else {
#pragma unroll
        for (int i = 0; i < BB / 16; ++i) {
          const uint4 v = reinterpret_cast<const uint4*>(zp)[i];
          F.z[4 * i] = v.x; F.z[4 * i + 1] = v.y; F.z[4 * i + 2] = v.z; F.z[4 * i + 3] = v.w;
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < ZW; ++i) F.z[i] = reinterpret_cast<const uint32_t*>(zp)[i];
    }
    if constexpr (q == 0) {
#pragma unroll
      for (int i = 0; i < GPT; ++i) {
        F.a[i] = xa[krow + kb * 8 + i];
        if constexpr (!kQ6) F.su[i] = xs[krow + kb * 8 + i];
      }
    }
  };

  // Stores step (kb, q) into LDS buffer q & 1 and super-block slot kb & 1.
  auto store = [&](auto qc, uint32_t kb, const Fetch<ZW, GPT, AW>& F) __attribute__((always_inline)) {
    constexpr uint32_t q = decltype(qc)::value, buf = q & 1u;
    const uint32_t kp = kb & 1u, g = 2 * q + asel;
    // ---- A: 32 FP16 values of (row ar, group g) ----
    if constexpr (!kQ6) {
      float sf, mf;
      q4_scale_min_lane(F.x[1], F.x[2], F.x[3], g, sf, mf);
      if (ah == 0 && a_on) Mq[kp][ar * 8 + g] = _Float16(mf);
      if (q == 0 && asel == 0 && ah == 0 && a_on)
        Dd[kp][ar] = make_float2(f16_to_f32(F.x[0] & 0xffffu), -f16_to_f32(F.x[0] >> 16));
      uint32_t v[2 * AW];
      q4_vectors<Layout, AW>(F.w, v);
      const _Float16 sh = _Float16(sf), bh = _Float16(-1024.f * sf);
      const h2 s2 = {sh, sh}, b2 = {bh, bh};
      uint32_t o[4 * AW];
#pragma unroll
      for (int j = 0; j < 2 * AW; ++j) {  // (1024 + c) s - 1024 s = c s exactly (c s <= 945)
        o[2 * j] = as_u32(__builtin_elementwise_fma(lo_pair(v[j]), s2, b2));
        o[2 * j + 1] = as_u32(__builtin_elementwise_fma(hi_pair(v[j]), s2, b2));
      }
      uint4* dst = reinterpret_cast<uint4*>(&As[buf][0][ar * kStride + asel * kG1 + ah * 8 * AW]);
      if (a_on) {
#pragma unroll
        for (int i = 0; i < AW; ++i) dst[i] = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
      }
    } else {
      if (q == 0 && asel == 0 && a_on) Dd[kp][ar] = make_float2(f16_to_f32(F.x[3]), 0.f);
      const h2 off = {_Float16(-1056.f), _Float16(-1056.f)};  // 1024 + q -> q - 32
      uint32_t oh[16], ol[16];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t nib = (j & 1) ? (F.w[j >> 1] >> 4) & 0x0f0f0f0fu : F.w[j >> 1] & 0x0f0f0f0fu;
        const uint32_t hh = (F.x[j >> 2] >> (2 * (j & 3))) & 0x03030303u;
        const uint32_t qv = nib | (hh << 4);
        const _Float16 sc = _Float16(float(int8_t(j < 4 ? F.x[2] & 0xffu : F.x[2] >> 8)));
        const h2 s2 = {sc, sc};
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const h2 c = (e ? hi_pair(qv) : lo_pair(qv)) + off;   // q - 32, exact
          const h2 hi = c * s2;                                  // RN(sc (q - 32))
          const h2 lo = __builtin_elementwise_fma(c, s2, -hi);  // exact remainder
          oh[2 * j + e] = as_u32(hi);
          ol[2 * j + e] = as_u32(lo);
        }
      }
      uint4* dh = reinterpret_cast<uint4*>(&As[buf][0][ar * kStride + asel * kG1]);
      uint4* dl = reinterpret_cast<uint4*>(&As[buf][kPlanes - 1][ar * kStride + asel * kG1]);
      if (a_on) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          dh[i] = make_uint4(oh[4 * i], oh[4 * i + 1], oh[4 * i + 2], oh[4 * i + 3]);
          dl[i] = make_uint4(ol[4 * i], ol[4 * i + 1], ol[4 * i + 2], ol[4 * i + 3]);
        }
      }
    }
    // ---- B: this thread's BB codes z of (token bt, group) as FP16 ----
    {
      const h2 off = {_Float16(-1152.f), _Float16(-1152.f)};
      uint32_t o[2 * ZW];
#pragma unroll
      for (int j = 0; j < ZW; ++j) {
        const uint32_t u = F.z[j] ^ 0x80808080u;  // z + 128 as unsigned bytes
        o[2 * j] = as_u32(lo_pair(u) + off);
        o[2 * j + 1] = as_u32(hi_pair(u) + off);
      }
      _Float16* dst = &Bs[buf][bt * kStride + bsel * 32 + bpart * BB];
      if constexpr (BB == 4) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(o[0], o[1]);
      } else if constexpr (BB == 8) {
        *reinterpret_cast<uint4*>(dst) = make_uint4(o[0], o[1], o[2], o[3]);
      } else {
#pragma unroll
        for (int i = 0; i < ZW / 2; ++i)
          reinterpret_cast<uint4*>(dst)[i] = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
      }
    }
    // ---- super-block token data: a * ts per group; for Q4_K the min-term
    // operand u = a * ts * sum split into FP16 hi + lo ----
    if (q == 0 && k_on) {
#pragma unroll
      for (int i = 0; i < GPT; ++i) {
        const float a = F.a[i] * ts;
        Aa[kp][kt * 8 + kg + i] = a;
        if constexpr (!kQ6) {
          const float v = a * float(F.su[i]);
          const _Float16 h = _Float16(v);
          Uh[kp][kt * 8 + kg + i] = h;
          Ul[kp][kt * 8 + kg + i] = _Float16(v - float(h));
        }
      }
    }
  };

  float acc[NI][NJ][4], X[NI][NJ][4];
  // Q6_K: sum of the completed K segments (see seg_kb)
  float tot[kQ6 ? NI : 1][kQ6 ? NJ : 1][4];
  bool have_tot = false;
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[i][j][v] = 0.f;

  // X += a P, or X = a P for the super-block's first group
  auto scale_add = [&](bool first, float at, const f4& P, float (&x)[4]) {
#pragma unroll
    for (int v = 0; v < 4; ++v) x[v] = first ? at * P[v] : fmaf(at, P[v], x[v]);
  };

  auto compute = [&](auto qc, uint32_t kb) __attribute__((always_inline)) {
    constexpr uint32_t q = decltype(qc)::value, buf = q & 1u;
    const uint32_t kp = kb & 1u;
    // Q4_K: the wave in its matrix-core section issues ahead of the other
    // wave of its SIMD (1-5% at config 4; Q6_K measured neutral to 3% slower)
    if constexpr (!kQ6) __builtin_amdgcn_s_setprio(1);
    // ---- one 16x16x32 MFMA per (row tile, token tile, group). Small wave
    // tiles issue the MFMAs of both groups of the step before any result is
    // scaled, so the matrix core pipelines them while the VALU applies a_tg;
    // large wave tiles scale row tile i while the MFMAs of row tile i+1 run. ----
    if constexpr (NI * NJ <= 8 && WR * WT <= 4) {
      f4 P[2][NI][NJ];
      float at[2][NJ];
#pragma unroll
      for (uint32_t gsel = 0; gsel < 2; ++gsel) {
        const uint32_t g = 2 * q + gsel;
        half8 af[NI], bf[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const uint32_t t = wt * NJ * 16 + j * 16 + lr;
          at[gsel][j] = Aa[kp][t * 8 + g];
          bf[j] = *reinterpret_cast<const half8*>(&Bs[buf][t * kStride + gsel * 32 + lk * 8]);
        }
#pragma unroll
        for (int i = 0; i < NI; ++i)
          af[i] = *reinterpret_cast<const half8*>(
              &As[buf][0][(wr * NI * 16 + i * 16 + lr) * kStride + gsel * kG1 + lk * 8]);
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
          for (int j = 0; j < NJ; ++j)
            P[gsel][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], f4{0, 0, 0, 0}, 0, 0, 0);
        if constexpr (kQ6) {
#pragma unroll
          for (int i = 0; i < NI; ++i) {
            af[i] = *reinterpret_cast<const half8*>(
                &As[buf][kPlanes - 1][(wr * NI * 16 + i * 16 + lr) * kStride + gsel * kG1 + lk * 8]);
#pragma unroll
            for (int j = 0; j < NJ; ++j)  // hi + lo partial sums stay exact integers below 2^24
              P[gsel][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], P[gsel][i][j], 0, 0, 0);
          }
        }
      }
#pragma unroll
      for (uint32_t gsel = 0; gsel < 2; ++gsel)
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
          for (int j = 0; j < NJ; ++j) scale_add(q == 0 && gsel == 0, at[gsel][j], P[gsel][i][j], X[i][j]);
    } else if constexpr (WR * WT <= 4) {
      // One wave per SIMD (512 registers): software pipeline over the 2 * NI
      // (group, row tile) items of the
      // step. The MFMAs of item u are issued before the scaling FMAs of item
      // u - 1, whose results are complete by then, so the matrix core and the
      // VALU work side by side instead of the FMAs waiting on the MFMAs they
      // read. The sched_group_barrier hints keep one MFMA and four FMAs
      // interleaved.
      float at[2][NJ];
      half8 bf[NJ];  // reloaded per group: all MFMAs of group 0 precede group 1's
      f4 Pp[NJ];
#pragma unroll
      for (uint32_t u = 0; u <= 2 * NI; ++u) {
        const uint32_t gsel = u / NI, i = u % NI;
        f4 Pc[NJ];
        if (u < 2 * NI) {
          if (i == 0) {
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
              const uint32_t t = wt * NJ * 16 + j * 16 + lr;
              at[gsel][j] = Aa[kp][t * 8 + 2 * q + gsel];
              bf[j] = *reinterpret_cast<const half8*>(&Bs[buf][t * kStride + gsel * 32 + lk * 8]);
            }
          }
          const uint32_t ro = (wr * NI * 16 + i * 16 + lr) * kStride + gsel * kG1 + lk * 8;
          const half8 af = *reinterpret_cast<const half8*>(&As[buf][0][ro]);
#pragma unroll
          for (int j = 0; j < NJ; ++j)
            Pc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[j], f4{0, 0, 0, 0}, 0, 0, 0);
          if constexpr (kQ6) {
            const half8 al = *reinterpret_cast<const half8*>(&As[buf][kPlanes - 1][ro]);
#pragma unroll
            for (int j = 0; j < NJ; ++j)  // hi + lo partial sums stay exact integers below 2^24
              Pc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bf[j], Pc[j], 0, 0, 0);
          }
        }
        if (u > 0) {
          const uint32_t pg = (u - 1) / NI, pi = (u - 1) % NI;
#pragma unroll
          for (int j = 0; j < NJ; ++j) scale_add(q == 0 && pg == 0, at[pg][j], Pp[j], X[pi][j]);
        }
        if (u > 0 && u < 2 * NI) {
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            __builtin_amdgcn_sched_group_barrier(0x008, kQ6 ? 2 : 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);            // VALU
          }
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) Pp[j] = Pc[j];
      }
    } else {  // two waves per SIMD: row tile i is scaled while row tile i + 1's MFMAs run
#pragma unroll
      for (uint32_t gsel = 0; gsel < 2; ++gsel) {
        const uint32_t g = 2 * q + gsel;
        float at[NJ];
        half8 bf[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const uint32_t t = wt * NJ * 16 + j * 16 + lr;
          at[j] = Aa[kp][t * 8 + g];
          bf[j] = *reinterpret_cast<const half8*>(&Bs[buf][t * kStride + gsel * 32 + lk * 8]);
        }
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          const uint32_t ro = (wr * NI * 16 + i * 16 + lr) * kStride + gsel * kG1 + lk * 8;
          const half8 af = *reinterpret_cast<const half8*>(&As[buf][0][ro]);
          f4 P[NJ];
#pragma unroll
          for (int j = 0; j < NJ; ++j)
            P[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[j], f4{0, 0, 0, 0}, 0, 0, 0);
          if constexpr (kQ6) {
            const half8 al = *reinterpret_cast<const half8*>(&As[buf][kPlanes - 1][ro]);
#pragma unroll
            for (int j = 0; j < NJ; ++j)  // hi + lo partial sums stay exact integers below 2^24
              P[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bf[j], P[j], 0, 0, 0);
          }
#pragma unroll
          for (int j = 0; j < NJ; ++j) scale_add(q == 0 && gsel == 0, at[j], P[j], X[i][j]);
        }
      }
    }

    if constexpr (!kQ6) __builtin_amdgcn_s_setprio(0);
    // Pin X here: otherwise the compiler defers the scaling FMAs of a
    // super-block's first steps and keeps (spills) their MFMA results.
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) asm volatile("" : "+v"(X[i][j][v]));

    // ---- end of super-block: acc' += d X' - dmin Y' (Dd holds d, -dmin) ----
    if constexpr (q == 3) {
      __builtin_amdgcn_sched_barrier(0);  // epilogue operands load after the step's MFMAs
      half4 mf[NI], uh[NJ], ul[NJ];
      if constexpr (!kQ6) {
#pragma unroll
        for (int i = 0; i < NI; ++i)
          mf[i] = lk < 2 ? *reinterpret_cast<const half4*>(&Mq[kp][(wr * NI * 16 + i * 16 + lr) * 8 + lk * 4])
                         : half4{0, 0, 0, 0};  // K = 8..15 of the MFMA: zero padding
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const uint32_t t = wt * NJ * 16 + j * 16 + lr;
          uh[j] = lk < 2 ? *reinterpret_cast<const half4*>(&Uh[kp][t * 8 + lk * 4]) : half4{0, 0, 0, 0};
          ul[j] = lk < 2 ? *reinterpret_cast<const half4*>(&Ul[kp][t * 8 + lk * 4]) : half4{0, 0, 0, 0};
        }
      }
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        float2 dd[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) dd[v] = Dd[kp][wr * NI * 16 + i * 16 + lk * 4 + v];
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          if constexpr (!kQ6) {
            f4 Y = __builtin_amdgcn_mfma_f32_16x16x16f16(mf[i], uh[j], f4{0, 0, 0, 0}, 0, 0, 0);
            Y = __builtin_amdgcn_mfma_f32_16x16x16f16(mf[i], ul[j], Y, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v)
              acc[i][j][v] = fmaf(dd[v].y, Y[v], fmaf(dd[v].x, X[i][j][v], acc[i][j][v]));
          } else {
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[i][j][v] = fmaf(dd[v].x, X[i][j][v], acc[i][j][v]);
          }
        }
      }
      if constexpr (kQ6) {
        if (seg_kb && (kb + 1) % seg_kb == 0 && kb + 1 < kb_hi) {  // a segment ends inside the range
#pragma unroll
          for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
              for (int v = 0; v < 4; ++v) {
                tot[i][j][v] = have_tot ? tot[i][j][v] + acc[i][j][v] : acc[i][j][v];
                acc[i][j][v] = 0.f;
              }
          have_tot = true;
        }
      }
    }
  };

  // One step: wait for step (kb, q) to be staged, stage step s+1 from the
  // registers, load a later step into them, then compute step s. The stores
  // of the last step and the loads past the end land in the buffer and
  // super-block slot that no remaining step reads (or re-read the last
  // super-block).
  // Between two barriers the store of step s+1 and the compute of step s touch
  // different LDS buffers and super-block slots, so either order is valid. In
  // eight-wave tiles the second wave of each SIMD (waves 4..7) computes
  // first and stages second, so the two waves sharing a SIMD overlap staging
  // with matrix-core work instead of passing the phases together. compute,
  // store and fetch are then called from two places each; they are forced
  // inline, because an out-of-line copy takes the accumulator arrays by
  // reference and puts them in scratch (608 B per lane on the 256 x 128 tile).
  constexpr bool kPingPong = WR * WT == 8 && NI * NJ <= 16;
  const bool compute_first = kPingPong && wave >= 4;
  // Register sets: with two, step s+3 is loaded at step s (a load has two
  // steps to arrive before its store); with one, step s+2 (one step).
  // Small wave tiles have the registers for the second set.
  constexpr int kSets = NI * NJ <= 8 ? 2 : 1;
  Fetch<ZW, GPT, AW> F[kSets];
  auto step = [&](auto qc, uint32_t kb) {
    constexpr uint32_t q = decltype(qc)::value, f = kSets == 2 ? (q + 1) & 1u : 0u;
    __syncthreads();  // step s staged; step s-1 fully consumed
    if (compute_first) compute(qc, kb);
    store(std::integral_constant<uint32_t, (q + 1) & 3u>{}, kb + (q == 3 ? 1u : 0u), F[f]);
    if constexpr (kSets == 2)
      fetch(std::integral_constant<uint32_t, (q + 3) & 3u>{}, kb + (q >= 1 ? 1u : 0u), F[f]);
    else
      fetch(std::integral_constant<uint32_t, (q + 2) & 3u>{}, kb + (q >= 2 ? 1u : 0u), F[f]);
    if (!compute_first) compute(qc, kb);
  };

  fetch(std::integral_constant<uint32_t, 0>{}, kb_lo, F[0]);
  store(std::integral_constant<uint32_t, 0>{}, kb_lo, F[0]);
  fetch(std::integral_constant<uint32_t, 1>{}, kb_lo, F[kSets - 1]);
  if constexpr (kSets == 2) fetch(std::integral_constant<uint32_t, 2>{}, kb_lo, F[0]);
  for (uint32_t kb = kb_lo; kb < kb_hi; ++kb) {
    step(std::integral_constant<uint32_t, 0>{}, kb);
    step(std::integral_constant<uint32_t, 1>{}, kb);
    step(std::integral_constant<uint32_t, 2>{}, kb);
    step(std::integral_constant<uint32_t, 3>{}, kb);
  }
  __syncthreads();  // Ti visible (also when kbs is small)
  if constexpr (kQ6) {
    if (have_tot && splitk) {  // the run's first segment: its own partial
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const uint32_t tok = tok0 + wt * NJ * 16 + j * 16 + lr;
          const uint32_t r4 = row0 + wr * NI * 16 + i * 16 + lk * 4;
          if (tok >= m || r4 >= n) continue;
#pragma unroll
          for (int v = 0; v < 4; ++v)
            if (r4 + v < n) part_first[size_t(tok) * n + r4 + v] = tot[i][j][v];
        }
    } else if (have_tot) {
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[i][j][v] = tot[i][j][v] + acc[i][j][v];
    }
  }
  if constexpr (Glu) {
    // ---- SwiGLU -> Q8 epilogue. Gate waves (wr < WR / 2) park g in LDS (the
    // A tiles are free now); up wave wr + WR / 2 holds u of the same features
    // in the same register positions. A K32 feature group of token lr is row
    // tiles 2p, 2p + 1 of lanes lr + 16 lk: eight values in each of 4 lanes. ----
    static_assert(sizeof(As) >= size_t(HR) * BT * sizeof(float), "g tile fits the A tiles");
    float* gl = reinterpret_cast<float*>(&As[0][0][0]);
    const bool gate_wave = wr < uint32_t(WR / 2);
    const uint32_t wq = gate_wave ? wr : wr - WR / 2;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const float inv = Ti[wt * NJ * 16 + j * 16 + lr];
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[i][j][v] *= inv;
    }
    if (gate_wave) {
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int v = 0; v < 4; ++v)
            gl[(wq * NI * 16 + i * 16 + lk * 4 + v) * BT + wt * NJ * 16 + j * 16 + lr] = acc[i][j][v];
    }
    __syncthreads();
    if (gate_wave) return;
    const uint32_t groups_out = n / 32;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint32_t tl = wt * NJ * 16 + j * 16 + lr, tok = tok0 + tl;
#pragma unroll
      for (int p = 0; p < NI / 2; ++p) {
        float x[8];
        float peak = 0.f;
        int finite = 1;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const float g = gl[(wq * NI * 16 + (2 * p + h) * 16 + lk * 4 + v) * BT + tl];
            const float y = swiglu_q8_value(g, acc[2 * p + h][j][v]);
            x[4 * h + v] = y;
            const bool f = isfinite(y);
            finite &= int(f);
            peak = fmaxf(peak, f ? fabsf(y) : 0.f);
          }
        peak = fmaxf(peak, __shfl_xor(peak, 16));
        peak = fmaxf(peak, __shfl_xor(peak, 32));
        finite &= __shfl_xor(finite, 16);
        finite &= __shfl_xor(finite, 32);
        const float a = peak == 0.f ? 1.f : peak / 127.f;
        const bool valid = finite && isfinite(a) && a > 0.f;
        uint32_t word[2] = {0u, 0u};
        int sum = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int z = valid ? max(-127, min(127, int(rintf(x[e] / a)))) : 0;
          sum += z;
          word[e / 4] |= uint32_t(uint8_t(int8_t(z))) << (8 * (e % 4));
        }
        sum += __shfl_xor(sum, 16);
        sum += __shfl_xor(sum, 32);
        const uint32_t f0 = row0 + wq * NI * 16 + p * 32;  // first feature of the group
        if (tok >= m || f0 >= n) continue;
        int8_t* cp = glu.qc + size_t(tok) * n + f0 + lk * 4;
        *reinterpret_cast<uint32_t*>(cp) = word[0];
        *reinterpret_cast<uint32_t*>(cp + 16) = word[1];
        if (lk == 0) {
          const size_t gi = size_t(tok) * groups_out + f0 / 32;
          glu.qa[gi] = valid ? a : __uint_as_float(0x7fc00000u);
          glu.qs[gi] = sum;
          if (!valid) *glu.failure = 1;  // sticky flag, plain vector store
        }
      }
    }
    return;
  }
  // ---- store: lane holds rows 4*lk..4*lk+3 of token lr in each tile ----
  const bool vec = (n % 4 == 0) &&
                   ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(residual)) & 15u) == 0;
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint32_t tok = tok0 + wt * NJ * 16 + j * 16 + lr;
      const uint32_t r4 = row0 + wr * NI * 16 + i * 16 + lk * 4;
      if (tok >= m || r4 >= n) continue;
      const size_t o = size_t(tok) * n + r4;
      if constexpr (!kQ6) {  // acc' = ts acc: unscale (exact, a power of two)
        const float inv = Ti[wt * NJ * 16 + j * 16 + lr];
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[i][j][v] *= inv;
      }
      if (vec) {  // n % 4 == 0, so all four rows are in range
        float4 y = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
        if (residual) {
          const float4 rv = *reinterpret_cast<const float4*>(residual + o);
          y.x += rv.x; y.y += rv.y; y.z += rv.z; y.w += rv.w;
        }
        *reinterpret_cast<float4*>(out + o) = y;
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (r4 + v < n) out[o + v] = acc[i][j][v] + (residual ? residual[o + v] : 0.f);
      }
    }
}

// Launches one tile shape over weight rows [row_begin, row_end) (row_begin a
// multiple of the tile height; row_end = pn or a multiple of it).
// Glu: rows are features, glu carries the up weight and the Q8 outputs.
// Sum of the split segments in ascending order (plus the residual), the
// operation sequence of the unsplit kernel's segment sums and store.
__global__ void mmq_seg_reduce_kernel(const float* __restrict__ part, uint32_t segs, uint64_t count,
                                      const float* __restrict__ residual, float* __restrict__ out) {
  const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
  for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride) {
    float y = part[i];
    for (uint32_t sgm = 1; sgm < segs; ++sgm) y = y + part[sgm * count + i];
    out[i] = residual ? y + residual[i] : y;
  }
}

template <uint16_t Layout, int WR, int WT, int NI, int NJ, bool Glu = false>
hipError_t launch_cfg(const WeightView& w, const Q8View& x, float* out, const float* residual,
                      hipStream_t s, uint32_t row_begin, uint32_t row_end, GluOut glu = {},
                      uint32_t split = 1, float* part = nullptr) {
  using C = Cfg<WR, WT, NI, NJ>;
  constexpr uint32_t H = Glu ? C::BR / 2 : C::BR;
  const uint32_t row_blocks = (row_end - row_begin + H - 1) / H;
  const uint32_t tok_blocks = (x.m + C::BT - 1) / C::BT;
  if (row_blocks == 0) return hipSuccess;
  const uint32_t seg_kb = Layout == QW38_LAYOUT_Q6K_WAVE64 ? q6_seg_kb(w.pk / 256) : 0u;
  const uint32_t segs = seg_kb ? (w.pk / 256 + seg_kb - 1) / seg_kb : 1u;
  const dim3 grid(row_blocks * tok_blocks * (split > 1 ? split : 1));
  // 0x020D spans are 4-byte (codes) / 2-byte (metadata) aligned in general;
  // 16-byte aligned ones (every span this library allocates) load wide.
  const bool vec = ((reinterpret_cast<uintptr_t>(w.codes) | reinterpret_cast<uintptr_t>(w.scales) |
                     reinterpret_cast<uintptr_t>(glu.codes2) | reinterpret_cast<uintptr_t>(glu.meta2)) %
                    16) == 0;
  auto kern = mmq_kernel<Layout, true, WR, WT, NI, NJ, Glu>;
  if constexpr (Layout == QW38_LAYOUT_Q4K_CANDIDATE_V2)
    if (!vec) kern = mmq_kernel<Layout, false, WR, WT, NI, NJ, Glu>;
  hipLaunchKernelGGL(kern, grid, dim3(WR * WT * 64), 0, s, w.codes, w.scales,
                     w.n, w.pn, w.pk / 256, x.codes, x.scales, x.sums, x.m, x.pk, out, residual,
                     row_begin, row_blocks, tok_blocks, glu, seg_kb, split, part);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || split <= 1) return e;
  const uint64_t count = uint64_t(x.m) * w.n;
  const uint32_t rgrid = uint32_t(std::min<uint64_t>((count + 255) / 256, 4096));
  hipLaunchKernelGGL(mmq_seg_reduce_kernel, dim3(rgrid), dim3(256), 0, s, part, segs, count, residual, out);
  return hipGetLastError();
}

// The direct-copy Q6_K path's segment sum (mmq_seg_reduce_kernel).
hipError_t q6_seg_reduce(const float* part, uint32_t segs, uint32_t m, uint32_t n, const float* residual,
                         float* out, hipStream_t s) {
  const uint64_t count = uint64_t(m) * n;
  const uint32_t rgrid = uint32_t(std::min<uint64_t>((count + 255) / 256, 4096));
  hipLaunchKernelGGL(mmq_seg_reduce_kernel, dim3(rgrid), dim3(256), 0, s, part, segs, count, residual, out);
  return hipGetLastError();
}

// Q6_K 160 x 128 eight-wave tile: microseconds per two-group K step at one
// block per CU (measured).
constexpr double kQ6Step160 = 1.71;

// Glu: the tile cost model runs over the 2 n virtual rows of gate and up, and
// the launches get feature ranges (virtual rows / 2).
// QW38_MMQ_I8=1: the direct-copy 256 x 128 tiles on the int8 matrix cores
// (unfused calls; the same bits).
static bool mmq_i8_env() {
  static const bool v = [] {
    const char* e = std::getenv("QW38_MMQ_I8");
    return e && std::atoi(e) == 1;
  }();
  return v;
}

// QW38_MMQ_DMA: 0 turns the direct-copy tiles off, 2 keeps them off the
// 128 x 32 tiles (tuning aids: every setting gives the same bits).
static int mmq_dma_env() {
  static const int v = [] {
    const char* e = std::getenv("QW38_MMQ_DMA");
    return e ? std::atoi(e) : 1;
  }();
  return v;
}

// Batched-decode passes for M = 9..24 (unfused projections): ceil(M / 8)
// token slices of 4..8 tokens through launch_gemv. Its kernels at M 2..8
// (Q4_K 0x020D) and 3..8 (Q6_K) compute each token's rows independently of
// the call's other tokens, so every token gets that family's bits. The
// estimate per pass is those kernels' time at M = 8 (about 8 us plus the
// weight bytes at 4.5 TB/s: 5120 x 5120 11.7 us, 12288 x 5120 15, 34816 x
// 5120 29, Q6_K 5120 x 17408 21 with its segment sum); the caller compares it
// with its MMQ estimate. QW38_DECODE_PASSES=0 turns it off.
static double decode_passes_us(const WeightView& w, const Q8View& x) {
  static const int env = [] {
    const char* e = std::getenv("QW38_DECODE_PASSES");
    return e ? std::atoi(e) : 1;
  }();
  const bool q6 = w.layout == QW38_LAYOUT_Q6K_WAVE64;
  if (!env || x.m < 9 || x.m > 24 || (!q6 && w.layout != QW38_LAYOUT_Q4K_CANDIDATE_V2)) return 1e30;
  // the batched-decode kernels' alignment (other spans take other kernels)
  if ((reinterpret_cast<uintptr_t>(w.codes) | reinterpret_cast<uintptr_t>(w.scales) |
       reinterpret_cast<uintptr_t>(x.codes)) % 16)
    return 1e30;
  const double bytes = double(w.pn) * w.pk * (q6 ? 210.0 / 256 : 144.0 / 256);
  return double((x.m + 7) / 8) * (8.0 + bytes / 4.5e6);
}

static hipError_t run_decode_passes(const WeightView& w, const Q8View& x, float* out, const float* residual,
                                    hipStream_t s) {
  const uint32_t p = (x.m + 7) / 8, base = x.m / p, extra = x.m % p, groups = x.pk / 32;
  uint32_t t0 = 0;
  for (uint32_t i = 0; i < p; ++i) {
    const uint32_t mi = base + (i < extra ? 1u : 0u);
    const Q8View xi{x.codes + size_t(t0) * x.pk, x.scales + size_t(t0) * groups, x.sums + size_t(t0) * groups,
                    mi, x.k, x.pk};
    const hipError_t e = launch_gemv(w, xi, out + size_t(t0) * w.n, residual ? residual + size_t(t0) * w.n : nullptr, s);
    if (e != hipSuccess) return e;
    t0 += mi;
  }
  return hipSuccess;
}

template <uint16_t Layout, bool Glu = false>
hipError_t mmq_dispatch(const WeightView& w, const Q8View& x, float* out, const float* residual,
                        hipStream_t s, GluOut glu = {}) {
  // QW38_MMQ_TILE=32|64|128 pins the token tile (256: 256 rows x 128 tokens;
  // 80: 80 x 128 on four waves; 33, 81, 129, 192: 128 x 32, 80 x 128,
  // 128 x 128 and 192 x 128 on eight waves; 34: 128 x 32 direct-copy);
  // QW38_MMQ_SPLIT=0 disables the tail split (tuning aids; every tile shape
  // and split gives bitwise-identical results).
  static const int forced = [] {
    const char* e = std::getenv("QW38_MMQ_TILE");
    return e ? std::atoi(e) : 0;
  }();
  static const bool split = [] {
    const char* e = std::getenv("QW38_MMQ_SPLIT");
    return !(e && std::atoi(e) == 0);
  }();
  // Tile choice by a cost model of the busiest CU: with b blocks on it, a
  // shape that runs two blocks per CU costs floor(b/2) * t2 + (b % 2) * t1
  // per K step, a one-per-CU shape b * t1. Step times measured on MI355X
  // (microseconds per two-group K step): 256 x 128 t1 = 1.9 (Q6_K's 128 x 128:
  // 1.77); 128 x 64 t1 = 1.07, t2 = 1.39 (Q6_K 1.33, 2.65); 128 x 32
  // t1 = 0.70, t2 = 0.89 (Q6_K 1.0, 2.0). Small grids thus take smaller tiles
  // so that every CU has work.
  const uint32_t pn = Glu ? 2 * w.pn : w.pn;
  constexpr uint32_t kv = Glu ? 2 : 1;  // virtual rows per feature
  const uint32_t cus = uint32_t(cu_count());
  constexpr bool q6 = Layout == QW38_LAYOUT_Q6K_WAVE64;
  auto per_cu = [&](uint32_t rows, uint32_t toks) {
    const uint64_t tiles = uint64_t((pn + rows - 1) / rows) * ((x.m + toks - 1) / toks);
    return double((tiles + cus - 1) / cus);
  };
  auto two = [](double b, double t1, double t2) { return std::floor(b / 2) * t2 + std::fmod(b, 2.0) * t1; };
  // 256 x 128 tiles, one block per CU. When the last round of tiles would
  // leave most CUs idle, the big tiles cover whole rounds of row blocks and
  // the remaining rows run as 128 x 32 tiles (two blocks per CU) when they
  // fit one such round, which takes about half as long as a big round.
  uint32_t big_rows = pn;
  double b_big = per_cu(q6 ? 128u : 256u, 128);
  if constexpr (!q6) {
    const uint32_t rb = (pn + 255) / 256, tb = (x.m + 127) / 128;
    if (split && !forced && uint64_t(rb) * tb > cus) {
      const uint32_t full_rb = uint32_t(uint64_t(rb * tb / cus) * cus / tb);
      if (full_rb > 0 && full_rb < rb) {
        const uint64_t tail_blocks = uint64_t((pn - full_rb * 256 + 127) / 128) * ((x.m + 31) / 32);
        const uint64_t tail_rounds = (tail_blocks + 2 * cus - 1) / (2 * cus);
        if (tail_rounds <= 1) {
          big_rows = full_rb * 256;
          b_big = double(uint64_t(full_rb) * tb / cus) + 0.5;
        }
      }
    }
  }
  const double c_big = b_big * (q6 ? 1.77 : 1.9);
  const double c64 = q6 ? two(per_cu(128, 64), 1.33, 2.65) : two(per_cu(128, 64), 1.07, 1.39);
  // The direct-copy 128 x 32 tile (Q4_K 0x020D with the library scratch)
  // takes 0.86 of mmq_kernel's time at every grid size measured (5120 to
  // 34816 rows, M = 16 to 512).
  const bool dma32 = Layout == QW38_LAYOUT_Q4K_CANDIDATE_V2 && mmq_dma_env() == 1 && x.pk == w.pk &&
                      (w.pk / 256) % 2 == 0;
  const double c32 = q6 ? two(per_cu(128, 32), 1.0, 2.0) : two(per_cu(128, 32), 0.70, 0.89) * (dma32 ? 0.86 : 1.0);
  // 128 x 16 direct-copy tiles (the same kernel with one 16-token tile per
  // wave): a block step takes about 0.8 of the 128 x 32 direct-copy one
  // (5120 rows at M = 16: 41 against 50 us; 34816 rows at M = 16: 57 / 73,
  // M = 40: 94 / 106); no half-empty token tiles at M <= 16.
  const double c16 = dma32 ? two(per_cu(128, 16), 0.70, 0.89) * 0.86 * 0.8 : 1e30;
  // 80 x 128 on eight waves (one block per CU, two waves per SIMD; the
  // four-wave 80 x 128 tile, QW38_MMQ_TILE=80, is always slower): 5120-row
  // weights make 64 row blocks, so a 512-token chunk fills 256 CUs in one
  // round where 128-row tiles leave 96 idle. 1.07 us per step for Q6_K (the
  // down projection at M = 512: 290 against 393 us on four waves), 1.02 for
  // Q4_K.
  const double c81 = Glu ? 1e30 : per_cu(80, 128) * (q6 ? 1.07 : 1.02);
  // 128 x 128 with eight waves (two per SIMD, like the 256 x 128 tile; Q4_K
  // only): 1.18 us per step at one block per CU. It wins where 256-row
  // tiles leave CUs idle and the four-wave tiles lack the second wave per
  // SIMD (1.15 us per step at one block per CU).
  const double c129 = q6 ? 1e30 : per_cu(128, 128) * 1.15;
  // 192 x 128 on eight waves (Q4_K, unfused): 1.82 us per step; a 12288-row
  // weight makes 64 row blocks, one full round at M = 512 (146 against 162 us).
  const double c192 = (q6 || Glu) ? 1e30 : per_cu(192, 128) * 1.82;
  int bt = 32;
  double best = c32;
  if (c16 < best) bt = 35, best = c16;
  if (x.m > 32 && c64 < best) bt = 64, best = c64;
  if (x.m > 64 && c_big < best) bt = 256, best = c_big;
  if (x.m > 64 && c81 < best) bt = 81, best = c81;
  if (x.m > 64 && c129 < best) bt = 129, best = c129;
  if (x.m > 64 && c192 < best) bt = 192, best = c192;
  if (forced) bt = forced;
  if constexpr (!q6 && !Glu)  // MMQ estimate: the pick's steps + the direct-copy pre-pass
    if (!forced && decode_passes_us(w, x) < best * (w.pk / 256) * 4 + 7.0)
      return run_decode_passes(w, x, out, residual, s);
  // Q6_K: two more shapes, each unsplit or with the fixed K segments split
  // over blocks (one segment of one tile per block, then the ordered segment
  // sum, c_sum):
  //   80 x 128 eight-wave tile (1.07 us per step): split, the down projection
  //     at M = 128 makes 64 tiles x 4 segments = 256 blocks;
  //   160 x 128 eight-wave tile (wave tile 80 x 32: half the LDS fragment
  //     reads per MFMA of 80 x 16; 1.71 us per step).
  // Each cost is the busiest CU's share, rounds x steps x step time; taken
  // when below the unsplit pick (split launches only with the library scratch).
  if constexpr (q6 && !Glu) {
    const uint32_t kbs = w.pk / 256, seg = q6_seg_kb(kbs), segs = (kbs + seg - 1) / seg;
    static const bool split_env = [] {
      const char* e = std::getenv("QW38_MMQ_SPLITK");
      return !(e && std::atoi(e) == 0);
    }();
    auto rounds = [&](uint32_t rows, uint32_t runs) {
      const uint64_t blocks = uint64_t((pn + rows - 1) / rows) * ((x.m + 127) / 128) * runs;
      return double((blocks + cus - 1) / cus);
    };
    // the ordered segment sum reads every partial once: about 1.5 us plus the
    // partial bytes at 5 TB/s (3 us at M = 128, 9 us at M = 512 on 5120 rows)
    const double c_sum = 1.5 + double(segs) * x.m * w.n * 4 / 5e6;
    double c_best = forced ? 1e30 : best * kbs * 4;  // unsplit pick, whole launch
    int pick = 0;                                    // 81 / 160 unsplit, 82 / 162 split
    auto consider = [&](int id, double c) {
      if ((!forced && c < c_best) || forced == id) c_best = c, pick = id;
    };
    consider(160, rounds(160, 1) * kbs * 4 * kQ6Step160);
    if (split_env && segs > 1) {
      consider(82, rounds(80, segs) * seg * 4 * 1.07 + c_sum);
      consider(162, rounds(160, segs) * seg * 4 * kQ6Step160 + c_sum);
      if (segs % 2 == 0)  // runs of two segments
        consider(163, rounds(160, segs / 2) * 2 * seg * 4 * kQ6Step160 + c_sum);
    }
    // The direct-copy 160 x 128 tile (q4k_mmq_dma.hip; one fixed segment per
    // block, tokens in chunks the scratch holds) measured faster than every
    // tile above for all M > 128 at 5120 x 17408 (M = 160: 132 against
    // 146 us; 512: 230 / 260; 1536: 668 / 853; 2048: 887 / 924) and slower
    // at M = 128 (126 / 95), where one token tile leaves half the CUs idle.
    // M <= 128 with several K segments takes its 160 x 64 form (172: two
    // token tiles per 128 tokens, two blocks per CU): 5120 x 17408 at
    // M = 64 / 96 / 128 81 / 86 / 88 us against 90 / 92 / 92 for the split
    // tiles; 776 rows at M = 130 77 against 116. One segment (K = 2304,
    // M = 96): 45 against 32, so not there. M = 9..24 keeps the decode
    // passes (5120 rows, M = 24: 65.5 against 73.5 us for 172). 171 (80 x 128)
    // is a tuning id only. Each is priced just under the best tile above.
    if (mmq_dma_env() != 0 && x.pk == w.pk && w.pn % 8 == 0) {
      consider(170, x.m > 128 ? c_best * 0.9 : 1e30);
      consider(171, 1e30);
      consider(172, (x.m > 24 && x.m <= 128 && segs > 1) ? c_best * 0.95 : 1e30);
    }
    if (!forced && decode_passes_us(w, x) < c_best) return run_decode_passes(w, x, out, residual, s);
    if (pick == 170 || pick == 171 || pick == 172) {  // direct-copy 160 x 128 / 80 x 128 / 160 x 64, one segment per block
      const uint32_t cap = (x.m + 127) / 128 * 128;
      uint32_t mc = 0;
      for (uint32_t c = 128; c <= cap; c += 128)
        if (q6_mmq_dma_scratch_bytes(c, w.n, w.pk) <= kScratchBytes) mc = c;
      int dev = 0;
      if (void* sc = mc ? scratch_acquire(s, q6_mmq_dma_scratch_bytes(mc, w.n, w.pk), &dev) : nullptr) {
        const hipError_t e = launch_q6_mmq_dma(w, x, out, residual, s, sc, pick == 171 ? 5 : 10, pick == 172 ? 4 : 8, mc,
                                               q6_seg_reduce);
        scratch_release(dev, s, e == hipSuccess);
        return e;
      }
    }
    if (pick == 160) return launch_cfg<Layout, 2, 4, 5, 2>(w, x, out, residual, s, 0, pn);  // 160 x 128
    if (pick == 82 || pick == 162 || pick == 163) {
      int dev = 0;
      if (void* part = scratch_acquire(s, uint64_t(segs) * x.m * w.n * 4, &dev)) {
        float* pp = static_cast<float*>(part);
        const uint32_t runs = pick == 163 ? segs / 2 : segs;
        const hipError_t e = pick == 82
                                 ? launch_cfg<Layout, 1, 8, 5, 1>(w, x, out, residual, s, 0, pn, {}, runs, pp)
                                 : launch_cfg<Layout, 2, 4, 5, 2>(w, x, out, residual, s, 0, pn, {}, runs, pp);
        scratch_release(dev, s, e == hipSuccess);
        return e;
      }
    }
  }
  if (bt == 82 || (bt > 160 && bt < 192)) bt = 81;  // Q6_K split ids without the scratch
  if (bt == 80) return launch_cfg<Layout, 1, 4, 5, 2>(w, x, out, residual, s, 0, pn);  // 80 x 128
  // Q6_K grids of at most one 128 x 32 block per CU (M <= 128 on 5120 rows)
  // run it on eight waves (16 x 32 each, two per SIMD, ping-pong order):
  // down projection at M=128 241 -> 219 us. Q4_K gained nothing this way.
  if constexpr (q6)
    if (bt == 32 && !forced && per_cu(128, 32) <= 1.0) bt = 33;
  if constexpr (!Glu)
    if (bt == 33) return launch_cfg<Layout, 8, 1, 1, 2>(w, x, out, residual, s, 0, pn);  // 128 x 32, 8 waves
  if constexpr (!q6)
    if (bt == 129) return launch_cfg<Layout, 2, 4, 4, 2, Glu>(w, x, out, residual, s, 0, pn / kv, glu);  // 128 x 128, 8 waves
  if constexpr (!q6 && !Glu)
    if (bt == 192) return launch_cfg<Layout, 4, 2, 3, 4>(w, x, out, residual, s, 0, pn);  // 192 x 128, 8 waves
  if constexpr (!Glu)
    if (bt == 81) return launch_cfg<Layout, 1, 8, 5, 1>(w, x, out, residual, s, 0, pn);  // 80 x 128, 8 waves
  const uint32_t end = pn / kv;
  // 0x020D with 16-byte aligned spans: the direct-copy form of the 256 x 128
  // and 128 x 32 tiles (q4k_mmq_dma.hip, bitwise-equal outputs) when the
  // library scratch holds its pre-pass: rows [0, big) on the big tile, [big,
  // end) on the small one. hipErrorNotReady when it does not apply.
  const int dma_env = mmq_dma_env();
  // QW38_MMQ_DMA=2, or the int8 form (QW38_MMQ_I8=1, unfused; it has no tail
  // tiles): the direct-copy launch stops at the big tiles and mmq_kernel runs
  // the rest
  const bool dma_end_at_big = dma_env == 2 || (mmq_i8_env() && !Glu);
  auto try_dma = [&](uint32_t big, uint32_t tail_end, int tail_nj = 2) -> hipError_t {
    if constexpr (Layout == QW38_LAYOUT_Q4K_CANDIDATE_V2) {
      const bool aligned = ((reinterpret_cast<uintptr_t>(w.codes) | reinterpret_cast<uintptr_t>(w.scales) |
                             reinterpret_cast<uintptr_t>(x.codes) | reinterpret_cast<uintptr_t>(glu.codes2) |
                             reinterpret_cast<uintptr_t>(glu.meta2)) % 16) == 0;
      if (!dma_env || !aligned || x.pk != w.pk || (w.pk / 256) % 2 != 0) return hipErrorNotReady;
      if (dma_end_at_big) tail_end = big;
      if (tail_end == 0) return hipErrorNotReady;
      int dev = 0;
      void* sc = scratch_acquire(s, mmq_dma_scratch_bytes(x.m, x.pk), &dev);
      if (!sc) return hipErrorNotReady;
      hipError_t e;
      if constexpr (Glu) {
        const WeightView up{glu.codes2, glu.meta2, w.layout, w.n, w.k, w.pn, w.pk};
        e = launch_mmq_dma(w, x, nullptr, nullptr, s, big, tail_end, sc, &up, glu.qc, glu.qa, glu.qs,
                           glu.failure, tail_nj);
      } else {
        e = launch_mmq_dma(w, x, out, residual, s, big, tail_end, sc, nullptr, nullptr, nullptr, nullptr, nullptr,
                           tail_nj);
      }
      scratch_release(dev, s, e == hipSuccess);
      return e;
    }
    return hipErrorNotReady;
  };
  if (bt == 32 && !forced && dma32) bt = 34;
  if (bt == 34 || bt == 35) {  // 128 x 32 / 128 x 16 direct-copy over all rows
    const hipError_t e = try_dma(0, end, bt == 35 ? 1 : 2);
    if (e != hipErrorNotReady) return e;
    bt = 32;
  }
  if (bt == 32) return launch_cfg<Layout, 4, 1, 2, 2, Glu>(w, x, out, residual, s, 0, end, glu);  // 128 x 32
  if (bt == 64) return launch_cfg<Layout, 4, 1, 2, 4, Glu>(w, x, out, residual, s, 0, end, glu);  // 128 x 64
  if constexpr (q6) {  // Q6_K's two A planes: 128 x 128 at most
    return launch_cfg<Layout, 2, 2, 4, 4>(w, x, out, residual, s, 0, pn);
  } else {
    if (bt == 128) return launch_cfg<Layout, 2, 2, 4, 4, Glu>(w, x, out, residual, s, 0, end, glu);  // 128 x 128
    if (forced) big_rows = pn;
    const uint32_t dma_end = dma_end_at_big ? big_rows / kv : end;
    hipError_t e = try_dma(big_rows / kv, dma_end, dma_env == 3 ? 1 : 2);
    if (e == hipSuccess && dma_end == end) return e;
    if (e == hipErrorNotReady) e = launch_cfg<Layout, 4, 2, 4, 4, Glu>(w, x, out, residual, s, 0, big_rows / kv, glu);
    if (e != hipSuccess || big_rows == pn) return e;
    return launch_cfg<Layout, 4, 1, 2, 2, Glu>(w, x, out, residual, s, big_rows / kv, end, glu);
  }
}

}  // namespace

// Compute units of the current device (cached per device).
int cu_count() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cached[dev] = v;
  }
  return cached[dev];
}

hipError_t launch_mmq(const WeightView& w, const Q8View& x, float* out, const float* residual,
                      hipStream_t s) {
  switch (w.layout) {
    case QW38_LAYOUT_Q4K_CANDIDATE_V2:
      return mmq_dispatch<QW38_LAYOUT_Q4K_CANDIDATE_V2>(w, x, out, residual, s);
    case QW38_LAYOUT_Q4K_WAVE64:
      return mmq_dispatch<QW38_LAYOUT_Q4K_WAVE64>(w, x, out, residual, s);
    case QW38_LAYOUT_Q6K_WAVE64:
      return mmq_dispatch<QW38_LAYOUT_Q6K_WAVE64>(w, x, out, residual, s);
    default:
      return hipErrorInvalidValue;
  }
}

hipError_t launch_mmq_glu(const WeightView& gate, const WeightView& up, const Q8View& x,
                          int8_t* codes, float* scales, int32_t* sums, int* failure,
                          hipStream_t s) {
  if (gate.layout != up.layout || gate.n != up.n || gate.pn != up.pn || gate.pk != up.pk ||
      gate.n % 32 != 0 || gate.pn != gate.n)
    return hipErrorInvalidValue;
  const GluOut glu{up.codes, up.scales, codes, scales, sums, failure};
  switch (gate.layout) {
    case QW38_LAYOUT_Q4K_CANDIDATE_V2:
      return mmq_dispatch<QW38_LAYOUT_Q4K_CANDIDATE_V2, true>(gate, x, nullptr, nullptr, s, glu);
    case QW38_LAYOUT_Q4K_WAVE64:
      return mmq_dispatch<QW38_LAYOUT_Q4K_WAVE64, true>(gate, x, nullptr, nullptr, s, glu);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace qw38hip
