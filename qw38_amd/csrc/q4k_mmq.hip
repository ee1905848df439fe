// Prefill MMQ (M > 8) on gfx950 matrix cores.
//
// Exactness argument. For a Q4_K weight row r and K32 group g the reference
// contraction (cuda/q4k_q8.cu:140,245) is a_tg * (d_r s_rg dot_rtg -
// dmin_r m_rg sum_tg) with an exact int32 dot. Here the A operand holds the
// integers s_rg * w_rk (<= 63 * 15 = 945) and the B operand the int8 codes
// z_tk, both exact in FP16; one v_mfma_f32_16x16x32_f16 covers exactly one
// K32 group, and every partial sum of its products is an integer below 2^24,
// so the FP32 result P = s_rg * dot_rtg is exact regardless of the hardware's
// accumulation order. The FP32 affine is then, per super-block kb,
//   X_rt = sum_{g in kb} a_tg * P_rtg            (one FMA per output-group)
//   acc_rt += d_r * X_rt - dmin_r * sum_g m_rg (a_tg sum_tg)
// -- the same value as the reference's per-group expression, reassociated.
// Every tiling below runs the same per-(row, token) operation sequence, so all
// M-tile shapes give bitwise-identical outputs (the reference's J32 == J128
// property, tests/q4k_q8_test.cpp:118-120).
//
// Q6_K (layout 0x0241): A holds q - 32 (exact), two v_mfma_f32_16x16x16_f16
// per group give the sub-block dots, combined as a_tg * d * (sc0 P0 + sc1 P1).
#include "common.hpp"

namespace qw38hip {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int kStepK = 64;       // two K32 groups per LDS stage
constexpr int kLdsStride = 72;   // halfs per LDS row (64 + 8 pad: 144 B)

template <uint16_t Layout>
__device__ __forceinline__ void unpack32(const uint32_t w[4], uint32_t v[8]) {
#pragma unroll
  for (int t = 0; t < 4; ++t) {
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

// Tile config: 4 waves as WR x WT, each wave NI x NJ 16x16 output tiles.
template <int WR, int WT, int NI, int NJ>
struct Cfg {
  static constexpr int BR = WR * NI * 16;  // weight rows per block
  static constexpr int BT = WT * NJ * 16;  // tokens per block
};

template <uint16_t Layout, int WR, int WT, int NI, int NJ>
__global__ __launch_bounds__(256) void mmq_kernel(
    const uint8_t* __restrict__ codes, const uint8_t* __restrict__ meta, uint32_t n,
    uint32_t pn, uint32_t kbs, const int8_t* __restrict__ xc, const float* __restrict__ xa,
    const int32_t* __restrict__ xs, uint32_t m, uint32_t pk, float* __restrict__ out,
    const float* __restrict__ residual, uint32_t row_blocks, uint32_t tok_blocks) {
  using C = Cfg<WR, WT, NI, NJ>;
  constexpr bool kQ6 = Layout == QW38_LAYOUT_Q6K_WAVE64;
  __shared__ _Float16 As[C::BR * kLdsStride];
  __shared__ _Float16 Bs[C::BT * kLdsStride];
  __shared__ float Mm[C::BR * 8];   // Q4: m per group (float); Q6: sc0, sc1 per group pair
  __shared__ float Mq6[kQ6 ? C::BR * 8 : 1];
  __shared__ float Dd[C::BR * 2];   // d, dmin
  __shared__ float Aa[C::BT * 8];   // a per group
  __shared__ float Uu[C::BT * 8];   // a * sum per group

  // XCD-aware tile order: hardware places block b on XCD b % 8; give each XCD
  // a contiguous range of logical tiles so the token blocks of one weight-row
  // block share that XCD's L2.
  const uint32_t nblk = row_blocks * tok_blocks;
  const uint32_t b = blockIdx.x;
  // (a bijection only when the block count is a multiple of 8; else identity)
  const uint32_t tile = (nblk % 8 == 0) ? (b % 8) * (nblk / 8) + b / 8 : b;
  const uint32_t rb = tile / tok_blocks, tb = tile % tok_blocks;
  const uint32_t row0 = rb * C::BR, tok0 = tb * C::BT;

  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t wr = wave / WT, wt = wave % WT;
  const uint32_t lr = lane & 15u, lk = lane >> 4;
  const uint32_t groups = pk / 32;

  float acc[NI][NJ][4], X[NI][NJ][4];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[i][j][v] = X[i][j][v] = 0.f;

  const uint32_t steps = kbs * 4;
  for (uint32_t st = 0; st < steps; ++st) {
    const uint32_t kb = st / 4, q = st % 4;
    __syncthreads();
    // ---- stage A: BR rows x 2 groups (one row-group of 32 codes per thread) ----
    for (uint32_t idx = tid; idx < C::BR * 2; idx += 256) {
      const uint32_t r = idx / 2, gs = idx % 2, g = 2 * q + gs;
      const uint32_t row = row0 + r;
      _Float16* dst = As + r * kLdsStride + gs * 32;
      if (row < pn) {
        const uint64_t tr = (uint64_t(row / 8) * kbs + kb) * 8 + row % 8;
        uint32_t v[8];
        if constexpr (!kQ6) {
          const uint32_t* cp =
              reinterpret_cast<const uint32_t*>(codes + q4k_code_word(Layout, row, kb, g, kbs, pn / 8));
          uint32_t w[4] = {cp[0], cp[1], cp[2], cp[3]};
          unpack32<Layout>(w, v);
          const uint16_t* mp =
              reinterpret_cast<const uint16_t*>(meta + q4k_meta_row(Layout, row, kb, kbs, pn / 8));
          uint32_t mw[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) mw[i] = mp[i];
          const uint32_t p0 = mw[2] | (mw[3] << 16), p1 = mw[4] | (mw[5] << 16),
                         p2 = mw[6] | (mw[7] << 16);
          uint32_t s, mm;
          q4k_scale_min(p0, p1, p2, g, s, mm);
          Mm[r * 8 + g] = float(mm);
          if (q == 0 && gs == 0) {
            Dd[r * 2] = f16_to_f32(mw[0]);
            Dd[r * 2 + 1] = f16_to_f32(mw[1]);
          }
#pragma unroll
          for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              dst[4 * i + e] = _Float16(float(((v[i] >> (8 * e)) & 0xffu) * s));
        } else {
          const uint8_t* rowp = codes + tr * 192;
          const uint32_t* cp = reinterpret_cast<const uint32_t*>(rowp + g * 16);
          const uint32_t* hp = reinterpret_cast<const uint32_t*>(rowp + 128 + g * 8);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const uint32_t w = cp[j >> 1];
            const uint32_t nib = (j & 1) ? (w >> 4) & 0x0f0f0f0fu : w & 0x0f0f0f0fu;
            const uint32_t hh = (hp[j >> 2] >> (2 * (j & 3))) & 0x03030303u;
            v[j] = nib | (hh << 4);
          }
          const uint16_t scw = *reinterpret_cast<const uint16_t*>(meta + tr * 16 + g * 2);
          Mm[r * 8 + g] = float(int8_t(scw & 0xffu));
          Mq6[r * 8 + g] = float(int8_t(scw >> 8));
          if (q == 0 && gs == 0) {
            const uint64_t rows = uint64_t(pn) * kbs;
            Dd[r * 2] = f16_to_f32(*reinterpret_cast<const uint16_t*>(meta + rows * 16 + tr * 2));
            Dd[r * 2 + 1] = 0.f;
          }
#pragma unroll
          for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              dst[4 * i + e] = _Float16(float(int((v[i] >> (8 * e)) & 0xffu) - 32));
        }
      } else {
        for (int i = 0; i < 32; ++i) dst[i] = _Float16(0.f);
        Mm[r * 8 + g] = 0.f;
        if constexpr (kQ6) Mq6[r * 8 + g] = 0.f;
        if (q == 0 && gs == 0) { Dd[r * 2] = 0.f; Dd[r * 2 + 1] = 0.f; }
      }
    }
    // ---- stage B: BT tokens x 2 groups -----------------------------------------
    for (uint32_t idx = tid; idx < C::BT * 2; idx += 256) {
      const uint32_t t = idx / 2, gs = idx % 2, g = 2 * q + gs;
      const uint32_t tok = tok0 + t;
      _Float16* dst = Bs + t * kLdsStride + gs * 32;
      if (tok < m) {
        const size_t gi = size_t(tok) * groups + kb * 8 + g;
        const uint32_t* zp = reinterpret_cast<const uint32_t*>(xc + gi * 32);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t zw = zp[i];
#pragma unroll
          for (int e = 0; e < 4; ++e) dst[4 * i + e] = _Float16(float(int8_t(zw >> (8 * e))));
        }
        const float a = xa[gi];
        Aa[t * 8 + g] = a;
        Uu[t * 8 + g] = a * float(xs[gi]);
      } else {
        for (int i = 0; i < 32; ++i) dst[i] = _Float16(0.f);
        Aa[t * 8 + g] = 0.f;
        Uu[t * 8 + g] = 0.f;
      }
    }
    __syncthreads();

    // ---- MFMA over the two groups of this stage -------------------------------
#pragma unroll
    for (uint32_t gs = 0; gs < 2; ++gs) {
      const uint32_t g = 2 * q + gs;
      float at[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) at[j] = Aa[(wt * NJ * 16 + j * 16 + lr) * 8 + g];
      if constexpr (!kQ6) {
        half8 af[NI], bf[NJ];
#pragma unroll
        for (int i = 0; i < NI; ++i)
          af[i] = *reinterpret_cast<const half8*>(
              As + (wr * NI * 16 + i * 16 + lr) * kLdsStride + gs * 32 + lk * 8);
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          bf[j] = *reinterpret_cast<const half8*>(
              Bs + (wt * NJ * 16 + j * 16 + lr) * kLdsStride + gs * 32 + lk * 8);
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            const float4v zero = {0.f, 0.f, 0.f, 0.f};
            const float4v P = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], zero, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v) X[i][j][v] = fmaf(at[j], P[v], X[i][j][v]);
          }
      } else {
        // Two K16 sub-blocks: lanes hold k = 4*lk .. 4*lk+3 of each half.
        half4 af0[NI], af1[NI], bf0[NJ], bf1[NJ];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          const _Float16* p = As + (wr * NI * 16 + i * 16 + lr) * kLdsStride + gs * 32 + lk * 4;
          af0[i] = *reinterpret_cast<const half4*>(p);
          af1[i] = *reinterpret_cast<const half4*>(p + 16);
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const _Float16* p = Bs + (wt * NJ * 16 + j * 16 + lr) * kLdsStride + gs * 32 + lk * 4;
          bf0[j] = *reinterpret_cast<const half4*>(p);
          bf1[j] = *reinterpret_cast<const half4*>(p + 16);
        }
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          float s0[4], s1[4];
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const uint32_t r = wr * NI * 16 + i * 16 + lk * 4 + v;
            s0[v] = Mm[r * 8 + g];
            s1[v] = Mq6[r * 8 + g];
          }
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            const float4v zero = {0.f, 0.f, 0.f, 0.f};
            const float4v P0 = __builtin_amdgcn_mfma_f32_16x16x16f16(af0[i], bf0[j], zero, 0, 0, 0);
            const float4v P1 = __builtin_amdgcn_mfma_f32_16x16x16f16(af1[i], bf1[j], zero, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v)
              X[i][j][v] = fmaf(at[j], fmaf(s1[v], P1[v], s0[v] * P0[v]), X[i][j][v]);
          }
        }
      }
    }

    // ---- super-block epilogue: acc += d*X - dmin * sum_g m*(a*sum) -------------
    if (q == 3) {
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const uint32_t r = wr * NI * 16 + i * 16 + lk * 4 + v;
          const float d = Dd[r * 2], dmin = Dd[r * 2 + 1];
          float mg[8];
#pragma unroll
          for (int g = 0; g < 8; ++g) mg[g] = kQ6 ? 0.f : Mm[r * 8 + g];
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            if constexpr (!kQ6) {
              const uint32_t t = wt * NJ * 16 + j * 16 + lr;
              float mt = 0.f;
#pragma unroll
              for (int g = 0; g < 8; ++g) mt = fmaf(mg[g], Uu[t * 8 + g], mt);
              acc[i][j][v] = fmaf(-dmin, mt, fmaf(d, X[i][j][v], acc[i][j][v]));
            } else {
              acc[i][j][v] = fmaf(d, X[i][j][v], acc[i][j][v]);
            }
            X[i][j][v] = 0.f;
          }
        }
    }
  }

  // ---- store: lane holds rows 4*lk..4*lk+3 of token lr in each tile ------------
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint32_t tok = tok0 + wt * NJ * 16 + j * 16 + lr;
      if (tok >= m) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const uint32_t row = row0 + wr * NI * 16 + i * 16 + lk * 4 + v;
        if (row < n) {
          const size_t o = size_t(tok) * n + row;
          out[o] = acc[i][j][v] + (residual ? residual[o] : 0.f);
        }
      }
    }
}

template <uint16_t Layout, int WR, int WT, int NI, int NJ>
hipError_t mmq_launch(const WeightView& w, const Q8View& x, float* out, const float* residual,
                      hipStream_t s) {
  using C = Cfg<WR, WT, NI, NJ>;
  const uint32_t row_blocks = (w.pn + C::BR - 1) / C::BR;
  const uint32_t tok_blocks = (x.m + C::BT - 1) / C::BT;
  hipLaunchKernelGGL((mmq_kernel<Layout, WR, WT, NI, NJ>), dim3(row_blocks * tok_blocks),
                     dim3(256), 0, s, w.codes, w.scales, w.n, w.pn, w.pk / 256, x.codes,
                     x.scales, x.sums, x.m, x.pk, out, residual, row_blocks, tok_blocks);
  return hipGetLastError();
}

template <uint16_t Layout>
hipError_t mmq_dispatch(const WeightView& w, const Q8View& x, float* out, const float* residual,
                        hipStream_t s) {
  if (x.m <= 32) return mmq_launch<Layout, 4, 1, 2, 2>(w, x, out, residual, s);   // 128 x 32
  if (x.m <= 64) return mmq_launch<Layout, 2, 2, 4, 2>(w, x, out, residual, s);   // 128 x 64
  return mmq_launch<Layout, 2, 2, 4, 4>(w, x, out, residual, s);                  // 128 x 128
}

}  // namespace

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

}  // namespace qw38hip
