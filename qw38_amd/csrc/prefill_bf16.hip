// BF16 prefill projection over Q4_K weights (layout 0x020D) on gfx950 matrix
// cores: Y[m][n] = X[m][k] (BF16) * W^T, W rebuilt as BF16 operands.
//
// Semantics (cuda/prefill.cu:62-77, 116-142, 510-715): every weight is the
// BF16 operand BF16_RNE(fl(fl(d * s_g) * c) - fl(dmin * m_g)) -- the same
// operand as the BF16 decode GEMV, built here with fma(ds, c, -dm), which is
// bit-identical because fl(d * s) * c is exact -- and the products with the
// BF16 activations are summed in FP32 (v_mfma_f32_16x16x32_bf16, the matrix
// core accumulating over all of K). Epilogues: StoreBf16, StoreFp32,
// ResidualAddFp32; the paired gate/up launch writes BF16(SiLU(g) * u).
//
// Block: 128 weight rows x 64 tokens, four waves as 2 x 2, each a 64 x 32
// wave tile of 16x16 outputs. Per 64-wide K step every thread rebuilds one
// (row, K32 group) of the weight tile (v_cvt_pk_bf16_f32 on pairs) and copies
// a quarter of a (token, K32 group) activation row; operands for step s+2
// are loaded into registers while step s runs on the matrix cores.
#include <cmath>
#include <cstdlib>

#include "common.hpp"

namespace qw38hip {
namespace {

typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef float fl2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kRows = 128, kToks = 64;
// LDS row stride in halfs: 64 BF16 + 16 pad. A stride of 40 dwords (an odd
// multiple of 8) keeps the wave's b128 fragment reads free of bank conflicts on
// the 64-bank LDS; 36 dwords (64 + 8 halfs) halves the read rate.
constexpr int kStride = 80;
// Half offset of the second K32 group in a weight-tile row: 40 (20 dwords, an
// odd multiple of 4) instead of 32, so a store phase of lanes holding (row,
// group) pairs of four rows hits eight distinct 4-bank groups; the fragment
// reads stay conflict-free.
constexpr int kG1 = 40;

// Loads of one K step.
struct WFetch {
  uint32_t c[4];  // 16 code bytes of (row, group): sequential nibbles
  uint32_t m[4];  // the super-block's metadata row
};

template <bool Fast>
__device__ __forceinline__ void fetch_w(const uint8_t* codes, const uint8_t* meta, uint64_t tr,
                                        uint32_t g, WFetch& f) {
  const uint8_t* cp = codes + tr * 128 + g * 16;
  const uint8_t* mp = meta + tr * 16;
  if constexpr (Fast) {
    const uint4 cv = *reinterpret_cast<const uint4*>(cp);
    const uint4 mv = *reinterpret_cast<const uint4*>(mp);
    f.c[0] = cv.x; f.c[1] = cv.y; f.c[2] = cv.z; f.c[3] = cv.w;
    f.m[0] = mv.x; f.m[1] = mv.y; f.m[2] = mv.z; f.m[3] = mv.w;
  } else {  // 2-byte aligned spans (the reference's minimum)
    const uint16_t* c2 = reinterpret_cast<const uint16_t*>(cp);
    const uint16_t* m2 = reinterpret_cast<const uint16_t*>(mp);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f.c[i] = uint32_t(c2[2 * i]) | (uint32_t(c2[2 * i + 1]) << 16);
      f.m[i] = uint32_t(m2[2 * i]) | (uint32_t(m2[2 * i + 1]) << 16);
    }
  }
}

// 32 BF16 operands of (row, group g) into LDS (64 B).
__device__ __forceinline__ void store_w(const WFetch& f, uint32_t g, _Float16* dst_h) {
  float s, m;
  q4_scale_min_lane(f.m[1], f.m[2], f.m[3], g, s, m);
  const float ds = f16_to_f32(f.m[0] & 0xffffu) * s;            // exact
  const float ndm = -(f16_to_f32(f.m[0] >> 16) * m);           // exact
  uint32_t o[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // code word i = codes 8i..8i+7 (byte b: codes 2b, 2b+1)
    uint32_t lo = f.c[i] & 0x0f0f0f0fu, hv = (f.c[i] >> 4) & 0x0f0f0f0fu;
    // Opaque to the optimizer, so each byte converts with one
    // v_cvt_f32_ubyte{0..3} instead of a bit-field extract and a convert.
    asm volatile("" : "+v"(lo), "+v"(hv));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const fl2 wv = {fmaf(ds, float((lo >> (8 * q)) & 0xffu), ndm),
                      fmaf(ds, float((hv >> (8 * q)) & 0xffu), ndm)};
      o[4 * i + q] = __builtin_bit_cast(uint32_t, __builtin_convertvector(wv, bf2));
    }
  }
  uint4* dst = reinterpret_cast<uint4*>(dst_h);
#pragma unroll
  for (int i = 0; i < 4; ++i) dst[i] = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
}


template <bool Paired, bool Fast, int TT = kToks>
__global__ __launch_bounds__(256, 2) void prefill_bf16_kernel(
    const uint8_t* __restrict__ codes_a, const uint8_t* __restrict__ meta_a,
    const uint8_t* __restrict__ codes_b, const uint8_t* __restrict__ meta_b, uint32_t n,
    uint32_t k, const uint16_t* __restrict__ x, uint32_t m, void* out,
    const float* __restrict__ residual, int epi, uint32_t row_blocks, uint32_t tok_blocks,
    uint32_t row_base) {
  constexpr int NW = Paired ? 2 : 1, NJ = TT / 32, HPT = TT / 4;  // HPT: activation halfs per thread
  static_assert(TT == 32 || TT == 64, "token tile");
  __shared__ __align__(16) _Float16 As[NW][kRows * kStride];
  __shared__ __align__(16) _Float16 Bs[TT * kStride];

  const uint32_t nblk = row_blocks * tok_blocks;
  const uint32_t b = blockIdx.x;
  const uint32_t tile = (nblk % 8 == 0) ? (b % 8) * (nblk / 8) + b / 8 : b;  // XCD-contiguous
  const uint32_t row0 = row_base + (tile / tok_blocks) * kRows, tok0 = (tile % tok_blocks) * TT;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t wr = wave >> 1, wt = wave & 1u, lr = lane & 15u, lk = lane >> 4;
  const uint32_t kbs = k / 256, steps = k / 64;
  const uint32_t pn8 = (n + 7) / 8 * 8;

  // A role: row ar (clamped), group-in-step asel. B role: token bt, 16 B part bp.
  const uint32_t ar = tid >> 1, asel = tid & 1u;
  const uint32_t arow = min(row0 + ar, pn8 - 1);
  const uint64_t trow0 = uint64_t(arow / 8) * kbs * 8 + arow % 8;
  const uint32_t bt = tid / (256 / TT), bp = tid % (256 / TT);
  const uint16_t* xrow = x + size_t(min(tok0 + bt, m - 1)) * k + bp * HPT;

  f4 acc[NW][4][NJ];
#pragma unroll
  for (int w = 0; w < NW; ++w)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[w][i][j] = f4{0, 0, 0, 0};

  // Two register sets: step s+2's operands are loaded while step s runs, so
  // a step never waits on the loads issued by the one before it.
  struct Stage {
    WFetch fa, fb;
    uint32_t xv[HPT / 2];
  };
  Stage st[2];
  auto fetch = [&](uint32_t s, Stage& f) {
    const uint32_t kb = s >> 2, g = 2 * (s & 3u) + asel;
    fetch_w<Fast>(codes_a, meta_a, trow0 + kb * 8, g, f.fa);
    if constexpr (Paired) fetch_w<Fast>(codes_b, meta_b, trow0 + kb * 8, g, f.fb);
    const uint16_t* xp = xrow + s * 64;
    if constexpr (Fast) {
#pragma unroll
      for (int q = 0; q < HPT / 8; ++q) {
        const uint4 v = reinterpret_cast<const uint4*>(xp)[q];
        f.xv[4 * q] = v.x; f.xv[4 * q + 1] = v.y; f.xv[4 * q + 2] = v.z; f.xv[4 * q + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < HPT / 2; ++i) f.xv[i] = uint32_t(xp[2 * i]) | (uint32_t(xp[2 * i + 1]) << 16);
    }
  };
  auto step = [&](uint32_t s, Stage& f) {
    __syncthreads();  // previous step's tiles fully read
    const uint32_t g = 2 * (s & 3u) + asel;
    store_w(f.fa, g, &As[0][ar * kStride + asel * kG1]);
    if constexpr (Paired) store_w(f.fb, g, &As[NW - 1][ar * kStride + asel * kG1]);
    {
      uint4* dst = reinterpret_cast<uint4*>(&Bs[bt * kStride + bp * HPT]);
#pragma unroll
      for (int q = 0; q < HPT / 8; ++q)
        dst[q] = make_uint4(f.xv[4 * q], f.xv[4 * q + 1], f.xv[4 * q + 2], f.xv[4 * q + 3]);
    }
    __syncthreads();
    if (s + 2 < steps) fetch(s + 2, f);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf8 bfr[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        bfr[j] = *reinterpret_cast<const bf8*>(&Bs[(wt * (TT / 2) + j * 16 + lr) * kStride + ks * 32 + lk * 8]);
#pragma unroll
      for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bf8 afr = *reinterpret_cast<const bf8*>(
              &As[w][(wr * 64 + i * 16 + lr) * kStride + ks * kG1 + lk * 8]);
#pragma unroll
          for (int j = 0; j < NJ; ++j)
            acc[w][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(afr, bfr[j], acc[w][i][j], 0, 0, 0);
        }
    }
  };

  // K is a whole number of 256-wide super-blocks, so steps is a multiple of 4.
  fetch(0, st[0]);
  fetch(1, st[1]);
  for (uint32_t s = 0; s < steps; s += 2) {
    step(s, st[0]);
    step(s + 1, st[1]);
  }

  // ---- epilogue: lane holds rows 4 lk .. 4 lk + 3 of token lr in each tile ----
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint32_t tok = tok0 + wt * (TT / 2) + j * 16 + lr;
      if (tok >= m) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const uint32_t row = row0 + wr * 64 + i * 16 + lk * 4 + v;
        if (row >= n) continue;
        const size_t o = size_t(tok) * n + row;
        const float y = acc[0][i][j][v];
        if constexpr (Paired) {
          static_cast<uint16_t*>(out)[o] = f32_to_bf16_rne(silu(y) * acc[NW - 1][i][j][v]);
        } else if (epi == QW38_DECODE_STORE_BF16) {
          static_cast<uint16_t*>(out)[o] = f32_to_bf16_rne(y);
        } else if (epi == QW38_DECODE_STORE_FP32) {
          static_cast<float*>(out)[o] = y;
        } else {
          static_cast<float*>(out)[o] = residual[o] + y;
        }
      }
    }
}

// Large-M variants: 256 weight rows x BT tokens per block (BT = 128 or 256),
// eight waves as 4 x 2 with 64 x BT/2 wave tiles (sixteen or thirty-two
// independent accumulators each, so the matrix core never waits on its own
// results). LDS is double-buffered: one barrier per 64-wide K step separates
// the staging of step s+1 from the last reads of that buffer at step s-1,
// and step s+2's operands are loaded into registers while step s runs. The
// 256-token tile fills the 160 KB of LDS exactly; against the 128-token one
// it reads a quarter fewer LDS bytes and rebuilds half the weight operands
// per FLOP (gfx950 serves conflict-free b128 LDS reads at about 155 B per
// clock per CU, close to what the 128-token tile's MFMAs need).
//
// Paired (gate / up SwiGLU): a tile covers 128 features, its rows 0..127
// from the gate weight and 128..255 from the up weight (threads 0..255 stage
// gate rows, 256..511 up rows, so the weight choice is wave-uniform). Waves
// 0..3 hold g and waves 4..7 u of the same features in the same register
// positions; after K the gate waves park g in LDS and the up waves write
// BF16(SiLU(g) * u). Each g and u is the same MFMA chain as in the
// 128 x 64 paired kernel, so both give bitwise-identical outputs.
template <int BT, bool Fast, bool Paired = false>
__global__ __launch_bounds__(512, 1) void prefill_bf16_big_kernel(
    const uint8_t* __restrict__ codes, const uint8_t* __restrict__ meta,
    const uint8_t* __restrict__ codes_b, const uint8_t* __restrict__ meta_b, uint32_t n, uint32_t k,
    const uint16_t* __restrict__ x, uint32_t m, void* out, const float* __restrict__ residual,
    int epi, uint32_t row_blocks, uint32_t tok_blocks, uint32_t row_base) {
  constexpr int BR = 256, NJ = BT / 32, XP = BT / 128;  // XP: 32-byte activation parts per thread
  constexpr int HR = Paired ? BR / 2 : BR;              // output rows (features) per tile
  static_assert(BT == 128 || BT == 256, "token tile");
  // LDS: the plain kernel indexes separate A and B arrays, the paired one
  // offsets into a single array that also holds the parked gate tile after
  // K. Each form is the one measured fastest for its kernel on one box (plain
  // at N=34816, M=96: 96.7 against 113.6 us with per-buffer pointer
  // arithmetic; paired at 17408 features, M=512: 313 against 382 us with
  // two arrays), which the matrix-core issue order the compiler picks
  // follows.
  // (Each instantiation references only its own arrays.)
  __shared__ __align__(16) _Float16 smem[2 * (BR + BT) * kStride];
  __shared__ __align__(16) _Float16 a_lds[2][BR * kStride];
  __shared__ __align__(16) _Float16 b_lds[2][BT * kStride];
  static_assert(!Paired || sizeof(smem) >= size_t(HR) * BT * sizeof(float), "g tile fits");
  auto As = [&](uint32_t buf, uint32_t o) -> _Float16* {
    if constexpr (Paired) return smem + buf * (BR * kStride) + o;
    else return &a_lds[buf][o];
  };
  auto Bs = [&](uint32_t buf, uint32_t o) -> _Float16* {
    if constexpr (Paired) return smem + 2 * BR * kStride + buf * (BT * kStride) + o;
    else return &b_lds[buf][o];
  };

  const uint32_t nblk = row_blocks * tok_blocks, b = blockIdx.x;
  const uint32_t tile = (nblk % 8 == 0) ? (b % 8) * (nblk / 8) + b / 8 : b;
  const uint32_t row0 = row_base + (tile / tok_blocks) * HR, tok0 = (tile % tok_blocks) * BT;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t wr = wave >> 1, wt = wave & 1u, lr = lane & 15u, lk = lane >> 4;
  const uint32_t kbs = k / 256, steps = k / 64;
  const uint32_t pn8 = (n + 7) / 8 * 8;

  const uint32_t ar = tid >> 1, asel = tid & 1u;
  if constexpr (Paired) {
    if (__builtin_amdgcn_readfirstlane(tid >= 256u ? 1 : 0)) {
      codes = codes_b;
      meta = meta_b;
    }
  }
  const uint32_t arow = min(row0 + (Paired ? ar % HR : ar), pn8 - 1);
  const uint64_t trow0 = uint64_t(arow / 8) * kbs * 8 + arow % 8;
  // Activation role: token bt, 32-byte parts bp * XP .. bp * XP + XP - 1.
  const uint32_t bt = tid * XP / 4, bp = tid & (4u / XP - 1u);
  const uint16_t* xrow = x + size_t(min(tok0 + bt, m - 1)) * k + bp * XP * 16;

  f4 acc[4][NJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = f4{0, 0, 0, 0};

  WFetch fa;
  uint32_t xv[8 * XP];
  auto fetch = [&](uint32_t s) {
    fetch_w<Fast>(codes, meta, trow0 + (s >> 2) * 8, 2 * (s & 3u) + asel, fa);
    const uint16_t* xp = xrow + s * 64;
    if constexpr (Fast) {
#pragma unroll
      for (int q = 0; q < 2 * XP; ++q) {
        const uint4 v = reinterpret_cast<const uint4*>(xp)[q];
        xv[4 * q] = v.x; xv[4 * q + 1] = v.y; xv[4 * q + 2] = v.z; xv[4 * q + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8 * XP; ++i) xv[i] = uint32_t(xp[2 * i]) | (uint32_t(xp[2 * i + 1]) << 16);
    }
  };
  auto store = [&](uint32_t s) {
    const uint32_t buf = s & 1u;
    store_w(fa, 2 * (s & 3u) + asel, As(buf, ar * kStride + asel * kG1));
    uint4* dst = reinterpret_cast<uint4*>(Bs(buf, bt * kStride + bp * XP * 16));
#pragma unroll
    for (int q = 0; q < 2 * XP; ++q) dst[q] = make_uint4(xv[4 * q], xv[4 * q + 1], xv[4 * q + 2], xv[4 * q + 3]);
  };

  // Fragment reads of a K step are issued before the staging work that
  // follows the barrier, so LDS latency hides behind VALU and matrix-core
  // work. The 128-token tile holds both K halves' fragments at once; the
  // 256-token tile reads the second half's after the first half's MFMAs
  // (register budget: 128 accumulators of 256).
  constexpr int KH = BT == 128 ? 2 : 1;
  bf8 af[KH][4], bf[KH][NJ];
  auto read_frags = [&](uint32_t buf, int ks) {
    const int h = KH == 2 ? ks : 0;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      bf[h][j] = *reinterpret_cast<const bf8*>(Bs(buf, (wt * (BT / 2) + j * 16 + lr) * kStride + ks * 32 + lk * 8));
#pragma unroll
    for (int i = 0; i < 4; ++i)
      af[h][i] = *reinterpret_cast<const bf8*>(As(buf, (wr * 64 + i * 16 + lr) * kStride + ks * kG1 + lk * 8));
  };
  auto mma = [&](int ks) {
    const int h = KH == 2 ? ks : 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[h][i], bf[h][j], acc[i][j], 0, 0, 0);
  };

  fetch(0);
  store(0);
  if (steps > 1) fetch(1);
  // The second wave on each SIMD (waves 4-7) runs its MFMAs before its
  // staging work, so one wave's dequantization overlaps the other's matrix
  // work instead of both SIMD waves moving through the phases in step.
  const bool compute_first = wave >= 4;
  for (uint32_t s = 0; s < steps; ++s) {
    __syncthreads();
    const uint32_t buf = s & 1u;
    read_frags(buf, 0);
    // The wave in its matrix-core section issues ahead of the other wave of
    // its SIMD (s_setprio).
    if (compute_first) {
      __builtin_amdgcn_s_setprio(1);
      if constexpr (KH == 2) {
        read_frags(buf, 1);
        mma(0);
        mma(1);
      } else {
        mma(0);
        read_frags(buf, 1);
        mma(1);
      }
      __builtin_amdgcn_s_setprio(0);
      if (s + 1 < steps) store(s + 1);
      if (s + 2 < steps) fetch(s + 2);
    } else {
      if (s + 1 < steps) store(s + 1);
      if (s + 2 < steps) fetch(s + 2);
      __builtin_amdgcn_s_setprio(1);
      if constexpr (KH == 2) read_frags(buf, 1);
      mma(0);
      if constexpr (KH == 1) read_frags(buf, 1);
      mma(1);
      __builtin_amdgcn_s_setprio(0);
    }
  }

  if constexpr (Paired) {
    __syncthreads();  // every wave is past its last fragment read
    float* gl = reinterpret_cast<float*>(smem);
    const bool gate_wave = wave < 4;
    const uint32_t wq = wr & 1u;  // feature half of the tile
    if (gate_wave) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int v = 0; v < 4; ++v)
            gl[(wq * 64 + i * 16 + lk * 4 + v) * BT + wt * (BT / 2) + j * 16 + lr] = acc[i][j][v];
    }
    __syncthreads();
    if (gate_wave) return;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const uint32_t tl = wt * (BT / 2) + j * 16 + lr, tok = tok0 + tl;
        if (tok >= m) continue;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const uint32_t f = wq * 64 + i * 16 + lk * 4 + v, row = row0 + f;
          if (row >= n) continue;
          static_cast<uint16_t*>(out)[size_t(tok) * n + row] =
              f32_to_bf16_rne(silu(gl[f * BT + tl]) * acc[i][j][v]);
        }
      }
    return;
  }
  const bool vec = (n % 4 == 0) &&
                   ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(residual)) & 15u) == 0;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint32_t tok = tok0 + wt * (BT / 2) + j * 16 + lr;
      const uint32_t r4 = row0 + wr * 64 + i * 16 + lk * 4;
      if (tok >= m || r4 >= n) continue;
      const size_t o = size_t(tok) * n + r4;
      if (epi == QW38_DECODE_STORE_FP32 && vec) {
        *reinterpret_cast<float4*>(static_cast<float*>(out) + o) =
            make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
        continue;
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        if (r4 + v >= n) continue;
        const float y = acc[i][j][v];
        if (epi == QW38_DECODE_STORE_BF16) {
          static_cast<uint16_t*>(out)[o + v] = f32_to_bf16_rne(y);
        } else if (epi == QW38_DECODE_STORE_FP32) {
          static_cast<float*>(out)[o + v] = y;
        } else {
          static_cast<float*>(out)[o + v] = residual[o + v] + y;
        }
      }
    }
}

}  // namespace

hipError_t launch_prefill_bf16(const WeightView& a, const WeightView* b, const uint16_t* x,
                               uint32_t m, void* out, const float* residual, int epilogue,
                               hipStream_t s) {
  if (a.layout != QW38_LAYOUT_Q4K_CANDIDATE_V2 || a.pk != a.k) return hipErrorInvalidValue;
  auto al = [](const void* p, uintptr_t q) { return reinterpret_cast<uintptr_t>(p) % q == 0; };
  const bool fast = al(a.codes, 16) && al(a.scales, 16) && al(x, 16) && a.k % 8 == 0 &&
                    (!b || (al(b->codes, 16) && al(b->scales, 16)));
  // QW38_PREFILL_TILE=32|64|128|256 pins the token tile (tuning aid; every
  // tile gives bitwise-identical results).
  static const int forced = [] {
    const char* e = std::getenv("QW38_PREFILL_TILE");
    return e ? std::atoi(e) : 0;
  }();
  const uint32_t cus = uint32_t(cu_count());
  // 256 x BT tiles run one block per CU; a paired tile's 256 rows are 128
  // gate and 128 up rows of the same features. When their last round would
  // leave most CUs idle, they cover whole rounds of row blocks and the
  // remaining rows run as 128-row tiles when those fit one round. All
  // kernels chain the same MFMAs over K in the same order, so every split
  // gives bitwise-identical results.
  const uint32_t hr = b ? 128 : 256;  // output rows per big tile
  auto big_rows = [&](uint32_t bt) {
    const uint32_t rb = (a.n + hr - 1) / hr, tb = (m + bt - 1) / bt;
    if (uint64_t(rb) * tb > cus) {
      const uint32_t full_rb = uint32_t(uint64_t(rb) * tb / cus * cus / tb);
      const uint64_t tail = uint64_t((a.n - full_rb * hr + kRows - 1) / kRows) * ((m + kToks - 1) / kToks);
      if (full_rb > 0 && full_rb < rb && tail <= 2ull * cus) return full_rb;
    }
    return rb;
  };
  // Tile choice by a cost model of the busiest CU, in microseconds per
  // 64-wide K step measured on MI355X: 256 x 256 2.2, 256 x 128 1.2 (one
  // block per CU, paired or not); 128 x 64 0.79 alone, 0.86 for two
  // co-resident blocks (paired: 1.0 and 2.0).
  const double t1 = b ? 1.0 : 0.79, t2 = b ? 2.0 : 0.86;
  auto small_cost = [&](uint32_t rows) {
    const double bl = double((uint64_t(rows + kRows - 1) / kRows * ((m + kToks - 1) / kToks) + cus - 1) / cus);
    return std::floor(bl / 2) * t2 + std::fmod(bl, 2.0) * t1;
  };
  auto big_cost = [&](uint32_t bt, double t) {
    const uint32_t rb = big_rows(bt), tb = (m + bt - 1) / bt;
    const double rounds = double((uint64_t(rb) * tb + cus - 1) / cus);
    return rounds * t + (rb * hr < a.n ? small_cost(a.n - rb * hr) : 0.0);
  };
  int bt = 64;
  if (forced) {
    bt = forced;
  } else if (m > 64) {
    double best = small_cost(a.n);
    const double c128 = big_cost(128, 1.2), c256 = m > 128 ? big_cost(256, 2.2) : 1e30;
    if (c128 < best) bt = 128, best = c128;
    if (c256 < best) bt = 256;
  }
  const uint8_t* cb = b ? b->codes : nullptr;
  const uint8_t* mb = b ? b->scales : nullptr;
  uint32_t row_base = 0;
  if (bt == 128 || bt == 256) {
    const uint32_t rb = big_rows(uint32_t(bt)), tb = (m + bt - 1) / bt;
#define QW38_PF_BIG(T, F, P)                                                                          \
  hipLaunchKernelGGL((prefill_bf16_big_kernel<T, F, P>), dim3(rb * tb), dim3(512), 0, s, a.codes,      \
                     a.scales, cb, mb, a.n, a.k, x, m, out, residual, epilogue, rb, tb, 0u)
#define QW38_PF_BIG_F(T, P) \
  if (fast) QW38_PF_BIG(T, true, P); else QW38_PF_BIG(T, false, P)
    if (b) {
      if (bt == 256) { QW38_PF_BIG_F(256, true); } else { QW38_PF_BIG_F(128, true); }
    } else {
      if (bt == 256) { QW38_PF_BIG_F(256, false); } else { QW38_PF_BIG_F(128, false); }
    }
#undef QW38_PF_BIG_F
#undef QW38_PF_BIG
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || rb * hr >= a.n) return e;
    row_base = rb * hr;
  }
  // 128 x 32 tiles where 128 x 64 ones would leave CUs idle (a tail after
  // the big tiles, or at most 32 tokens).
  const uint32_t row_blocks = (a.n - row_base + kRows - 1) / kRows;
  const bool t32 = bt == 32 || (forced != 64 && (m <= 32 || uint64_t(row_blocks) * ((m + 63) / 64) < cus));
  const uint32_t tok_blocks = (m + (t32 ? 31 : 63)) / (t32 ? 32 : 64);
  const dim3 grid(row_blocks * tok_blocks);
#define QW38_PF_LAUNCH(P, F, T)                                                                      \
  hipLaunchKernelGGL((prefill_bf16_kernel<P, F, T>), grid, dim3(256), 0, s, a.codes, a.scales, cb, mb, \
                     a.n, a.k, x, m, out, residual, epilogue, row_blocks, tok_blocks, row_base)
#define QW38_PF_T(P, F) \
  if (t32) QW38_PF_LAUNCH(P, F, 32); else QW38_PF_LAUNCH(P, F, 64)
  if (b) {
    if (fast) { QW38_PF_T(true, true); } else { QW38_PF_T(true, false); }
  } else {
    if (fast) { QW38_PF_T(false, true); } else { QW38_PF_T(false, false); }
  }
#undef QW38_PF_T
#undef QW38_PF_LAUNCH
  return hipGetLastError();
}

}  // namespace qw38hip
