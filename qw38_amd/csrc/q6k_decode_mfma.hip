// Batched decode GEMV (M = 3..8 tokens) for Q6_K (layout 0x0241) on the int8
// matrix cores: v_mfma_i32_16x16x64_i8 with a block-diagonal activation
// operand, the Q6_K counterpart of the Q4_K kernel in q4k_decode_mfma.hip.
//
// Q6_K (GGML; the reference has no Q6_K code) gives row r and 16-code
// sub-block b the integer sc_rb (int8) and codes q in 0..63 with the weight
// d_r sc_rb (q - 32). Per row, token t and K32 group g the exact integer is
//   I_rtg = sum_{b in g} sc_rb (sum_16 q z - 32 S_tb),  S_tb = sum_16 z,
// and out[t][r] = sum_g d_r a_tg I_rtg. One MFMA gives, for 16 weight rows,
// 4 sub-block slots x 4 tokens: the A side holds activation rows
// (slot, token), nonzero only in their own slot's 16-code chunk, the B side
// the codes of (row, chunk). Chunk lk of MFMA p (p = 0..3 per super-block) is
// sub-block 4 lk + p, so each lane reads its row's 32 low-nibble bytes and
// 16 high-pair bytes of groups 2 lk, 2 lk + 1 with three 16-byte loads per
// super-block. The MFMA's C input is -32 S_tb (staged per token and sub-block
// in LDS), so D = sum (q - 32) z exactly (|D| <= 16 * 32 * 127). The low
// nibbles come in the 0x0240 order and the high pairs in bit pairs, so
// (d & 0x0f0f0f0f) | ((h << (4 - 2s)) & 0x30303030) rebuilds codes in
// natural K order and the activation operand is read straight from the Q8
// codes (16 bytes per lane). M > 4 runs two token passes over the same
// unpacked codes.
//
// Output lane (r = lane % 16, j = lane / 16) holds sub-block 4j + p for four
// tokens; MFMAs p and p + 1 are the two sub-blocks of one group, so
// X_t += a_tg * f32(sc0 D0_t + sc1 D1_t) (exact int32 below 2^24) per group,
// acc_t += d X_t per super-block, the four sub-block lanes of a row summed as
// ((j0 + j1) + (j2 + j3)), then the K-splitting waves of the block in
// ascending order: a fixed operation sequence per (row, token), so every M in
// 3..8 gives bitwise-identical rows for the same token.
#include <cstdlib>

#include "common.hpp"

namespace qw38hip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

template <int TP, int W, int PD, int Occ = 1>
__global__ __launch_bounds__(W * 64, Occ) void q6k_mfma_decode_kernel(
    const uint8_t* __restrict__ codes, const uint8_t* __restrict__ meta, uint32_t n, uint32_t pn,
    uint32_t kbs, const int8_t* __restrict__ xc, const float* __restrict__ xa, uint32_t m,
    uint32_t pk, float* __restrict__ out, const float* __restrict__ residual, uint32_t tiles) {
  constexpr int T = 4 * TP;  // tokens staged (zero past m)
  extern __shared__ __align__(16) uint8_t lds[];
  // -32 S per [sub-block][token] (int32), a per [group][token] (fp32), then
  // the wave partials [w][16][T]
  const uint32_t subs = pk / 16, groups = pk / 32;
  int32_t* s16 = reinterpret_cast<int32_t*>(lds);
  float* as = reinterpret_cast<float*>(s16 + subs * T);
  float* red = as + groups * T;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;

  for (uint32_t e = tid; e < subs * T; e += blockDim.x) {
    const uint32_t b = e / T, t = e % T;
    int v = 0;
    if (t < m) {
      const uint32_t* src = reinterpret_cast<const uint32_t*>(xc + size_t(t) * pk + b * 16);
#pragma unroll
      for (int i = 0; i < 4; ++i) v = dot4(src[i], 0x01010101u, v);
    }
    s16[e] = -32 * v;
  }
  for (uint32_t e = tid; e < groups * T; e += blockDim.x) {
    const uint32_t g = e / T, t = e % T;
    as[e] = t < m ? xa[size_t(t) * groups + g] : 0.f;
  }
  __syncthreads();

  const uint32_t r = lane & 15u, j = lane >> 4;
  const uint32_t ai = lane & 15u, a_slot = ai / 4, a_tok = ai % 4;  // A row (slot, token)
  const bool a_on = a_slot == j;
  const uint32_t kb_per = (kbs + W - 1) / W;
  const uint32_t kb0 = min(kbs, wave * kb_per), kb1 = min(kbs, kb0 + kb_per);
  const uint64_t tiles_total = uint64_t(pn) * kbs;

  for (uint32_t tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
    const uint32_t row = min(tile * 16 + r, pn - 1);  // rows past pn: clamped, never stored
    const uint64_t tr_base = uint64_t(row / 8) * kbs * 8 + row % 8;
    float acc[TP][4] = {};
    // Loads run PD super-blocks ahead of the arithmetic (a ring of PD + 1
    // register slots; past kb1 the ring re-reads the wave's last super-block).
    struct Slot {
      uint4 l0, l1, hh;
      uint4 za[TP][4];  // activation chunks of this lane's slot (zero off the diagonal)
      uint32_t scw;
      uint16_t dh;
    };
    Slot ring[PD + 1];
    auto fetch = [&](uint32_t kb, Slot& sl) {
      const uint64_t tr = tr_base + uint64_t(kb) * 8;
      // groups 2j and 2j+1 of the row: adjacent chunks in both planes
      const uint8_t* cp = codes + (tr - row % 8) * kQ6CodeBytes;
      const uint32_t c0 = q6_chunk(row % 8, 2 * j);
      sl.l0 = *reinterpret_cast<const uint4*>(cp + c0 * 16);
      sl.l1 = *reinterpret_cast<const uint4*>(cp + c0 * 16 + 16);
      sl.hh = *reinterpret_cast<const uint4*>(cp + kQ6HiPlane + c0 * 8);
      sl.scw = *reinterpret_cast<const uint32_t*>(meta + tr * 16 + 4 * j);
      sl.dh = *reinterpret_cast<const uint16_t*>(meta + tiles_total * 16 + tr * 2);
#pragma unroll
      for (int tp = 0; tp < TP; ++tp) {
        const uint32_t tok = tp * 4 + a_tok;
        if (a_on && tok < m) {  // off-diagonal lanes keep the zeros set once per tile
          const uint4* zp = reinterpret_cast<const uint4*>(xc + size_t(tok) * pk +
                                                           (size_t(kb) * 16 + 4 * j) * 16);
#pragma unroll
          for (int p = 0; p < 4; ++p) sl.za[tp][p] = zp[p];
        }
      }
    };
#pragma unroll
    for (int q = 0; q <= PD; ++q)
#pragma unroll
      for (int tp = 0; tp < TP; ++tp)
#pragma unroll
        for (int p = 0; p < 4; ++p) ring[q].za[tp][p] = make_uint4(0, 0, 0, 0);
    if (kb0 < kb1) {
#pragma unroll
      for (int q = 0; q < PD; ++q) fetch(min(kb0 + q, kb1 - 1), ring[q]);
    }
    for (uint32_t kc = kb0; kc < kb1; kc += PD + 1) {
#pragma unroll
    for (int q = 0; q <= PD; ++q) {
      if (kc + q >= kb1) break;
      const uint32_t kb = kc + q;
      fetch(min(kb + PD, kb1 - 1), ring[(q + PD) % (PD + 1)]);
      const Slot& cur = ring[q];
      const float d = f16_to_f32(cur.dh);
      const uint32_t scw = cur.scw;
      const uint32_t lo[8] = {cur.l0.x, cur.l0.y, cur.l0.z, cur.l0.w, cur.l1.x, cur.l1.y, cur.l1.z, cur.l1.w};
      const uint32_t hi[4] = {cur.hh.x, cur.hh.y, cur.hh.z, cur.hh.w};
      float X[TP][4];
      int I[TP][4];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const uint32_t d0 = lo[2 * p], d1 = lo[2 * p + 1], h = hi[p];
        v4i B;
        B[0] = int((d0 & 0x0f0f0f0fu) | ((h << 4) & 0x30303030u));
        B[1] = int(((d0 >> 4) & 0x0f0f0f0fu) | ((h << 2) & 0x30303030u));
        B[2] = int((d1 & 0x0f0f0f0fu) | (h & 0x30303030u));
        B[3] = int(((d1 >> 4) & 0x0f0f0f0fu) | ((h >> 2) & 0x30303030u));
        const uint32_t sb = kb * 16 + 4 * j + p;  // this lane's sub-block (operand and output)
        const int sc = int(int8_t((scw >> (8 * p)) & 0xffu));
        const uint32_t g = kb * 8 + 2 * j + p / 2;  // sub-blocks p, p ^ 1 share group g
#pragma unroll
        for (int tp = 0; tp < TP; ++tp) {
          const uint4 z = cur.za[tp][p];
          const v4i A = {int(z.x), int(z.y), int(z.z), int(z.w)};
          const int4 c4 = *reinterpret_cast<const int4*>(&s16[sb * T + tp * 4]);
          v4i C = {c4.x, c4.y, c4.z, c4.w};
          const v4i D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, C, 0, 0, 0);
          if (p % 2 == 0) {
#pragma unroll
            for (int v = 0; v < 4; ++v) I[tp][v] = __mul24(sc, D[v]);
          } else {  // the group's exact integer sc0 D0 + sc1 D1, then a_tg once
            const float4 a4 = *reinterpret_cast<const float4*>(&as[g * T + tp * 4]);
            const float av[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const float iv = float(__mul24(sc, D[v]) + I[tp][v]);
              X[tp][v] = p == 1 ? av[v] * iv : fmaf(av[v], iv, X[tp][v]);
            }
          }
        }
      }
#pragma unroll
      for (int tp = 0; tp < TP; ++tp)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[tp][v] = fmaf(d, X[tp][v], acc[tp][v]);
    }
    }
#pragma unroll
    for (int tp = 0; tp < TP; ++tp)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float c01 = acc[tp][v] + __shfl_xor(acc[tp][v], 16);
        acc[tp][v] = c01 + __shfl_xor(c01, 32);
      }
    if (j == 0) {
#pragma unroll
      for (int tp = 0; tp < TP; ++tp)
#pragma unroll
        for (int v = 0; v < 4; ++v) red[(wave * 16 + r) * T + tp * 4 + v] = acc[tp][v];
    }
    __syncthreads();
    for (uint32_t e = tid; e < 16 * T; e += blockDim.x) {
      const uint32_t rr = e % 16, t = e / 16;
      const uint32_t orow = tile * 16 + rr;
      float y = red[rr * T + t];
#pragma unroll
      for (int w = 1; w < W; ++w) y += red[(w * 16 + rr) * T + t];
      if (t < m && orow < n) {
        const size_t o = size_t(t) * n + orow;
        out[o] = residual ? y + residual[o] : y;
      }
    }
    __syncthreads();
  }
}

template <int TP, int W, int PD, int Occ = 1>
hipError_t launch_t(const WeightView& w, const Q8View& x, float* out, const float* residual,
                    hipStream_t s, uint32_t per_cu_cap) {
  constexpr int T = 4 * TP;
  const uint32_t kbs = w.pk / 256, tiles = (w.pn + 15) / 16;
  const size_t lds = size_t(w.pk / 16) * T * 4 + size_t(w.pk / 32) * T * 4 + size_t(W) * 16 * T * 4;
  if (lds > 160 * 1024) return hipErrorNotSupported;
  uint32_t per_cu = std::max<uint32_t>(1, std::min<uint32_t>(uint32_t(160 * 1024 / lds), 32u / W));
  // Fewer tiles than two per CU: one block per CU, looping over its tiles.
  // Every block stages the whole activation operand in LDS first, and a
  // second block on a CU only pays for that with a full round of its own
  // (5120 rows = 320 tiles: M=3 26.1 -> 25.2 us, M=4 26.9 -> 25.8, M=8
  // 36.3 -> 34.6).
  if (tiles < 2 * uint32_t(cu_count())) per_cu = 1;
  if (per_cu_cap) per_cu = std::min(per_cu, per_cu_cap);
  const uint32_t grid = std::min<uint32_t>(tiles, uint32_t(cu_count()) * per_cu);
  auto kern = q6k_mfma_decode_kernel<TP, W, PD, Occ>;
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3(grid), dim3(W * 64), lds, s, w.codes, w.scales, w.n, w.pn, kbs,
                     x.codes, x.scales, x.m, x.pk, out, residual, tiles);
  return hipGetLastError();
}

}  // namespace

// Q6_K 0x0241 at M = 3..8 with 16-byte aligned code spans and Q8 codes;
// hipErrorNotSupported otherwise (the caller falls back to the dot4 kernels).
hipError_t launch_q6k_mfma_decode(const WeightView& w, const Q8View& x, float* out,
                                  const float* residual, hipStream_t s) {
  static const int env = [] {
    const char* e = std::getenv("QW38_DECODE_MFMA");
    return e ? std::atoi(e) : 1;
  }();
  static const uint32_t cap = [] {  // tuning aid: blocks per CU
    const char* e = std::getenv("QW38_DECODE_MFMA_BLOCKS");
    return e ? uint32_t(std::atoi(e)) : 0u;
  }();
  if (!env || w.layout != QW38_LAYOUT_Q6K_WAVE64 || x.m > 8 || x.m < (env >= 2 ? 1u : 3u))
    return hipErrorNotSupported;
  if ((reinterpret_cast<uintptr_t>(w.codes) | reinterpret_cast<uintptr_t>(x.codes)) % 16 ||
      reinterpret_cast<uintptr_t>(w.scales) % 4)
    return hipErrorNotSupported;
  // M 5..8 (two token passes): no load ring, bounded to four waves per SIMD
  // (112 VGPRs); with the ring it needs 186 VGPRs (config 3, M=8, both at
  // 320 blocks: 38.2 against 43.1 us). M 3..4 keeps the ring (118 VGPRs
  // either way).
  return x.m <= 4 ? launch_t<1, 8, 1>(w, x, out, residual, s, cap)
                  : launch_t<2, 8, 0, 4>(w, x, out, residual, s, cap);
}

}  // namespace qw38hip
