// Batched decode GEMV (M = 2..8 tokens) for Q4_K 0x020D on the int8 matrix
// cores: v_mfma_i32_16x16x64_i8 with a block-diagonal activation operand.
//
// The reference (cuda/q4k_q8.cu:103-158, mmq at 1 < M < 128) contracts
//   out[t][r] = sum_g a_tg * (d_r s_rg dot_rtg - dmin_r m_rg sum_tg)
// with an exact int32 K32 dot per (row, token, group). Here one MFMA computes
// those exact dots for 16 weight rows x 16 "slots": the MFMA's A side is the
// activations, one A row per (group slot gs, token t) = gs*T + t, and its 64-K
// operand is 4 lane chunks of 16 codes. A chunk belongs to one group slot; an A
// row is nonzero only in the chunks of its own slot (the block-diagonal), so
// output (slot, t, r) is the dot of token t with row r over exactly that
// slot's codes:
//   T = 8 (M 5..8): 2 slots x 8 tokens; MFMA p of a super-block covers groups
//          2p, 2p+1, each slot spanning 2 chunks (the two 16-code halves);
//   T = 4 (M 2..4): 4 slots x 4 tokens; two chained MFMAs (half 0, half 1)
//          cover groups 4q..4q+3, one chunk per slot per MFMA.
// Every partial sum is an integer (|dot| <= 32*15*127), so the int32 result is
// the reference's dot exactly. The B side is the weight rows: lane (r, lk)
// supplies 16 codes (8 bytes of 0x020D sequential nibbles, unpacked with one
// AND and one shift+AND per dword) of row r for chunk lk. The unpack leaves
// codes in the order 0,2,4,6,1,3,5,7,8,10,...; the activation operand is
// staged once per block in LDS in that same order, so the dot is unchanged.
//
// Output lane (r = lane % 16, j = lane / 16) holds slot 4j/T and four tokens,
// so the row's 6-bit scale/min of that slot's group are lane-uniform values:
//   X_t += a_tg * f32(s_g * D_t)  (v_mul_u32_u24, cvt, fma)
//   Y_t += m_g * (a_tg sum_tg)     (one fma; a*sum staged per token and group)
// and per super-block acc_t += d X_t - dmin Y_t, the reassociated expression
// of the reference that the other decode kernels use. A block of four waves
// owns 16-row tiles of the persistent grid; the waves split K and their
// partials are summed in LDS in a fixed order (bitwise deterministic).
#include <cstdlib>

#include "common.hpp"

namespace qw38hip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));


// Code chunk (16 codes, index within the super-block: 0..15) that operand
// chunk lk of MFMA p reads, and the group slot it belongs to.
template <int T>
__device__ __forceinline__ uint32_t chunk_of(uint32_t p, uint32_t lk) {
  if constexpr (T == 8) return 4 * p + lk;                      // group 2p + lk/2, half lk%2
  else return 8 * (p / 2) + 2 * lk + (p % 2);                   // group 4(p/2) + lk, half p%2
}
template <int T>
__device__ __forceinline__ uint32_t slot_of(uint32_t lk) {
  return T == 8 ? lk / 2 : lk;
}

// 8 bytes of sequential nibbles -> 16 int8 codes in the order
// 0,2,4,6 | 1,3,5,7 | 8,10,12,14 | 9,11,13,15.
__device__ __forceinline__ v4i unpack8(uint32_t w0, uint32_t w1) {
  v4i b;
  b[0] = int(w0 & 0x0f0f0f0fu);
  b[1] = int((w0 >> 4) & 0x0f0f0f0fu);
  b[2] = int(w1 & 0x0f0f0f0fu);
  b[3] = int((w1 >> 4) & 0x0f0f0f0fu);
  return b;
}

template <int T, int kWaves>
__global__ __launch_bounds__(kWaves * 64) void q4k_mfma_decode_kernel(
    const uint8_t* __restrict__ codes, const uint8_t* __restrict__ meta, uint32_t n, uint32_t pn,
    uint32_t kbs, const int8_t* __restrict__ xc, const float* __restrict__ xa,
    const int32_t* __restrict__ xs, uint32_t m, uint32_t pk, float* __restrict__ out,
    const float* __restrict__ residual, uint32_t tiles) {
  extern __shared__ __align__(16) uint8_t lds[];
  // [chunk][t] 16-byte operand rows (pk/16 chunks), then a zero row, then
  // a [g][t] and u = a*sum [g][t] (fp32), then the wave partials
  // [slot][w][16][T] of up to six tiles.
  const uint32_t chunks = pk / 16, groups = pk / 32;
  uint4* zs = reinterpret_cast<uint4*>(lds);
  uint4* zero = zs + chunks * T;
  float* as = reinterpret_cast<float*>(zero + 1);
  float* us = as + groups * T;
  float* red = us + groups * T;

  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;

  // ---- stage the activations once per block ----
  // Loads are unconditional (clamped token) with a select after: a
  // conditional load becomes a branch with its own wait.
  for (uint32_t e = tid; e < chunks * T; e += blockDim.x) {
    const uint32_t c = e / T, t = e % T;
    const uint32_t* src = reinterpret_cast<const uint32_t*>(xc + size_t(min(t, m - 1)) * pk + c * 16);
    const uint32_t z0 = src[0], z1 = src[1], z2 = src[2], z3 = src[3];
    uint4 v;
    v.x = perm(z1, z0, 0x06040200u);
    v.y = perm(z1, z0, 0x07050301u);
    v.z = perm(z3, z2, 0x06040200u);
    v.w = perm(z3, z2, 0x07050301u);
    zs[e] = t < m ? v : make_uint4(0, 0, 0, 0);
  }
  if (tid == 0) *zero = make_uint4(0, 0, 0, 0);
  for (uint32_t e = tid; e < groups * T; e += blockDim.x) {
    const uint32_t g = e / T, t = e % T;
    const size_t gi = size_t(min(t, m - 1)) * groups + g;
    const float a = xa[gi];
    const float u = a * float(xs[gi]);
    as[e] = t < m ? a : 0.f;
    us[e] = t < m ? u : 0.f;
  }
  __syncthreads();

  const uint32_t r = lane & 15u, j = lane >> 4;
  // operand side: A row i = lane % 16 = (slot i / T, token i % T); chunk lk = j
  const uint32_t ai = lane & 15u, a_slot = ai / T, a_tok = ai % T;
  // output side: rows 4j..4j+3 = slot (4j)/T, tokens t0..t0+3
  const uint32_t o_slot = (4 * j) / T, t0 = (4 * j) % T;
  const uint32_t kb_per = (kbs + kWaves - 1) / kWaves;
  const uint32_t kb0 = min(kbs, wave * kb_per), kb1 = min(kbs, kb0 + kb_per);

  // Partials per group class c = g % 4 (groups c and c + 4 of a super-block,
  // in that order), summed at the end as ((c0 + c1) + (c2 + c3)): the same
  // operation sequence for T = 4 and T = 8, so every M in 3..8 gives
  // bitwise-identical rows for the same token. A T = 8 lane of slot gs owns
  // classes gs and gs + 2, a T = 4 lane of slot j class j.
  constexpr int NX = T == 8 ? 2 : 1;
  // The block's tiles (blockIdx.x + i gridDim.x) and the wave's K range form
  // one stream of (tile, super-block) items; the next item's five loads are
  // issued before the current one's arithmetic, across tile boundaries, so a
  // wave never waits a full memory latency at the start of a tile. Each
  // tile's row partial goes to an LDS slot; every kRing tiles (and at the
  // end) the block sums the waves' partials of those tiles in wave order.
  constexpr uint32_t kRing = 48 / kWaves;
  const uint32_t nkb = kb1 - kb0;
  const uint32_t ntl = blockIdx.x < tiles ? (tiles - blockIdx.x + gridDim.x - 1) / gridDim.x : 0u;
  struct Item {
    uint4 mw;
    uint2 wq[4];
  };
  auto load = [&](uint32_t ti, uint32_t kb, Item& L) __attribute__((always_inline)) {
    const uint32_t row = min((blockIdx.x + ti * gridDim.x) * 16 + r, pn - 1);  // clamped, never stored
    const uint64_t tr = uint64_t(row / 8) * kbs * 8 + row % 8 + uint64_t(kb) * 8;
    L.mw = *reinterpret_cast<const uint4*>(meta + tr * 16);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      L.wq[i] = *reinterpret_cast<const uint2*>(codes + tr * 128 + chunk_of<T>(i, j) * 8);
  };
  // Sums the wave partials of tiles [t_lo, t_hi) of this block (slots ti % kRing).
  auto flush = [&](uint32_t t_lo, uint32_t t_hi) __attribute__((always_inline)) {
    __syncthreads();
    const uint32_t cnt = t_hi - t_lo;
    for (uint32_t e = tid; e < cnt * 16 * T; e += blockDim.x) {
      const uint32_t ti = t_lo + e / (16 * T), rem = e % (16 * T);
      const uint32_t rr = rem % 16, t = rem / 16, slot = ti % kRing;
      const uint32_t orow = (blockIdx.x + ti * gridDim.x) * 16 + rr;
      float y = red[((slot * kWaves + 0) * 16 + rr) * T + t];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) y += red[((slot * kWaves + w) * 16 + rr) * T + t];
      if (t < m && orow < n) {
        const size_t o = size_t(t) * n + orow;
        out[o] = residual ? y + residual[o] : y;
      }
    }
    __syncthreads();
  };
  // Writes this wave's partial of tile ti (zeros for a wave without K range).
  auto park = [&](uint32_t ti, const float (&acc)[NX][4]) __attribute__((always_inline)) {
    float tot[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      if constexpr (T == 8) {  // lanes j, j + 2 hold classes (0, 2) and (1, 3)
        const float c01 = acc[0][v] + __shfl_xor(acc[0][v], 32);
        const float c23 = acc[1][v] + __shfl_xor(acc[1][v], 32);
        tot[v] = c01 + c23;
      } else {  // lane j holds class j
        const float c01 = acc[0][v] + __shfl_xor(acc[0][v], 16);
        tot[v] = c01 + __shfl_xor(c01, 32);
      }
    }
    if (j < (T == 8 ? 2u : 1u)) {
#pragma unroll
      for (int v = 0; v < 4; ++v) red[(((ti % kRing) * kWaves + wave) * 16 + r) * T + t0 + v] = tot[v];
    }
  };

  float acc[NX][4] = {};
  Item cur, nxt;
  if (nkb && ntl) load(0, kb0, cur);
  uint32_t t_done = 0;  // tiles already summed
  for (uint32_t ti = 0; ti < ntl; ++ti) {
    for (uint32_t kq = 0; kq < nkb; ++kq) {
      const uint32_t kb = kb0 + kq;
      // T = 8: the next item (the following super-block, or the next tile's
      // first) is loaded now. T = 4 loads each item right before its use:
      // a second item in registers would leave fewer than four eight-wave
      // blocks per CU (72 VGPRs; M = 2 / 4 took 25.8 / 26.8 against 21 /
      // 22.5 us), and its four blocks per CU keep enough loads in flight.
      if constexpr (T == 8) {
        if (kq + 1 < nkb) load(ti, kb + 1, nxt);
        else if (ti + 1 < ntl) load(ti + 1, kb0, nxt);
      } else if (kq > 0 || ti > 0) {
        load(ti, kb, cur);
      }
      const uint4 mw = cur.mw;
      float X[NX][4], Y[NX][4];
      constexpr int P = T == 8 ? 4 : 2;  // epilogues per super-block
#pragma unroll
      for (int p = 0; p < P; ++p) {
        v4i D = {0, 0, 0, 0};
        constexpr int CH = T == 8 ? 1 : 2;  // chained MFMAs per epilogue
#pragma unroll
        for (int h = 0; h < CH; ++h) {
          const uint32_t mp = uint32_t(p * CH + h);
          const uint32_t c = chunk_of<T>(mp, j);
          const v4i B = unpack8(cur.wq[mp].x, cur.wq[mp].y);
          const bool on = slot_of<T>(j) == a_slot;
          const uint4 av = on ? zs[(kb * 16 + c) * T + a_tok] : *zero;
          const v4i A = {int(av.x), int(av.y), int(av.z), int(av.w)};
          D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, D, 0, 0, 0);
        }
        const uint32_t g = T == 8 ? 2 * p + o_slot : 4 * p + o_slot;  // group in the super-block
        constexpr bool kFirst[4] = {true, T == 8, false, false};
        const int xi = p % NX;
        uint32_t s, mn;
        q4k_scale_min(mw.y, mw.z, mw.w, g, s, mn);
        const float mf = float(mn);
        const float4 a4 = *reinterpret_cast<const float4*>(&as[(kb * 8 + g) * T + t0]);
        const float4 u4 = *reinterpret_cast<const float4*>(&us[(kb * 8 + g) * T + t0]);
        const float av4[4] = {a4.x, a4.y, a4.z, a4.w}, uv4[4] = {u4.x, u4.y, u4.z, u4.w};
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float sd = float(__mul24(int(s), D[v]));
          if (kFirst[p]) {
            X[xi][v] = av4[v] * sd;
            Y[xi][v] = mf * uv4[v];
          } else {
            X[xi][v] = fmaf(av4[v], sd, X[xi][v]);
            Y[xi][v] = fmaf(mf, uv4[v], Y[xi][v]);
          }
        }
      }
      const float d = f16_to_f32(mw.x & 0xffffu), dmin = f16_to_f32(mw.x >> 16);
#pragma unroll
      for (int c = 0; c < NX; ++c)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[c][v] = fmaf(-dmin, Y[c][v], fmaf(d, X[c][v], acc[c][v]));
      if constexpr (T == 8) cur = nxt;
    }
    park(ti, acc);
#pragma unroll
    for (int c = 0; c < NX; ++c)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[c][v] = 0.f;
    if (ti + 1 - t_done == kRing) {
      flush(t_done, ti + 1);
      t_done = ti + 1;
    }
  }
  if (t_done < ntl) flush(t_done, ntl);
}

template <int T, int W>
hipError_t launch_t(const WeightView& w, const Q8View& x, float* out, const float* residual,
                    hipStream_t s, uint32_t per_cu_cap) {
  const uint32_t kbs = w.pk / 256, tiles = (w.pn + 15) / 16;
  const size_t lds = size_t(w.pk / 16) * T * 16 + 16 + size_t(w.pk / 32) * T * 8 +
                     size_t(48 / W) * W * 16 * T * 4;  // partial slots of 48 / W tiles
  if (lds > 160 * 1024) return hipErrorNotSupported;
  uint32_t per_cu = uint32_t(160 * 1024 / lds);
  per_cu = std::max(1u, std::min(per_cu, 32u / W));
  if (per_cu_cap) per_cu = std::min(per_cu, per_cu_cap);
  const uint32_t grid = std::min<uint32_t>(tiles, uint32_t(cu_count()) * per_cu);
  auto kern = q4k_mfma_decode_kernel<T, W>;
  if (lds > 64 * 1024) {
    const hipError_t e = set_max_lds(reinterpret_cast<const void*>(kern), int(lds));
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3(grid), dim3(W * 64), lds, s, w.codes, w.scales, w.n, w.pn,
                     kbs, x.codes, x.scales, x.sums, x.m, x.pk, out, residual, tiles);
  return hipGetLastError();
}

}  // namespace

// M = 2..8 on Q4_K 0x020D with 16-byte aligned code and metadata spans and
// 4-byte aligned Q8 codes; hipErrorNotSupported otherwise (the caller falls
// back to the dot4 kernels).
hipError_t launch_q4k_mfma_decode(const WeightView& w, const Q8View& x, float* out,
                                  const float* residual, hipStream_t s) {
  static const int env = [] {
    const char* e = std::getenv("QW38_DECODE_MFMA");
    return e ? std::atoi(e) : 1;
  }();
  if (!env || w.layout != QW38_LAYOUT_Q4K_CANDIDATE_V2 || x.m > 8 || x.m < (env >= 2 ? 1u : 2u))
    return hipErrorNotSupported;
  if ((reinterpret_cast<uintptr_t>(w.codes) | reinterpret_cast<uintptr_t>(w.scales)) % 16 ||
      reinterpret_cast<uintptr_t>(x.codes) % 4)
    return hipErrorNotSupported;
  static const uint32_t cap = [] {  // tuning aid: blocks per CU
    const char* e = std::getenv("QW38_DECODE_MFMA_BLOCKS");
    return e ? uint32_t(std::atoi(e)) : 0u;
  }();
  if (x.m <= 4) return launch_t<4, 8>(w, x, out, residual, s, cap);
  return launch_t<8, 8>(w, x, out, residual, s, cap);
}

}  // namespace qw38hip
