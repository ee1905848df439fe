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
// acc_t += d X_t per super-block, and the four sub-block lanes of a row are
// summed as ((j0 + j1) + (j2 + j3)).
//
// Work split. K is cut into the fixed Q6_K segments (q6_seg_kb: four at
// K = 17408, a function of K alone) and each segment into two halves; one
// wave streams one (16-row tile, segment, half) with its loads PD super-
// blocks ahead. A segment's partial is half 0 + half 1, and a row's result is
// the segment partials added in ascending order (+ residual): a fixed
// operation sequence per (row, token), so every M in 3..8 and both launch
// modes give bitwise-identical rows for the same token.
//   Spread mode (the library scratch is available): a block of 2 IPB waves
//   takes IPB consecutive (tile, segment) items, so every CU gets the same
//   number of items (5120 rows x K 17408: 320 tiles x 4 segments = 1280
//   items = 5 per CU, where whole tiles give 64 CUs two and the others one).
//   Segment partials go to the library scratch and a second small kernel
//   adds them in order. (A last-arriving-block sum with device-scope fences
//   was 4x slower: the acquire fence invalidates the whole L2 of the XCD,
//   which the other blocks' activation reads then miss.)
//   Own mode (no scratch): a block takes whole tiles and adds the partials in
//   LDS.
#include <cstdlib>

#include "common.hpp"

namespace qw38hip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kIPB = 5;            // items per block (spread mode)
constexpr int kW = 2 * kIPB;       // waves per block: two halves per item

// Weight bytes of one (row, super-block) for lane (r, j): low nibbles and high
// pairs of groups 2j, 2j + 1, the four sub-block scales 4j..4j+3 and d.
struct Q6Slot {
  uint4 l0, l1, hh;
  uint32_t scw;
  uint16_t dh;
};

__device__ __forceinline__ void q6_fetch(const uint8_t* __restrict__ codes, const uint8_t* __restrict__ meta,
                                         uint64_t tiles_total, uint32_t row, uint64_t tr, uint32_t j,
                                         Q6Slot& sl) {
  const uint8_t* cp = codes + (tr - row % 8) * kQ6CodeBytes;  // the 8-row tile
  const uint32_t c0 = q6_chunk(row % 8, 2 * j);                // adjacent chunks in both planes
  sl.l0 = *reinterpret_cast<const uint4*>(cp + c0 * 16);
  sl.l1 = *reinterpret_cast<const uint4*>(cp + c0 * 16 + 16);
  sl.hh = *reinterpret_cast<const uint4*>(cp + kQ6HiPlane + c0 * 8);
  sl.scw = *reinterpret_cast<const uint32_t*>(meta + tr * 16 + 4 * j);
  sl.dh = *reinterpret_cast<const uint16_t*>(meta + tiles_total * 16 + tr * 2);
}

// One super-block of one lane: acc_t += d X_t with X_t = sum_g a_tg (sc0 D0 +
// sc1 D1). za[tp][p]: the lane's activation chunk (sub-block 4j + p) for
// token pass tp (zero off the diagonal); s16p / asp: -32 S and a of the
// super-block, [sub-block][T] and [group][T]. Shared by both launch modes,
// so their per-(row, token) operation sequences are the same.
template <int TP>
__device__ __forceinline__ void q6_superblock(const Q6Slot& cur, const uint4 (&za)[TP][4],
                                              const int32_t* s16p, const float* asp, uint32_t j,
                                              float (&acc)[TP][4]) {
  constexpr int T = 4 * TP;
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
    const uint32_t sb = 4 * j + p;  // this lane's sub-block (operand and output)
    const int sc = int(int8_t((scw >> (8 * p)) & 0xffu));
    const uint32_t g = 2 * j + p / 2;  // sub-blocks p, p ^ 1 share group g
#pragma unroll
    for (int tp = 0; tp < TP; ++tp) {
      const uint4 z = za[tp][p];
      const v4i A = {int(z.x), int(z.y), int(z.z), int(z.w)};
      const int4 c4 = *reinterpret_cast<const int4*>(&s16p[sb * T + tp * 4]);
      v4i C = {c4.x, c4.y, c4.z, c4.w};
      const v4i D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, C, 0, 0, 0);
      if (p % 2 == 0) {
#pragma unroll
        for (int v = 0; v < 4; ++v) I[tp][v] = __mul24(sc, D[v]);
      } else {  // the group's exact integer sc0 D0 + sc1 D1, then a_tg once
        const float4 a4 = *reinterpret_cast<const float4*>(&asp[g * T + tp * 4]);
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

// The row's sub-block lanes summed as ((j0 + j1) + (j2 + j3)) and parked in
// red[slot][half] by the j = 0 lanes.
template <int TP>
__device__ __forceinline__ void q6_park(float (&acc)[TP][4], float* red, uint32_t slot, uint32_t half,
                                        uint32_t r, uint32_t j) {
  constexpr int T = 4 * TP;
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
      for (int v = 0; v < 4; ++v) red[((slot * 2 + half) * 16 + r) * T + tp * 4 + v] = acc[tp][v];
  }
}

// The K range of half `half` of segment `seg`.
__device__ __forceinline__ void q6_half_range(uint32_t kbs, uint32_t seg_kb, uint32_t seg, uint32_t half,
                                              uint32_t& kb0, uint32_t& kb1) {
  const uint32_t k0 = seg * seg_kb, k1 = min(kbs, k0 + seg_kb), hk = (k1 - k0 + 1) / 2;
  kb0 = half ? k0 + hk : k0;
  kb1 = half ? k1 : k0 + hk;
}

// Own mode: a block takes whole tiles (waves 2s, 2s + 1 take segment s) and
// adds the partials in LDS; the activation chunks are read from global memory
// (L2) with the weights, PD super-blocks ahead.
template <int TP, int PD>
__global__ __launch_bounds__(kW * 64) void q6k_decode_own_kernel(
    const uint8_t* __restrict__ codes, const uint8_t* __restrict__ meta, uint32_t n, uint32_t pn,
    uint32_t kbs, const int8_t* __restrict__ xc, const float* __restrict__ xa, uint32_t m,
    uint32_t pk, float* __restrict__ out, const float* __restrict__ residual, uint32_t tiles) {
  constexpr int T = 4 * TP;  // tokens staged (zero past m)
  extern __shared__ __align__(16) uint8_t lds[];
  // -32 S per [sub-block][token] (int32), a per [group][token] (fp32), then
  // the half partials [segment][half][16][T]
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
  const uint32_t a_tok = lane % 4;
  const bool a_on = (lane & 15u) / 4 == j;  // A row (slot, token) = (lane % 16) / 4, lane % 4
  const uint64_t tiles_total = uint64_t(pn) * kbs;
  const uint32_t seg_kb = q6_seg_kb(kbs), segs = (kbs + seg_kb - 1) / seg_kb;
  const uint32_t slot = wave / 2, half = wave % 2;
  for (uint32_t tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
    if (slot < segs) {
      uint32_t kb0, kb1;
      q6_half_range(kbs, seg_kb, slot, half, kb0, kb1);
      const uint32_t row = min(tile * 16 + r, pn - 1);  // rows past pn: clamped, never stored
      const uint64_t tr_base = uint64_t(row / 8) * kbs * 8 + row % 8;
      float acc[TP][4] = {};
      struct Slot {
        Q6Slot w;
        uint4 za[TP][4];
      };
      Slot ring[PD + 1];
      auto fetch = [&](uint32_t kb, Slot& sl) __attribute__((always_inline)) {
        q6_fetch(codes, meta, tiles_total, row, tr_base + uint64_t(kb) * 8, j, sl.w);
#pragma unroll
        for (int tp = 0; tp < TP; ++tp) {
          const uint32_t tok = tp * 4 + a_tok;
          if (a_on && tok < m) {  // off-diagonal lanes keep their zeros
            const uint4* zp = reinterpret_cast<const uint4*>(xc + size_t(tok) * pk + (size_t(kb) * 16 + 4 * j) * 16);
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
          q6_superblock<TP>(ring[q].w, ring[q].za, s16 + kb * 16 * T, as + kb * 8 * T, j, acc);
        }
      }
      q6_park<TP>(acc, red, slot, half, r, j);
    }
    __syncthreads();
    for (uint32_t e = tid; e < 16 * T; e += blockDim.x) {
      const uint32_t rr = e % 16, t = e / 16;
      float y = red[(0 * 16 + rr) * T + t] + red[(1 * 16 + rr) * T + t];
      for (uint32_t sg = 1; sg < segs; ++sg)
        y = y + (red[((sg * 2) * 16 + rr) * T + t] + red[((sg * 2 + 1) * 16 + rr) * T + t]);
      const uint32_t orow = tile * 16 + rr;
      if (t < m && orow < n) {
        const size_t o = size_t(t) * n + orow;
        out[o] = residual ? y + residual[o] : y;
      }
    }
    __syncthreads();
  }
}

// Spread mode: items in segment-major order (it = segment * tiles + tile),
// kIPB consecutive items per block, so a block's items lie in at most two
// segments whose activations it stages in LDS: the codes as the MFMA's A
// chunks [super-block][chunk][token], -32 S and a per segment. The weight
// loads of the first PD super-blocks are issued before that staging. The
// (tile, segment) partials go to `part` ([tile][segment][16][T]) for
// q6k_seg_sum_kernel.
template <int TP, int PD>
__global__ __launch_bounds__(kW * 64) void q6k_decode_spread_kernel(
    const uint8_t* __restrict__ codes, const uint8_t* __restrict__ meta, uint32_t pn, uint32_t kbs,
    const int8_t* __restrict__ xc, const float* __restrict__ xa, uint32_t m, uint32_t pk, uint32_t tiles,
    float* __restrict__ part) {
  constexpr int T = 4 * TP;
  extern __shared__ __align__(16) uint8_t lds[];
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t r = lane & 15u, j = lane >> 4;
  const uint32_t a_tok = lane % 4;
  const bool a_on = (lane & 15u) / 4 == j;
  const uint64_t tiles_total = uint64_t(pn) * kbs;
  const uint32_t seg_kb = q6_seg_kb(kbs), segs = (kbs + seg_kb - 1) / seg_kb;
  const uint32_t items = tiles * segs;
  const uint32_t slot = wave / 2, half = wave % 2;
  const uint32_t it0 = blockIdx.x * kIPB, seg_lo = it0 / tiles;
  // LDS per staged segment: A chunks (seg_kb * 16 * T uint4), -32 S
  // (seg_kb * 16 * T int32), a (seg_kb * 8 * T fp32); two segments, then red.
  const uint32_t seg_bytes = seg_kb * 16 * T * 16 + seg_kb * 16 * T * 4 + seg_kb * 8 * T * 4;
  float* red = reinterpret_cast<float*>(lds + 2 * seg_bytes);

  const uint32_t it = it0 + slot;
  const bool live = it < items;
  const uint32_t seg = live ? it / tiles : seg_lo, tile = live ? it % tiles : 0u;
  uint32_t kb0 = 0, kb1 = 0;
  if (live) q6_half_range(kbs, seg_kb, seg, half, kb0, kb1);
  const uint32_t row = min(tile * 16 + r, pn - 1);  // rows past pn: clamped, never stored
  const uint64_t tr_base = uint64_t(row / 8) * kbs * 8 + row % 8;
  Q6Slot ring[PD + 1];
  if (kb0 < kb1) {
#pragma unroll
    for (int q = 0; q < PD; ++q) q6_fetch(codes, meta, tiles_total, row, tr_base + uint64_t(min(kb0 + q, kb1 - 1)) * 8, j, ring[q]);
  }

  // stage segments seg_lo and seg_lo + 1 (the second only if some item needs it)
  const uint32_t seg_hi = min(it0 + kIPB, items) - 1;
  const uint32_t nseg = (seg_hi / tiles) > seg_lo ? 2u : 1u;
  for (uint32_t q = 0; q < nseg; ++q) {
    const uint32_t sg = seg_lo + q;
    uint8_t* base = lds + q * seg_bytes;
    uint4* zs = reinterpret_cast<uint4*>(base);
    int32_t* s16 = reinterpret_cast<int32_t*>(base + seg_kb * 16 * T * 16);
    float* as = reinterpret_cast<float*>(base + seg_kb * 16 * T * 16 + seg_kb * 16 * T * 4);
    const uint32_t kbase = sg * seg_kb, nkb = min(kbs, kbase + seg_kb) - kbase;
    for (uint32_t e = tid; e < nkb * 16 * T; e += blockDim.x) {
      const uint32_t c = e / T, t = e % T;  // chunk (sub-block) of the segment, token
      uint4 v = make_uint4(0, 0, 0, 0);
      if (t < m) v = *reinterpret_cast<const uint4*>(xc + size_t(t) * pk + (size_t(kbase) * 16 + c) * 16);
      zs[e] = v;
      int sm = 0;
      sm = dot4(v.x, 0x01010101u, sm);
      sm = dot4(v.y, 0x01010101u, sm);
      sm = dot4(v.z, 0x01010101u, sm);
      sm = dot4(v.w, 0x01010101u, sm);
      s16[e] = -32 * sm;
    }
    for (uint32_t e = tid; e < nkb * 8 * T; e += blockDim.x) {
      const uint32_t g = e / T, t = e % T;
      as[e] = t < m ? xa[size_t(t) * (pk / 32) + kbase * 8 + g] : 0.f;
    }
  }
  __syncthreads();

  if (live) {
    const uint32_t q = seg - seg_lo;
    const uint8_t* base = lds + q * seg_bytes;
    const uint4* zs = reinterpret_cast<const uint4*>(base);
    const int32_t* s16 = reinterpret_cast<const int32_t*>(base + seg_kb * 16 * T * 16);
    const float* as = reinterpret_cast<const float*>(base + seg_kb * 16 * T * 16 + seg_kb * 16 * T * 4);
    const uint32_t kbase = seg * seg_kb;
    float acc[TP][4] = {};
    for (uint32_t kc = kb0; kc < kb1; kc += PD + 1) {
#pragma unroll
      for (int u = 0; u <= PD; ++u) {
        if (kc + u >= kb1) break;
        const uint32_t kb = kc + u;
        q6_fetch(codes, meta, tiles_total, row, tr_base + uint64_t(min(kb + PD, kb1 - 1)) * 8, j,
                 ring[(u + PD) % (PD + 1)]);
        const uint32_t lkb = kb - kbase;
        uint4 za[TP][4];
#pragma unroll
        for (int tp = 0; tp < TP; ++tp)
#pragma unroll
          for (int p = 0; p < 4; ++p)
            za[tp][p] = a_on ? zs[(lkb * 16 + 4 * j + p) * T + tp * 4 + a_tok] : make_uint4(0, 0, 0, 0);
        q6_superblock<TP>(ring[u], za, s16 + lkb * 16 * T, as + lkb * 8 * T, j, acc);
      }
    }
    q6_park<TP>(acc, red, slot, half, r, j);
  }
  __syncthreads();
  for (uint32_t e = tid; e < kIPB * 16 * T; e += blockDim.x) {
    const uint32_t sl = e / (16 * T), rem = e % (16 * T), i2 = it0 + sl;
    if (i2 >= items) continue;
    const uint32_t sg = i2 / tiles, tl = i2 % tiles;
    part[(size_t(tl) * segs + sg) * 16 * T + rem] = red[((sl * 2) * 16) * T + rem] + red[((sl * 2 + 1) * 16) * T + rem];
  }
}

// Spread mode's second step: row results as the segment partials added in
// ascending order (+ residual), the own mode's operation sequence.
template <int T>
__global__ __launch_bounds__(256) void q6k_seg_sum_kernel(const float* __restrict__ part, uint32_t segs,
                                                          uint32_t tiles, uint32_t n, uint32_t m,
                                                          float* __restrict__ out,
                                                          const float* __restrict__ residual) {
  const uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= tiles * 16 * T) return;
  const uint32_t tile = e / (16 * T), rem = e % (16 * T), rr = rem / T, t = rem % T;
  const uint32_t orow = tile * 16 + rr;
  if (t >= m || orow >= n) return;
  const float* pp = part + size_t(tile) * segs * 16 * T + rem;
  float y = pp[0];
  for (uint32_t sg = 1; sg < segs; ++sg) y = y + pp[sg * 16 * T];
  const size_t o = size_t(t) * n + orow;
  out[o] = residual ? y + residual[o] : y;
}

template <int TP, int PDO, int PDS>
hipError_t launch_t(const WeightView& w, const Q8View& x, float* out, const float* residual,
                    hipStream_t s, bool own) {
  constexpr int T = 4 * TP;
  const uint32_t kbs = w.pk / 256, tiles = (w.pn + 15) / 16;
  const uint32_t seg_kb = q6_seg_kb(kbs), segs = (kbs + seg_kb - 1) / seg_kb;
  const size_t red_bytes = size_t(kIPB) * 2 * 16 * T * 4;
  const size_t lds_own = size_t(w.pk / 16) * T * 4 + size_t(w.pk / 32) * T * 4 + red_bytes;
  const size_t lds_spread = 2 * (size_t(seg_kb) * 16 * T * 20 + size_t(seg_kb) * 8 * T * 4) + red_bytes;
  const uint64_t items = uint64_t(tiles) * segs;
  int dev = 0;
  void* sc = nullptr;
  if (!own && segs > 1 && tiles >= kIPB && lds_spread <= 160 * 1024)
    sc = scratch_acquire(s, items * 16 * T * 4, &dev);
  if (!sc) {
    if (lds_own > 160 * 1024 || segs > kIPB) return hipErrorNotSupported;
    auto kern = q6k_decode_own_kernel<TP, PDO>;
    if (lds_own > 64 * 1024) {
      const hipError_t e = set_max_lds(reinterpret_cast<const void*>(kern), int(lds_own));
      if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kern, dim3(std::min<uint32_t>(tiles, uint32_t(cu_count()))), dim3(kW * 64), lds_own, s,
                       w.codes, w.scales, w.n, w.pn, kbs, x.codes, x.scales, x.m, x.pk, out, residual, tiles);
    return hipGetLastError();
  }
  auto kern = q6k_decode_spread_kernel<TP, PDS>;
  hipError_t e = hipSuccess;
  if (lds_spread > 64 * 1024)
    e = set_max_lds(reinterpret_cast<const void*>(kern), int(lds_spread));
  float* part = static_cast<float*>(sc);
  if (e == hipSuccess) {
    hipLaunchKernelGGL(kern, dim3(uint32_t((items + kIPB - 1) / kIPB)), dim3(kW * 64), lds_spread, s, w.codes,
                       w.scales, w.pn, kbs, x.codes, x.scales, x.m, x.pk, tiles, part);
    e = hipGetLastError();
  }
  if (e == hipSuccess) {
    hipLaunchKernelGGL(q6k_seg_sum_kernel<T>, dim3((tiles * 16 * T + 255) / 256), dim3(256), 0, s, part, segs,
                       tiles, w.n, x.m, out, residual);
    e = hipGetLastError();
  }
  scratch_release(dev, s, e == hipSuccess);
  return e;
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
  static const bool own_env = [] {  // tuning aid: 1 = whole tiles per block (no scratch)
    const char* e = std::getenv("QW38_Q6_DECODE_OWN");
    return e && std::atoi(e) == 1;
  }();
  if (!env || w.layout != QW38_LAYOUT_Q6K_WAVE64 || x.m > 8 || x.m < (env >= 2 ? 1u : 3u))
    return hipErrorNotSupported;
  if ((reinterpret_cast<uintptr_t>(w.codes) | reinterpret_cast<uintptr_t>(x.codes)) % 16 ||
      reinterpret_cast<uintptr_t>(w.scales) % 4)
    return hipErrorNotSupported;
  // Spread-mode weight ring: one super-block ahead (config 3 M=3 / M=8 with
  // 1, 2, 3, 4, 5 ahead: 20.4 / 22.3, 20.6 / 22.8, 20.8 / 23.5, 21.6 / 24.4,
  // 22.1 / 29.1 us; the staging and the LDS operand reads, not the weight
  // latency, set the pace). Own mode at M 5..8 keeps no ring (144 VGPRs).
  return x.m <= 4 ? launch_t<1, 1, 1>(w, x, out, residual, s, own_env)
                  : launch_t<2, 0, 1>(w, x, out, residual, s, own_env);
}

}  // namespace qw38hip
