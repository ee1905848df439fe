// Linear-streaming Q4_K GEMV for M = 1..2 tokens (the decode hot path).
//
// In the 8-row x K256 tiling an 8-row strip's codes are contiguous (kbs x
// 1 KB) and so is its metadata (kbs x 128 B in the scales span). One wave
// streams one strip two tiles at a time: lane l owns 32 contiguous code bytes
// at l*32 of the tile pair -- tile h = l/32, row r = (l%32)/4, K32 groups
// 2j, 2j+1 with j = l%4 -- so the wave's two 16 B loads read 2 KB with no
// gaps. One 4 B/lane load reads the pair's 256 B of metadata; the four dwords
// of (row r, tile h) land exactly in lane l's quad, so DPP quad broadcasts
// hand them over without LDS traffic. Loads run one tile pair ahead of the
// pair being consumed.
//
// The Q8 activations are staged once per block in LDS as codes plus
// (a, a*sum) pairs. Per (row, token, super-block) the affine is factored as
//   acc += d * sum_g (a_g s_g) dot_g - dmin * sum_g (a_g sum_g) m_g,
// the reference's sum_g a_g (d s_g dot_g - dmin m_g sum_g)
// (cuda/q4k_q8.cu:97) reassociated, with exact int32 K32 dots from
// v_dot4_i32_i8. Row partials are summed over the row's 8 lanes (xor 1, 2, 32)
// and, when WS waves split K, across those waves in LDS in a fixed order.
// Unaligned (4-byte) code / activation spans and 2-byte metadata spans use
// narrower loads with identical arithmetic, so results are bitwise equal.
#include <cstdlib>

#include "common.hpp"

namespace qw38hip {
namespace {

template <uint16_t Layout>
__device__ __forceinline__ void unpack8(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3,
                                        uint32_t v[8]) {
  const uint32_t ws[4] = {w0, w1, w2, w3};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t lo = ws[t] & 0x0f0f0f0fu;
    const uint32_t hi = (ws[t] >> 4) & 0x0f0f0f0fu;
    if constexpr (Layout == QW38_LAYOUT_Q4K_WAVE64) {
      v[2 * t] = lo;
      v[2 * t + 1] = hi;
    } else {
      v[2 * t] = perm(hi, lo, 0x05010400u);
      v[2 * t + 1] = perm(hi, lo, 0x07030602u);
    }
  }
}

// DPP quad broadcast of lane (quad base + J).
template <int J>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
  constexpr int ctrl = J | (J << 2) | (J << 4) | (J << 6);  // quad_perm:[J,J,J,J]
  return uint32_t(__builtin_amdgcn_mov_dpp(int(v), ctrl, 0xf, 0xf, false));
}

struct Tile {
  uint32_t c[8];  // 32 code bytes of this lane
  uint32_t m;     // one metadata dword of the tile pair
};

template <bool Fast>
__device__ __forceinline__ void load_tile(const uint8_t* cbase, const uint8_t* mbase,
                                          uint32_t coff, uint32_t moff, Tile& t) {
  if constexpr (Fast) {
    const uint4 a = *reinterpret_cast<const uint4*>(cbase + coff);
    const uint4 b = *reinterpret_cast<const uint4*>(cbase + coff + 16);
    t.c[0] = a.x; t.c[1] = a.y; t.c[2] = a.z; t.c[3] = a.w;
    t.c[4] = b.x; t.c[5] = b.y; t.c[6] = b.z; t.c[7] = b.w;
    t.m = *reinterpret_cast<const uint32_t*>(mbase + moff);
  } else {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(cbase + coff);
#pragma unroll
    for (int i = 0; i < 8; ++i) t.c[i] = q[i];
    const uint16_t* h = reinterpret_cast<const uint16_t*>(mbase + moff);
    t.m = uint32_t(h[0]) | (uint32_t(h[1]) << 16);
  }
}

// 6-bit scale s and min m of groups g0 = 2j and g0 + 1 (j = lane % 4) from
// packed words p0 = bytes 4..7, p1 = 8..11, p2 = 12..15 (get_scale_min_k4,
// third_party/llama.cpp-q4k/reference.hpp:174-181), branch-free in j.
__device__ __forceinline__ void scale_min_pair(uint32_t p0, uint32_t p1, uint32_t p2, bool hi,
                                               uint32_t sh, float s[2], float m[2]) {
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const uint32_t o = sh + 8u * e;  // byte offset of group g0+e (mod 4) in bits
    const uint32_t sl = __builtin_amdgcn_ubfe(hi ? p2 : p0, o, hi ? 4u : 6u);
    const uint32_t ml = __builtin_amdgcn_ubfe(hi ? p2 : p1, hi ? o + 4u : o, hi ? 4u : 6u);
    const uint32_t sh2 = hi ? __builtin_amdgcn_ubfe(p0, o + 6u, 2u) << 4 : 0u;
    const uint32_t mh2 = hi ? __builtin_amdgcn_ubfe(p1, o + 6u, 2u) << 4 : 0u;
    s[e] = float(sl | sh2);
    m[e] = float(ml | mh2);
  }
}

// One lane's share of a tile: 32 code bytes = K32 groups g0, g0+1 of one
// row. z: the two groups' 64 activation codes; au = (a0, a0*sum0, a1,
// a1*sum1). acc += d * sum_e a_e s_e dot_e - dmin * sum_e (a_e sum_e) m_e.
template <uint16_t Layout>
__device__ __forceinline__ void consume_core(const Tile& t, bool hi, uint32_t sh, const uint4 (&z)[4],
                                             float4 au, float& acc) {
  const uint32_t dd = quad_bcast<0>(t.m), p0 = quad_bcast<1>(t.m), p1 = quad_bcast<2>(t.m),
                 p2 = quad_bcast<3>(t.m);
  float s[2], m[2];
  scale_min_pair(p0, p1, p2, hi, sh, s, m);
  const float d = f16_to_f32(dd & 0xffffu), dmin = f16_to_f32(dd >> 16);
  uint32_t v[2][8];
  unpack8<Layout>(t.c[0], t.c[1], t.c[2], t.c[3], v[0]);
  unpack8<Layout>(t.c[4], t.c[5], t.c[6], t.c[7], v[1]);
  float X = 0.f, Y = 0.f;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const uint4 za = z[2 * e], zb = z[2 * e + 1];
    int dot = 0;
    dot = dot4(v[e][0], za.x, dot);
    dot = dot4(v[e][1], za.y, dot);
    dot = dot4(v[e][2], za.z, dot);
    dot = dot4(v[e][3], za.w, dot);
    dot = dot4(v[e][4], zb.x, dot);
    dot = dot4(v[e][5], zb.y, dot);
    dot = dot4(v[e][6], zb.z, dot);
    dot = dot4(v[e][7], zb.w, dot);
    const float a = e ? au.z : au.x, u = e ? au.w : au.y;
    X = fmaf(a * s[e], float(dot), X);
    Y = fmaf(u, m[e], Y);
  }
  acc = fmaf(-dmin, Y, fmaf(d, X, acc));
}

// consume_core per token with the activations of tile kb read from LDS.
template <uint16_t Layout, int MT, bool Fast>
__device__ __forceinline__ void consume(const Tile& t, uint32_t kb, uint32_t g0, bool hi,
                                        uint32_t sh, const int8_t* sz, const float2* sau,
                                        uint32_t groups, float acc[MT]) {
#pragma unroll
  for (int tk = 0; tk < MT; ++tk) {
    const uint32_t gi = tk * groups + kb * 8 + g0;
    const uint4* zp = reinterpret_cast<const uint4*>(sz + size_t(gi) * 32);
    const uint4 z[4] = {zp[0], zp[1], zp[2], zp[3]};
    const float4 au = *reinterpret_cast<const float4*>(sau + gi);  // (a0, u0, a1, u1)
    consume_core<Layout>(t, hi, sh, z, au, acc[tk]);
  }
}

// K is cut into four quarters of whole tile pairs (the odd tail tile joins
// the last); every row's result is 0 + p0 + p1 + p2 + p3 over the quarter
// partials p_i, each reduced over the row's lanes (xor 1, 2, 32) first,
// whatever number of waves splits K. So the WS = 1, 2, 4 kernels and the fused
// gate + up kernel below give bitwise-identical rows.
__device__ __forceinline__ uint32_t quarter_begin(uint32_t pairs, uint32_t i) {
  return uint32_t(uint64_t(pairs) * i / 4);
}

// Streams quarter qi of one strip into part[MT] (zeroed here).
template <uint16_t Layout, int MT, bool Fast>
__device__ __forceinline__ void stream_quarter(const uint8_t* cstrip, const uint8_t* mstrip, uint32_t kbs,
                                               uint32_t qi, uint32_t lane, const int8_t* sz,
                                               const float2* sau, uint32_t groups, float part[MT]) {
  const uint32_t h = lane >> 5;         // tile of the pair
  const uint32_t j = lane & 3u;         // group pair 2j, 2j+1
  const uint32_t g0 = 2 * j;
  const bool hi = j >= 2;
  const uint32_t sh = 16u * (j & 1u);   // bit offset of group g0 % 4
  const uint32_t coff = lane * 32, moff = lane * 4;
  const uint32_t pairs = kbs / 2;
  const uint32_t q0 = quarter_begin(pairs, qi), q1 = quarter_begin(pairs, qi + 1);
#pragma unroll
  for (int t = 0; t < MT; ++t) part[t] = 0.f;
  // Double-buffered tile pairs: the loads of pair q+1 are issued before pair
  // q is consumed, so memory stays busy while this wave computes.
  uint32_t q = q0;
  const uint32_t nb = q1 - q0;
  if (nb > 0) {
    Tile A, B;
    auto ld = [&](Tile& T, uint32_t qq) {
      load_tile<Fast>(cstrip + size_t(qq) * 2048, mstrip + size_t(qq) * 256, coff, moff, T);
    };
    auto cs = [&](const Tile& T, uint32_t qq) {
      consume<Layout, MT, Fast>(T, 2 * qq + h, g0, hi, sh, sz, sau, groups, part);
    };
    ld(A, q);
    uint32_t b = 0;
    for (; b + 2 <= nb; b += 2) {
      ld(B, q + 1);
      cs(A, q);
      ++q;
      if (b + 2 < nb) ld(A, q + 1);
      cs(B, q);
      ++q;
    }
    if (b < nb) {
      cs(A, q);
      ++q;
    }
  }
  if ((kbs & 1u) && qi == 3) {  // odd last tile: only lanes of tile 0 hold data
    const uint32_t kb = kbs - 1;
    Tile T;
    if (h == 0) {
      load_tile<Fast>(cstrip + size_t(kb) * 1024, mstrip + size_t(kb) * 128, coff, moff, T);
    } else {
      for (int i = 0; i < 8; ++i) T.c[i] = 0;
      T.m = 0;
    }
    float tp[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) tp[t] = 0.f;
    consume<Layout, MT, Fast>(T, h == 0 ? kb : 0, g0, hi, sh, sz, sau, groups, tp);
    if (h == 0) {
#pragma unroll
      for (int t = 0; t < MT; ++t) part[t] += tp[t];
    }
  }
  // a row's partials live in lanes {4r..4r+3} and {32+4r..32+4r+3}
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    part[t] += __shfl_xor(part[t], 1);
    part[t] += __shfl_xor(part[t], 2);
    part[t] += __shfl_xor(part[t], 32);
  }
}

// A whole strip streamed by one wave into its four quarter partials: the
// same consume sequence, lane reduction and partials as four stream_quarter
// calls (so rows are bitwise theirs), with the next tile pair's loads in
// flight across the quarter boundaries instead of restarting at each. The
// odd tail tile (odd kbs) is left to the caller's stream_quarter semantics:
// this is used only for even kbs.
template <uint16_t Layout, int MT, bool Fast>
__device__ __forceinline__ void stream_strip(const uint8_t* cstrip, const uint8_t* mstrip, uint32_t kbs,
                                             uint32_t lane, const int8_t* sz, const float2* sau,
                                             uint32_t groups, float part[4][MT], const Tile& first) {
  const uint32_t h = lane >> 5, j = lane & 3u, g0 = 2 * j;
  const bool hi = j >= 2;
  const uint32_t sh = 16u * (j & 1u);
  const uint32_t coff = lane * 32, moff = lane * 4;
  const uint32_t pairs = kbs / 2;
  Tile cur = first, nxt;  // pair 0, loaded by the caller
  uint32_t q = 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
#pragma unroll
    for (int t = 0; t < MT; ++t) part[u][t] = 0.f;
    const uint32_t q1 = quarter_begin(pairs, uint32_t(u) + 1);
    for (; q < q1; ++q) {
      const uint32_t qn = min(q + 1, pairs - 1);  // past the end: a harmless re-read
      load_tile<Fast>(cstrip + size_t(qn) * 2048, mstrip + size_t(qn) * 256, coff, moff, nxt);
      consume<Layout, MT, Fast>(cur, 2 * q + h, g0, hi, sh, sz, sau, groups, part[u]);
      cur = nxt;
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      part[u][t] += __shfl_xor(part[u][t], 1);
      part[u][t] += __shfl_xor(part[u][t], 2);
      part[u][t] += __shfl_xor(part[u][t], 32);
    }
  }
}

// stream_quarter with the quarter's first pair already in registers (`t`, in)
// and, while the quarter's last pair is consumed, the first pair of the same
// quarter of the next strip loaded into `t` (out) when there is one: a wave
// of the persistent grid then never starts a strip with a full memory latency.
// The consume sequence and lane reduction are stream_quarter's (bitwise the
// same partials). Even kbs only (no odd tail tile).
template <uint16_t Layout, int MT, bool Fast>
__device__ __forceinline__ void stream_quarter_chain(const uint8_t* cstrip, const uint8_t* mstrip,
                                                     const uint8_t* ncstrip, const uint8_t* nmstrip,
                                                     bool have_next, uint32_t kbs, uint32_t qi, uint32_t lane,
                                                     const int8_t* sz, const float2* sau, uint32_t groups,
                                                     float part[MT], Tile& t) {
  const uint32_t h = lane >> 5, j = lane & 3u, g0 = 2 * j;
  const bool hi = j >= 2;
  const uint32_t sh = 16u * (j & 1u);
  const uint32_t coff = lane * 32, moff = lane * 4;
  const uint32_t pairs = kbs / 2;
  const uint32_t q0 = quarter_begin(pairs, qi), q1 = quarter_begin(pairs, qi + 1);
#pragma unroll
  for (int u = 0; u < MT; ++u) part[u] = 0.f;
  Tile cur = t, nxt;
  for (uint32_t q = q0; q < q1; ++q) {
    if (q + 1 < q1)
      load_tile<Fast>(cstrip + size_t(q + 1) * 2048, mstrip + size_t(q + 1) * 256, coff, moff, nxt);
    else if (have_next)
      load_tile<Fast>(ncstrip + size_t(q0) * 2048, nmstrip + size_t(q0) * 256, coff, moff, nxt);
    consume<Layout, MT, Fast>(cur, 2 * q + h, g0, hi, sh, sz, sau, groups, part);
    cur = nxt;
  }
  t = cur;
#pragma unroll
  for (int u = 0; u < MT; ++u) {
    part[u] += __shfl_xor(part[u], 1);
    part[u] += __shfl_xor(part[u], 2);
    part[u] += __shfl_xor(part[u], 32);
  }
}

// A wave's whole K quarter (one to three tile pairs: even kbs of 8 to 24, so
// every quarter is non-empty) loaded into registers before the block stages its activations, so
// the first weight loads overlap the staging instead of following it: short
// launches (few strips per CU) are otherwise a chain of three memory
// latencies. Branch-free (a shorter quarter re-reads its last pair), so the
// loads stay countable for the waits that follow.
struct QuarterPre {
  Tile t[3];
  uint32_t n = 0;   // pairs of the quarter
  uint32_t q0 = 0;  // first pair of the quarter
};

typedef __attribute__((address_space(1))) const uint8_t g_u8;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const u32x4 g_u4;
typedef __attribute__((address_space(1))) const uint32_t g_u32;

// 16-byte aligned spans only. The strip pointers are global-memory pointers
// whose provenance the caller hides from the optimizer (otherwise loads
// through the read-only kernel arguments may be sunk past the barrier to their
// first use).
__device__ __forceinline__ void preload_quarter(g_u8* cstrip, g_u8* mstrip, uint32_t kbs, uint32_t qi,
                                                uint32_t lane, QuarterPre& p) {
  const uint32_t pairs = kbs / 2;
  const uint32_t q0 = quarter_begin(pairs, qi), q1 = quarter_begin(pairs, qi + 1);
  p.n = q1 - q0;
  p.q0 = q0;
#pragma unroll
  for (uint32_t b = 0; b < 3; ++b) {
    const uint32_t q = min(q0 + b, q1 - 1);
    g_u4* c = reinterpret_cast<g_u4*>(cstrip + size_t(q) * 2048 + lane * 32);
    const u32x4 a = c[0], d = c[1];
    Tile& t = p.t[b];
    t.c[0] = a.x; t.c[1] = a.y; t.c[2] = a.z; t.c[3] = a.w;
    t.c[4] = d.x; t.c[5] = d.y; t.c[6] = d.z; t.c[7] = d.w;
    t.m = *reinterpret_cast<g_u32*>(mstrip + size_t(q) * 256 + lane * 4);
  }
}

// stream_quarter over preloaded pairs: the same consume sequence and lane
// reduction, so the rows are bitwise those of stream_quarter.
template <uint16_t Layout, int MT, bool Fast>
__device__ __forceinline__ void consume_quarter(const QuarterPre& p, uint32_t lane, const int8_t* sz,
                                                const float2* sau, uint32_t groups, float part[MT]) {
  const uint32_t h = lane >> 5, j = lane & 3u, g0 = 2 * j;
  const bool hi = j >= 2;
  const uint32_t sh = 16u * (j & 1u);
#pragma unroll
  for (int t = 0; t < MT; ++t) part[t] = 0.f;
#pragma unroll
  for (uint32_t b = 0; b < 3; ++b)
    if (b < p.n) consume<Layout, MT, Fast>(p.t[b], 2 * (p.q0 + b) + h, g0, hi, sh, sz, sau, groups, part);
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    part[t] += __shfl_xor(part[t], 1);
    part[t] += __shfl_xor(part[t], 2);
    part[t] += __shfl_xor(part[t], 32);
  }
}

// Stages the Q8 activations of MT tokens in LDS: codes and (a, a*sum).
template <int MT, bool Fast, int NT>
__device__ __forceinline__ void stage_q8(const int8_t* __restrict__ xc, const float* __restrict__ xa,
                                         const int32_t* __restrict__ xs, uint32_t pk, int8_t* sz,
                                         float2* sau) {
  const uint32_t groups = pk / 32;
  if constexpr (Fast) {
    const uint4* src = reinterpret_cast<const uint4*>(xc);
    uint4* dst = reinterpret_cast<uint4*>(sz);
    for (uint32_t i = threadIdx.x; i < MT * pk / 16; i += NT) dst[i] = src[i];
  } else {
    const uint32_t* src = reinterpret_cast<const uint32_t*>(xc);
    uint32_t* dst = reinterpret_cast<uint32_t*>(sz);
    for (uint32_t i = threadIdx.x; i < MT * pk / 4; i += NT) dst[i] = src[i];
  }
  for (uint32_t i = threadIdx.x; i < MT * groups; i += NT) {
    const float a = xa[i];
    sau[i] = make_float2(a, a * float(xs[i]));
  }
}

template <uint16_t Layout, int MT, bool Fast, int WS, bool Pre = false>
__global__ __launch_bounds__(256) void gemv_stream_kernel(
    const uint8_t* __restrict__ codes, const uint8_t* __restrict__ meta, uint32_t n,
    uint32_t strips, uint32_t kbs, const int8_t* __restrict__ xc,
    const float* __restrict__ xa, const int32_t* __restrict__ xs, uint32_t pk,
    float* __restrict__ out, const float* __restrict__ residual, uint32_t persistent, uint32_t chain) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int SPB = 4 / WS, QPW = 4 / WS;  // strips per block, quarters per wave
  const uint32_t groups = pk / 32;
  int8_t* sz = reinterpret_cast<int8_t*>(smem);
  float2* sau = reinterpret_cast<float2*>(smem + MT * pk);
  float* red = reinterpret_cast<float*>(smem + MT * pk + MT * groups * 8);
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t r = (lane >> 2) & 7u;       // row in the strip
  const uint32_t ks = wave % WS;
  // Pre (chosen by the launcher: WS = 4, M = 1, 16-byte spans, even kbs of
  // 8 to 24, K <= 8192): the activations are read into registers first
  // (two 16-byte code vectors and one group per thread, clamped reads), then
  // the weight pairs, then the activations are written to LDS: loads complete
  // in issue order, so those writes wait only for the activation loads.
  QuarterPre pre;
  if constexpr (Pre) {
    const uint32_t nv = pk / 16;
    const uint4* src = reinterpret_cast<const uint4*>(xc);
    const uint32_t i0 = min(threadIdx.x, nv - 1), i1 = min(threadIdx.x + 256, nv - 1);
    const uint32_t gi = min(threadIdx.x, groups - 1);
    const uint4 v0 = src[i0], v1 = src[i1];
    const float a = xa[gi];
    const int32_t sm = xs[gi];
    __builtin_amdgcn_sched_barrier(0);  // keep the activation loads ahead of the weight loads
    const uint32_t strip0 = min(blockIdx.x, strips - 1);  // WS = 4: one strip per block
    // Laundered pointers: loads through the read-only kernel arguments may
    // otherwise be sunk past the barrier to their first use.
    uintptr_t cp = reinterpret_cast<uintptr_t>(codes + size_t(strip0) * kbs * 1024);
    uintptr_t mp = reinterpret_cast<uintptr_t>(meta + size_t(strip0) * kbs * 128);
    asm volatile("" : "+s"(cp), "+s"(mp));
    preload_quarter(reinterpret_cast<g_u8*>(cp), reinterpret_cast<g_u8*>(mp), kbs, ks, lane, pre);
    asm volatile("" ::: "memory");  // nor the weight loads sunk below the LDS writes
    // unconditional stores (threads past the end rewrite the last element
    // with its own value), so no load is sunk below the weight loads
    uint4* dst = reinterpret_cast<uint4*>(sz);
    dst[i0] = v0;
    dst[i1] = v1;
    sau[gi] = make_float2(a, a * float(sm));
  } else {
  stage_q8<MT, Fast, 256>(xc, xa, xs, pk, sz, sau);
  }
  __syncthreads();

  // Blocks walk strip groups with a block-uniform stride (a persistent grid
  // when it is smaller than the strip groups); with WS > 1 every wave of the
  // block runs every iteration, since the K-split reduction synchronises.
  const uint32_t stride = persistent ? gridDim.x * SPB : SPB * gridDim.x + strips;
  // One strip group; the first one of the block consumes the preloaded
  // quarter (peeled, so the preloaded pairs are dead in the loop after it).
  auto strip_group = [&](uint32_t base, bool first) __attribute__((always_inline)) {
    const uint32_t strip = base + wave / WS;
    const bool live = strip < strips;
    if (WS == 1 && !live) return false;
    float part[QPW][MT];
    if (live) {
      const uint8_t* cstrip = codes + size_t(strip) * kbs * 1024;
      const uint8_t* mstrip = meta + size_t(strip) * kbs * 128;
      if (Pre && first) {
        consume_quarter<Layout, MT, Fast>(pre, lane, sz, sau, groups, part[0]);
      } else {
#pragma unroll
        for (int u = 0; u < QPW; ++u)
          stream_quarter<Layout, MT, Fast>(cstrip, mstrip, kbs, ks * QPW + u, lane, sz, sau, groups, part[u]);
      }
    }
    const uint32_t row = strip * 8 + r;
    const bool writer = (lane & 35u) == 0;
    if constexpr (WS == 1) {
      if (writer && row < n) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          float total = 0.f;
#pragma unroll
          for (int u = 0; u < 4; ++u) total += part[u][t];
          const size_t i = size_t(t) * n + row;
          out[i] = total + (residual ? residual[i] : 0.f);
        }
      }
    } else {
      if (writer && live) {
#pragma unroll
        for (int u = 0; u < QPW; ++u)
#pragma unroll
          for (int t = 0; t < MT; ++t) red[((wave * QPW + u) * MT + t) * 8 + r] = part[u][t];
      }
      __syncthreads();
      if (live && ks == 0 && writer && row < n) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          float total = 0.f;
#pragma unroll
          for (int q = 0; q < 4; ++q) total += red[((wave * QPW + q) * MT + t) * 8 + r];
          const size_t i = size_t(t) * n + row;
          out[i] = total + (residual ? residual[i] : 0.f);
        }
      }
      if (base + stride < strips) __syncthreads();  // red is rewritten by the next strip group
    }
    return true;
  };
  uint32_t base = blockIdx.x * SPB;
  if constexpr (WS == 4 && Fast) {
    // Persistent K-split grid with even kbs: strips chained, the next strip's
    // first pair in flight while the current strip's last pair is consumed.
    if (Pre || chain) {  // (the Pre launch is always chained)
      const uint32_t lane_off = lane * 32, moff = lane * 4;
      const uint32_t pairs = kbs / 2, q0 = quarter_begin(pairs, ks);
      Tile t;
      auto strip_ptrs = [&](uint32_t st, const uint8_t*& c, const uint8_t*& mm) __attribute__((always_inline)) {
        c = codes + size_t(min(st, strips - 1)) * kbs * 1024;
        mm = meta + size_t(min(st, strips - 1)) * kbs * 128;
      };
      // the K-split reduction of one strip (as strip_group's)
      auto finish = [&](uint32_t strip, const float (&part)[MT], bool more) __attribute__((always_inline)) {
        const uint32_t row = strip * 8 + r;
        const bool writer = (lane & 35u) == 0;
        if (writer) {
#pragma unroll
          for (int u = 0; u < MT; ++u) red[((wave * QPW + 0) * MT + u) * 8 + r] = part[u];
        }
        __syncthreads();
        if (ks == 0 && writer && row < n) {
#pragma unroll
          for (int u = 0; u < MT; ++u) {
            float total = 0.f;
#pragma unroll
            for (int q = 0; q < 4; ++q) total += red[((wave * QPW + q) * MT + u) * 8 + r];
            const size_t i = size_t(u) * n + row;
            out[i] = total + (residual ? residual[i] : 0.f);
          }
        }
        if (more) __syncthreads();  // red is rewritten by the next strip
      };
      if (base < strips) {
        const uint8_t *c, *mm;
        strip_ptrs(Pre ? base + stride : base, c, mm);
        if (!Pre || base + stride < strips)
          load_tile<Fast>(c + size_t(q0) * 2048, mm + size_t(q0) * 256, lane_off, moff, t);
      }
      if (Pre && base < strips) {  // the first strip from the preloaded quarter
        float part[MT];
        consume_quarter<Layout, MT, Fast>(pre, lane, sz, sau, groups, part);
        finish(base, part, base + stride < strips);
        base += stride;
      }
      for (; base < strips; base += stride) {
        const bool have_next = base + stride < strips;
        const uint8_t *cs, *ms, *nc, *nm;
        strip_ptrs(base, cs, ms);
        strip_ptrs(base + stride, nc, nm);
        float part[MT];
        stream_quarter_chain<Layout, MT, Fast>(cs, ms, nc, nm, have_next, kbs, ks, lane, sz, sau, groups, part, t);
        finish(base, part, have_next);
      }
      return;
    }
  }
  if constexpr (!(WS == 4 && Fast && Pre)) {
    if (Pre && base < strips) {
      strip_group(base, true);
      base += stride;
    }
    for (; base < strips; base += stride)
      if (!strip_group(base, false)) break;
  }
}

template <uint16_t Layout, int MT, bool Fast>
hipError_t stream_ws(const WeightView& w, const Q8View& x, float* out, const float* residual,
                     hipStream_t s, int ws, uint32_t max_blocks) {
  const uint32_t strips = w.pn / 8, kbs = w.pk / 256;
  const uint32_t groups = w.pk / 32;
  const size_t lds = size_t(MT) * w.pk + size_t(MT) * groups * 8 + 8 * MT * 8 * 4;
  // Chained strips (persistent K-split grid, even kbs >= 8); QW38_GEMV_CHAIN=0
  // turns it off (same bits).
  static const bool chain_env = [] {
    const char* e = std::getenv("QW38_GEMV_CHAIN");
    return !(e && std::atoi(e) == 0);
  }();
  const uint32_t chain = (chain_env && ws == 4 && Fast && kbs % 2 == 0 && kbs >= 8) ? 1u : 0u;
#define QW38_STREAM_LAUNCH(WSV)                                                          \
  do {                                                                                   \
    const uint32_t need = (strips + (4 / WSV) - 1) / (4 / WSV);                          \
    const uint32_t persistent = need > max_blocks ? 1u : 0u;                             \
    const uint32_t grid = persistent ? max_blocks : need;                                \
    auto kern = gemv_stream_kernel<Layout, MT, Fast, WSV>;                               \
    if constexpr (WSV == 4 && MT == 1 && Fast)                                           \
      if (kbs % 2 == 0 && kbs >= 8 && kbs <= 24 && x.pk <= 8192)                         \
        kern = gemv_stream_kernel<Layout, MT, Fast, WSV, true>;                          \
    hipLaunchKernelGGL(kern, dim3(grid), dim3(256), lds, s, w.codes, w.scales, w.n,      \
                       strips, kbs, x.codes, x.scales, x.sums, x.pk, out, residual,      \
                       persistent, chain);                                               \
  } while (0)
  if (ws == 4) QW38_STREAM_LAUNCH(4);
  else if (ws == 2) QW38_STREAM_LAUNCH(2);
  else QW38_STREAM_LAUNCH(1);
#undef QW38_STREAM_LAUNCH
  return hipGetLastError();
}

template <uint16_t Layout, bool Fast>
hipError_t stream_m(const WeightView& w, const Q8View& x, float* out, const float* residual,
                    hipStream_t s, int ws, uint32_t max_blocks) {
  return x.m == 1 ? stream_ws<Layout, 1, Fast>(w, x, out, residual, s, ws, max_blocks)
                  : stream_ws<Layout, 2, Fast>(w, x, out, residual, s, ws, max_blocks);
}

// Fused decode gate + up with the SwiGLU -> Q8 epilogue (M = 1, layout
// 0x020D): block G owns K32 feature group G, i.e. gate strips 4G..4G+3 (waves
// 0-3) and up strips 4G..4G+3 (waves 4-7), one whole strip per wave in K
// quarters. The rows meet in LDS, and wave 0 packs the group: per token one
// 32-lane half computes BF16(SiLU(g) u) and its Q8 codes, scale and sum. The
// gate / up values are those of gemv_stream_kernel (same quarter sums), so
// the codes equal swiglu_q8 of two separate projections bit for bit; no FP32
// slab is written.
template <uint16_t Layout, int MT, bool Fast, bool Pre = false>
__global__ __launch_bounds__(512) void glu_stream_kernel(
    const uint8_t* __restrict__ gcodes, const uint8_t* __restrict__ gmeta,
    const uint8_t* __restrict__ ucodes, const uint8_t* __restrict__ umeta, uint32_t n, uint32_t kbs,
    const int8_t* __restrict__ xc, const float* __restrict__ xa, const int32_t* __restrict__ xs,
    uint32_t pk, int8_t* __restrict__ qc, float* __restrict__ qa, int32_t* __restrict__ qs, int* failure) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ float rows[8][MT][8];  // [wave][token][row in strip]
  const uint32_t groups = pk / 32;
  int8_t* sz = reinterpret_cast<int8_t*>(smem);
  float2* sau = reinterpret_cast<float2*>(smem + MT * pk);
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t G = blockIdx.x;
  const uint32_t strip = G * 4 + (wave & 3u);
  const bool up = wave >= 4;
  const uint8_t* cstrip = (up ? ucodes : gcodes) + size_t(strip) * kbs * 1024;
  const uint8_t* mstrip = (up ? umeta : gmeta) + size_t(strip) * kbs * 128;
  // Strip path (Pre: even kbs >= 8, M = 1, 16-byte spans, K <= 8192): the
  // activations are read into registers, then the strip's first tile pair,
  // then the activations are written to LDS, so the staging latency and the
  // first weight latency overlap (as in gemv_stream_kernel's Pre path).
  Tile first;
  if constexpr (Pre) {
    const uint32_t nv = pk / 16;
    const uint4* src = reinterpret_cast<const uint4*>(xc);
    const uint32_t i0 = min(threadIdx.x, nv - 1);
    const uint32_t gi = min(threadIdx.x, groups - 1);
    const uint4 v0 = src[i0];
    const float a = xa[gi];
    const int32_t sm = xs[gi];
    __builtin_amdgcn_sched_barrier(0);
    uintptr_t cp = reinterpret_cast<uintptr_t>(cstrip), mp = reinterpret_cast<uintptr_t>(mstrip);
    asm volatile("" : "+v"(cp), "+v"(mp));
    {
      g_u4* c = reinterpret_cast<g_u4*>(reinterpret_cast<g_u8*>(cp) + lane * 32);
      const u32x4 x0 = c[0], x1 = c[1];
      first.c[0] = x0.x; first.c[1] = x0.y; first.c[2] = x0.z; first.c[3] = x0.w;
      first.c[4] = x1.x; first.c[5] = x1.y; first.c[6] = x1.z; first.c[7] = x1.w;
      first.m = *reinterpret_cast<g_u32*>(reinterpret_cast<g_u8*>(mp) + lane * 4);
    }
    asm volatile("" ::: "memory");
    float a2 = a;
    int32_t sm2 = sm;
    asm volatile("" : "+v"(a2), "+v"(sm2));  // their arithmetic stays behind the weight loads
    uint4* dst = reinterpret_cast<uint4*>(sz);
    dst[i0] = v0;  // nv <= 512: one vector per thread (threads past the end rewrite the last)
    sau[gi] = make_float2(a2, a2 * float(sm2));
  } else {
    stage_q8<MT, Fast, 512>(xc, xa, xs, pk, sz, sau);
  }
  __syncthreads();

  float part[4][MT];
  if constexpr (Pre) {
    stream_strip<Layout, MT, Fast>(cstrip, mstrip, kbs, lane, sz, sau, groups, part, first);
  } else {
#pragma unroll
    for (int u = 0; u < 4; ++u)
      stream_quarter<Layout, MT, Fast>(cstrip, mstrip, kbs, u, lane, sz, sau, groups, part[u]);
  }
  if ((lane & 35u) == 0) {
    const uint32_t r = (lane >> 2) & 7u;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      float total = 0.f;
#pragma unroll
      for (int u = 0; u < 4; ++u) total += part[u][t];
      rows[wave][t][r] = total;
    }
  }
  __syncthreads();
  if (wave != 0) return;
  const uint32_t t = lane >> 5, i = lane & 31u;  // token, feature in the group
  const bool on = t < uint32_t(MT);
  const uint32_t tt = on ? t : 0u;
  const float x = swiglu_q8_value(rows[i >> 3][tt][i & 7u], rows[4 + (i >> 3)][tt][i & 7u]);
  q8_group32(x, qc, qa, qs, size_t(tt) * (n / 32) + G, failure, on);
}

template <uint16_t Layout, int MT, bool Fast>
hipError_t glu_launch(const WeightView& g, const WeightView& u, const Q8View& x, int8_t* qc, float* qa,
                      int32_t* qs, int* failure, hipStream_t s) {
  const size_t lds = size_t(MT) * g.pk + size_t(MT) * (g.pk / 32) * 8;
  auto kern = glu_stream_kernel<Layout, MT, Fast>;
  if constexpr (MT == 1 && Fast)
    if (g.pk % 512 == 0 && g.pk >= 2048 && g.pk <= 8192) kern = glu_stream_kernel<Layout, MT, Fast, true>;
  hipLaunchKernelGGL(kern, dim3(g.n / 32), dim3(512), lds, s, g.codes,
                     g.scales, u.codes, u.scales, g.n, g.pk / 256, x.codes, x.scales, x.sums, x.pk, qc, qa,
                     qs, failure);
  return hipGetLastError();
}

}  // namespace

// Returns hipErrorNotSupported when this path does not apply (caller falls back).
hipError_t launch_gemv_stream(const WeightView& w, const Q8View& x, float* out,
                              const float* residual, hipStream_t s, int ws_override,
                              uint32_t max_blocks) {
  if (x.m > 2 || w.layout != QW38_LAYOUT_Q4K_CANDIDATE_V2) return hipErrorNotSupported;
  const size_t lds = size_t(x.m) * w.pk * 5 / 4 + 8 * x.m * 8 * 4;
  if (lds > 56 * 1024) return hipErrorNotSupported;
  const bool fast = ((reinterpret_cast<uintptr_t>(w.codes) | reinterpret_cast<uintptr_t>(x.codes)) %
                         16 == 0) &&
                    reinterpret_cast<uintptr_t>(w.scales) % 4 == 0;
  const uint32_t strips = w.pn / 8, kbs = w.pk / 256;
  // K split and grid. Long K: a persistent grid of four blocks per CU, so
  // each block stages the activations once for several strips; at M = 1 four
  // waves share a strip (short contiguous runs per wave read HBM best), at
  // M = 2 (twice the consume work per byte) one wave streams a whole strip.
  int ws = 1;
  if (strips < 6144 && kbs >= 8) ws = 2;
  if (strips < 1536 && kbs >= 16) ws = 4;
  uint32_t blocks = 0xffffffffu;
  if (kbs >= 16) {
    ws = x.m == 1 ? 4 : 1;
    blocks = 4u * uint32_t(cu_count());
  }
  if (ws_override == 1 || ws_override == 2 || ws_override == 4) ws = ws_override;
  if (max_blocks == 0) {
    max_blocks = blocks;
    // M = 1 (four waves per strip): one block per strip instead of the
    // persistent grid when that is a whole number of blocks per CU and at
    // most twice the persistent grid, which would give half its blocks two
    // strips and half one (12288 x 5120: 1536 blocks 8.26 us against
    // 8.70 us on 1024). Same bits: rows do not depend on the grid.
    const uint32_t need = (strips + (4 / ws) - 1) / (4 / ws), cus = uint32_t(cu_count());
    if (ws == 4 && blocks != 0xffffffffu && need > blocks && need <= 2 * blocks && need % cus == 0)
      max_blocks = need;
  }
  if (w.layout == QW38_LAYOUT_Q4K_CANDIDATE_V2)
    return fast ? stream_m<QW38_LAYOUT_Q4K_CANDIDATE_V2, true>(w, x, out, residual, s, ws, max_blocks)
                : stream_m<QW38_LAYOUT_Q4K_CANDIDATE_V2, false>(w, x, out, residual, s, ws, max_blocks);
  return fast ? stream_m<QW38_LAYOUT_Q4K_WAVE64, true>(w, x, out, residual, s, ws, max_blocks)
              : stream_m<QW38_LAYOUT_Q4K_WAVE64, false>(w, x, out, residual, s, ws, max_blocks);
}

bool gemv_glu_applies(const WeightView& gate, const WeightView& up, uint32_t m) {
  return m == 1 && gate.layout == QW38_LAYOUT_Q4K_CANDIDATE_V2 && up.layout == gate.layout &&
         gate.n == up.n && gate.k == up.k && gate.pk == up.pk && gate.n % 32 == 0 && gate.pn == gate.n &&
         size_t(m) * gate.pk * 5 / 4 <= 48 * 1024;
}

hipError_t launch_gemv_glu(const WeightView& gate, const WeightView& up, const Q8View& x, int8_t* codes,
                           float* scales, int32_t* sums, int* failure, hipStream_t s) {
  if (!gemv_glu_applies(gate, up, x.m)) return hipErrorNotSupported;
  const bool fast = ((reinterpret_cast<uintptr_t>(gate.codes) | reinterpret_cast<uintptr_t>(up.codes) |
                      reinterpret_cast<uintptr_t>(x.codes)) % 16 == 0) &&
                    ((reinterpret_cast<uintptr_t>(gate.scales) | reinterpret_cast<uintptr_t>(up.scales)) % 4 == 0);
  constexpr uint16_t L = QW38_LAYOUT_Q4K_CANDIDATE_V2;
  return fast ? glu_launch<L, 1, true>(gate, up, x, codes, scales, sums, failure, s)
              : glu_launch<L, 1, false>(gate, up, x, codes, scales, sums, failure, s);
}

}  // namespace qw38hip
