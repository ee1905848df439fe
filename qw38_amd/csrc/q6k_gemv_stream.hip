// Linear-streaming Q6_K GEMV for M = 1..2 tokens (layout 0x0241; the down
// projection of the Q4_K_M mixture at decode).
//
// In layout 0x0241 an 8-row x K256 tile is 1536 contiguous code bytes (a
// 1024-byte low-nibble plane and a 512-byte high-pair plane, 16 B and 8 B per
// (row, K32 group) chunk), 128 contiguous bytes of int8 sub-block scales and
// 16 contiguous bytes of fp16 d, and the tiles of an 8-row strip follow one
// another. One wave streams one tile per step: lane l = 8 g + r owns row r,
// K32 group g (its low-nibble and high-pair chunks, the group's two sub-block
// scales and the row's d), so each plane is one contiguous wave load. The activations of a
// tile (8 groups x 32 codes) are loaded once per wave, one dword per lane
// (lane 8 g + i holds codes 4i..4i+3 of group g), and each lane gathers its
// group's eight dwords with ds_swizzle broadcasts inside its 8-lane group, so
// no lane re-reads another row's copy through the vector cache. WS waves of a
// block split a strip's tiles into contiguous ranges; loads run D tiles
// ahead, and nothing is staged in LDS.
//
// With codes q = 0..63, sub-block scales sc0, sc1 and the 16-code sums s0, s1
// of the activations (v_dot4 against ones), the reference's per-group integer
// is I = sc0 (sum_{16} q z - 32 s0) + sc1 (sum_{16} q z - 32 s1), from exact
// v_dot4_i32_i8 dots; each lane accumulates a d I in FP32 in K order, the
// group partials of a row are summed over its 8 lanes (xor 8, 16, 32), then
// over the waves in ascending order, so results do not depend on the grid.
#include <cstdlib>

#include "common.hpp"

namespace qw38hip {
namespace {

// One lane's share of one tile: row r, K32 group g, plus the group's Q8
// activations for MT tokens.
template <int MT>
struct Q6Step {
  uint32_t lo[4];      // 16 low-nibble bytes of (row, group)
  uint32_t hi[2];      // 8 high-pair bytes
  uint32_t sc;         // the group's two int8 sub-block scales (low half)
  uint32_t d;          // fp16 d of the row (low half)
  uint32_t z[MT];      // activation dword r of the lane's group, per token
  float a[MT];         // activation scale per token
};

template <int MT, bool Fast>
__device__ __forceinline__ void load_q6(const uint8_t* ctile, uint32_t chunk, const uint8_t* srow,
                                        const uint8_t* drow, const int8_t* zp, const float* ap,
                                        uint32_t pk, uint32_t groups, Q6Step<MT>& t) {
  const uint8_t* lp = ctile + chunk * 16;
  const uint8_t* hp = ctile + kQ6HiPlane + chunk * 8;
  if constexpr (Fast) {
    const uint4 a = *reinterpret_cast<const uint4*>(lp);
    const uint2 b = *reinterpret_cast<const uint2*>(hp);
    t.lo[0] = a.x; t.lo[1] = a.y; t.lo[2] = a.z; t.lo[3] = a.w;
    t.hi[0] = b.x; t.hi[1] = b.y;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) t.lo[i] = reinterpret_cast<const uint32_t*>(lp)[i];
    t.hi[0] = reinterpret_cast<const uint32_t*>(hp)[0];
    t.hi[1] = reinterpret_cast<const uint32_t*>(hp)[1];
  }
  t.sc = *reinterpret_cast<const uint16_t*>(srow);
  t.d = *reinterpret_cast<const uint16_t*>(drow);
#pragma unroll
  for (int tk = 0; tk < MT; ++tk) {
    t.z[tk] = *reinterpret_cast<const uint32_t*>(zp + size_t(tk) * pk);
    t.a[tk] = ap[size_t(tk) * groups];
  }
}

// Lane (lane & ~7) | I's value, for every lane: ds_swizzle in bit mode with
// and-mask 0x18, or-mask I (lanes are remapped within each 32-lane half).
template <int I>
__device__ __forceinline__ uint32_t bcast8(uint32_t v) {
  return uint32_t(__builtin_amdgcn_ds_swizzle(int(v), 0x18 | (I << 5)));
}

template <int MT>
__device__ __forceinline__ void consume_q6(const Q6Step<MT>& t, float acc[MT]) {
  uint32_t v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {  // low nibbles (0x0240 order) + high pairs -> q = 0..63
    const uint32_t nib = (j & 1) ? (t.lo[j >> 1] >> 4) & 0x0f0f0f0fu : t.lo[j >> 1] & 0x0f0f0f0fu;
    const uint32_t hh = (t.hi[j >> 2] >> (2 * (j & 3))) & 0x03030303u;
    v[j] = nib | (hh << 4);
  }
  const int sc0 = int(int8_t(t.sc & 0xffu)), sc1 = int(int8_t((t.sc >> 8) & 0xffu));
  const float d = f16_to_f32(t.d);
#pragma unroll
  for (int tk = 0; tk < MT; ++tk) {
    // dword i of the lane's group comes from lane (lane & ~7) | i
    const uint32_t z[8] = {bcast8<0>(t.z[tk]), bcast8<1>(t.z[tk]), bcast8<2>(t.z[tk]), bcast8<3>(t.z[tk]),
                           bcast8<4>(t.z[tk]), bcast8<5>(t.z[tk]), bcast8<6>(t.z[tk]), bcast8<7>(t.z[tk])};
    int d0 = 0, d1 = 0, s0 = 0, s1 = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      d0 = dot4(v[i], z[i], d0);
      s0 = dot4(0x01010101u, z[i], s0);
    }
#pragma unroll
    for (int i = 4; i < 8; ++i) {
      d1 = dot4(v[i], z[i], d1);
      s1 = dot4(0x01010101u, z[i], s1);
    }
    const int I = sc0 * (d0 - 32 * s0) + sc1 * (d1 - 32 * s1);
    acc[tk] = fmaf(t.a[tk] * d, float(I), acc[tk]);
  }
}

template <int MT, bool Fast, int WS>
__global__ __launch_bounds__(256) void q6_stream_kernel(
    const uint8_t* __restrict__ codes, const uint8_t* __restrict__ meta, uint32_t n,
    uint32_t strips, uint32_t kbs, const int8_t* __restrict__ xc, const float* __restrict__ xa,
    uint32_t pk, float* __restrict__ out, const float* __restrict__ residual, uint32_t persistent) {
  constexpr int NW = 4;  // waves per block
  constexpr int SPB = NW / WS;
  // tiles of loads in flight per wave (config 3, M=1: 1 tile 18.1 us, 2 tiles
  // 16.2-16.5, 3 tiles 16.7, 4 tiles 17.5, 5 or 6 tiles 18.6; M=2: 2 tiles
  // 18.1, 3 tiles 18.55)
  constexpr int D = 2;
  __shared__ float red[WS > 1 ? NW * MT * 8 : 1];
  const uint32_t groups = pk / 32;
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t g = lane >> 3, r = lane & 7u;
  const uint32_t ks = wave % WS;
  const uint32_t kb0 = uint32_t(uint64_t(kbs) * ks / WS);
  const uint32_t nkb = uint32_t(uint64_t(kbs) * (ks + 1) / WS) - kb0;
  const uint64_t tiles = uint64_t(strips) * kbs * 8;  // tile rows: the d array follows the scales
  const int8_t* zbase = xc + (size_t(kb0) * 8 + g) * 32 + r * 4;
  const float* abase = xa + size_t(kb0) * 8 + g;

  const uint32_t stride = persistent ? gridDim.x * SPB : SPB * gridDim.x + strips;
  for (uint32_t base = blockIdx.x * SPB; base < strips; base += stride) {
    const uint32_t strip = base + wave / WS;
    const bool live = strip < strips;
    if (WS == 1 && !live) break;
    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = 0.f;
    if (live && nkb > 0) {
      const uint64_t tr0 = (uint64_t(strip) * kbs + kb0) * 8 + r;  // tile row of (strip, kb0, r)
      const uint8_t* cbase = codes + (tr0 - r) * kQ6CodeBytes;  // the tile's first byte
      const uint32_t chunk = q6_chunk(r, g);
      const uint8_t* sbase = meta + tr0 * 16 + g * 2;
      const uint8_t* dbase = meta + tiles * 16 + tr0 * 2;
      auto ld = [&](Q6Step<MT>& T, uint32_t i) {  // tile kb0 + i, clamped to the range
        const uint32_t j = min(i, nkb - 1);
        load_q6<MT, Fast>(cbase + size_t(j) * kQ6TileBytes, chunk, sbase + size_t(j) * 128, dbase + size_t(j) * 16,
                          zbase + size_t(j) * 256, abase + size_t(j) * 8, pk, groups, T);
      };
      Q6Step<MT> ring[D];
#pragma unroll
      for (int u = 0; u < D; ++u) ld(ring[u], u);
      uint32_t i = 0;
      for (; i + D <= nkb; i += D) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
          const Q6Step<MT> cur = ring[u];
          ld(ring[u], i + u + D);
          consume_q6<MT>(cur, acc);
        }
      }
#pragma unroll
      for (int u = 0; u < D; ++u)
        if (i + u < nkb) consume_q6<MT>(ring[u], acc);
    }
    // a row's partials live in lanes r, r + 8, ..., r + 56
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      acc[t] += __shfl_xor(acc[t], 8);
      acc[t] += __shfl_xor(acc[t], 16);
      acc[t] += __shfl_xor(acc[t], 32);
    }
    const uint32_t row = strip * 8 + r;
    const bool writer = g == 0;
    if constexpr (WS == 1) {
      if (live && writer && row < n) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const size_t o = size_t(t) * n + row;
          out[o] = acc[t] + (residual ? residual[o] : 0.f);
        }
      }
    } else {
      if (writer) {
#pragma unroll
        for (int t = 0; t < MT; ++t) red[(wave * MT + t) * 8 + r] = acc[t];
      }
      __syncthreads();
      if (live && ks == 0 && writer && row < n) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          float total = 0.f;
#pragma unroll
          for (int q = 0; q < WS; ++q) total += red[((wave + q) * MT + t) * 8 + r];
          const size_t o = size_t(t) * n + row;
          out[o] = total + (residual ? residual[o] : 0.f);
        }
      }
      if (base + stride < strips) __syncthreads();  // red is rewritten by the next strip group
    }
  }
}

template <int MT, bool Fast>
hipError_t q6_stream_ws(const WeightView& w, const Q8View& x, float* out, const float* residual,
                        hipStream_t s, int ws, uint32_t max_blocks) {
  const uint32_t strips = w.pn / 8, kbs = w.pk / 256;
#define QW38_Q6_LAUNCH(WSV)                                                                  \
  do {                                                                                       \
    constexpr uint32_t spb = 4u / WSV;                                                       \
    const uint32_t need = (strips + spb - 1) / spb;                                          \
    const uint32_t persistent = need > max_blocks ? 1u : 0u;                                 \
    const uint32_t grid = persistent ? max_blocks : need;                                    \
    hipLaunchKernelGGL((q6_stream_kernel<MT, Fast, WSV>), dim3(grid), dim3(256), 0, s,      \
                       w.codes, w.scales, w.n, strips, kbs, x.codes, x.scales, x.pk, out,    \
                       residual, persistent);                                                \
  } while (0)
  if (ws == 4) QW38_Q6_LAUNCH(4);
  else if (ws == 2) QW38_Q6_LAUNCH(2);
  else QW38_Q6_LAUNCH(1);
#undef QW38_Q6_LAUNCH
  return hipGetLastError();
}

}  // namespace

// Returns hipErrorNotSupported when this path does not apply (caller falls back).
hipError_t launch_q6k_stream(const WeightView& w, const Q8View& x, float* out, const float* residual,
                             hipStream_t s) {
  if (x.m > 2 || w.layout != QW38_LAYOUT_Q6K_WAVE64) return hipErrorNotSupported;
  static const int env = [] {
    const char* e = std::getenv("QW38_Q6_STREAM");
    return e ? std::atoi(e) : 1;
  }();
  static const int env_ws = [] {
    const char* e = std::getenv("QW38_Q6_STREAM_WS");
    return e ? std::atoi(e) : 0;
  }();
  static const int env_blocks = [] {
    const char* e = std::getenv("QW38_Q6_STREAM_BLOCKS");
    return e ? std::atoi(e) : 0;
  }();
  if (!env) return hipErrorNotSupported;
  // Fast: 16-byte aligned codes; otherwise 4-byte loads with identical
  // arithmetic (activations are read as dwords and the scales as 2-byte
  // words, the reference's minimum alignment of the scales span).
  const bool fast = (reinterpret_cast<uintptr_t>(w.codes) % 16) == 0;
  const uint32_t strips = w.pn / 8, kbs = w.pk / 256;
  int ws = 1;  // split K over more waves when the strips alone cannot fill the chip
  if (strips < 4096 && kbs >= 8) ws = 2;
  if (strips < 2048 && kbs >= 16) ws = 4;
  if (env_ws == 1 || env_ws == 2 || env_ws == 4) ws = env_ws;
  const uint32_t max_blocks = env_blocks > 0 ? uint32_t(env_blocks) : 4u * uint32_t(cu_count());
  if (x.m == 1)
    return fast ? q6_stream_ws<1, true>(w, x, out, residual, s, ws, max_blocks)
                : q6_stream_ws<1, false>(w, x, out, residual, s, ws, max_blocks);
  return fast ? q6_stream_ws<2, true>(w, x, out, residual, s, ws, max_blocks)
              : q6_stream_ws<2, false>(w, x, out, residual, s, ws, max_blocks);
}

}  // namespace qw38hip
