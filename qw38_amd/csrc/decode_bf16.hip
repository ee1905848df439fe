// BF16-activation decode GEMV over Q4_K weights (layout 0x020D), M = 1.
//
// Semantics (cuda/decode_mmv.cu:121-140, 182-250): every weight is rebuilt
// as the BF16 operand  w = BF16_RNE(fl(fl(d * s_g) * c) - fl(dmin * m_g))
// and y_r = sum_k w_rk * x_k in FP32, followed by the epilogue
// (StoreBf16 / StoreFp32 / ResidualAddFp32 / paired SwiGLU -> BF16).
//
// fl(d * s) and fl(dmin * m) are exact (an 11-bit by 6-bit significand
// product) and so is fl(d * s) * c (at most 21 bits), so
// fma(ds, c, -dm) == fl(fl(ds * c) - dm) bit for bit: one VALU op per weight.
// Pairs of weights become one BF16x2 word (v_cvt_pk_bf16_f32, round to
// nearest even) and meet the input pair in one v_dot2 (products of BF16 values
// are exact in FP32). A one-hot input therefore returns each rebuilt operand
// exactly.
//
// Mapping: one wave64 streams one 8-row strip two 1 KB tiles at a time; lane
// l owns 32 contiguous code bytes (tile l/32, row (l%32)/4, K32 groups 2j and
// 2j+1 with j = l%4), its metadata dword arrives by DPP quad broadcast, and
// the BF16 input is staged once per block in LDS. Row partials: xor 1, 2, 32
// lanes, then across the WS waves that split K, in a fixed order.
#include "common.hpp"

namespace qw38hip {
namespace {

typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
typedef float fl2 __attribute__((ext_vector_type(2)));

template <int J>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
  constexpr int ctrl = J | (J << 2) | (J << 4) | (J << 6);  // quad_perm:[J,J,J,J]
  return uint32_t(__builtin_amdgcn_mov_dpp(int(v), ctrl, 0xf, 0xf, false));
}


struct Tile {
  uint32_t c[8];
  uint32_t m;
};

template <bool Fast>
__device__ __forceinline__ void load_tile(const uint8_t* cbase, const uint8_t* mbase, Tile& t) {
  if constexpr (Fast) {
    const uint4 a = *reinterpret_cast<const uint4*>(cbase);
    const uint4 b = *reinterpret_cast<const uint4*>(cbase + 16);
    t.c[0] = a.x; t.c[1] = a.y; t.c[2] = a.z; t.c[3] = a.w;
    t.c[4] = b.x; t.c[5] = b.y; t.c[6] = b.z; t.c[7] = b.w;
    t.m = *reinterpret_cast<const uint32_t*>(mbase);
  } else {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(cbase);
#pragma unroll
    for (int i = 0; i < 8; ++i) t.c[i] = q[i];
    const uint16_t* h = reinterpret_cast<const uint16_t*>(mbase);
    t.m = uint32_t(h[0]) | (uint32_t(h[1]) << 16);
  }
}

// One lane's 64 weights of tile (row r, super-block kb, groups g0, g0+1)
// against the staged input; adds into acc.
__device__ __forceinline__ void consume(const Tile& t, uint32_t kb, uint32_t g0, bool hi,
                                        uint32_t sh, const uint32_t* xs, float& acc) {
  const uint32_t dd = quad_bcast<0>(t.m), p0 = quad_bcast<1>(t.m), p1 = quad_bcast<2>(t.m),
                 p2 = quad_bcast<3>(t.m);
  const float d = f16_to_f32(dd & 0xffffu), dmin = f16_to_f32(dd >> 16);
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const uint32_t o = sh + 8u * e;
    const uint32_t sl = __builtin_amdgcn_ubfe(hi ? p2 : p0, o, hi ? 4u : 6u);
    const uint32_t ml = __builtin_amdgcn_ubfe(hi ? p2 : p1, hi ? o + 4u : o, hi ? 4u : 6u);
    const uint32_t sh2 = hi ? __builtin_amdgcn_ubfe(p0, o + 6u, 2u) << 4 : 0u;
    const uint32_t mh2 = hi ? __builtin_amdgcn_ubfe(p1, o + 6u, 2u) << 4 : 0u;
    const float ds = d * float(sl | sh2);     // exact
    const float ndm = -(dmin * float(ml | mh2));  // exact
    // input words of this group: x pairs (2b, 2b+1), b = 0..15
    const uint4* xp = reinterpret_cast<const uint4*>(xs + (kb * 256 + (g0 + e) * 32) / 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // code word i: bytes 4i..4i+3 = codes 8i..8i+7
      const uint32_t w = t.c[4 * e + i];
      uint32_t lo = w & 0x0f0f0f0fu, hv = (w >> 4) & 0x0f0f0f0fu;
      // Opaque to the optimizer, so each byte converts with one
      // v_cvt_f32_ubyte{0..3} instead of a bit-field extract and a convert.
      asm volatile("" : "+v"(lo), "+v"(hv));
      const uint4 xv = xp[i];
      const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float c0 = float((lo >> (8 * q)) & 0xffu);   // code 8i + 2q
        const float c1 = float((hv >> (8 * q)) & 0xffu);   // code 8i + 2q + 1
        const fl2 wv = {fmaf(ds, c0, ndm), fmaf(ds, c1, ndm)};
        const bf2 wb = __builtin_convertvector(wv, bf2);  // v_cvt_pk_bf16_f32, RNE
        acc = __builtin_amdgcn_fdot2_f32_bf16(wb, __builtin_bit_cast(bf2, xw[q]), acc, false);
      }
    }
  }
}

__device__ __forceinline__ void epilogue(int epi, void* out, const float* residual, uint32_t row,
                                         float acc) {
  if (epi == QW38_DECODE_STORE_BF16) {
    static_cast<uint16_t*>(out)[row] = f32_to_bf16_rne(acc);
  } else if (epi == QW38_DECODE_STORE_FP32) {
    static_cast<float*>(out)[row] = acc;
  } else {  // residual add, in place when no separate output
    float* dst = out ? static_cast<float*>(out) : const_cast<float*>(residual);
    dst[row] = residual[row] + acc;
  }
}

template <bool Paired, bool Fast, int WS>
__global__ __launch_bounds__(256) void decode_bf16_kernel(
    const uint8_t* __restrict__ codes_a, const uint8_t* __restrict__ meta_a,
    const uint8_t* __restrict__ codes_b, const uint8_t* __restrict__ meta_b,
    const uint16_t* __restrict__ x, uint32_t k, uint32_t pk, uint32_t n, uint32_t strips,
    void* out_a, void* out_b, const float* res_a, const float* res_b, int epi) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int SPB = 4 / WS;
  uint32_t* xs = reinterpret_cast<uint32_t*>(smem);  // BF16 pairs
  float* red = reinterpret_cast<float*>(smem + size_t(pk) * 2);
  const uint32_t kbs = pk / 256;

  // ---- stage the BF16 input once per block, zero past k ----
  {
    uint16_t* x16 = reinterpret_cast<uint16_t*>(smem);
    for (uint32_t i = threadIdx.x; i < pk; i += 256) x16[i] = i < k ? x[i] : uint16_t(0);
  }
  __syncthreads();

  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t h = lane >> 5, r = (lane >> 2) & 7u, j = lane & 3u;
  const uint32_t g0 = 2 * j;
  const bool hi = j >= 2;
  const uint32_t sh = 16u * (j & 1u);
  const uint32_t ks = wave % WS;
  const uint32_t pairs = kbs / 2;
  const uint32_t q0 = uint32_t(uint64_t(pairs) * ks / WS);
  const uint32_t q1 = uint32_t(uint64_t(pairs) * (ks + 1) / WS);
  const bool tail = (kbs & 1u) && ks == WS - 1;
  const uint32_t strip = blockIdx.x * SPB + wave / WS;
  const bool live = strip < strips;

  float acc_a = 0.f, acc_b = 0.f;
  if (live) {
    const size_t cs = size_t(strip) * kbs * 1024 + lane * 32, ms = size_t(strip) * kbs * 128 + lane * 4;
    constexpr uint32_t kBatch = 4;
    uint32_t q = q0;
    for (; q + kBatch <= q1; q += kBatch) {
      Tile A[kBatch], B[Paired ? kBatch : 1];
#pragma unroll
      for (uint32_t u = 0; u < kBatch; ++u) {
        load_tile<Fast>(codes_a + cs + size_t(q + u) * 2048, meta_a + ms + size_t(q + u) * 256, A[u]);
        if constexpr (Paired)
          load_tile<Fast>(codes_b + cs + size_t(q + u) * 2048, meta_b + ms + size_t(q + u) * 256, B[u]);
      }
#pragma unroll
      for (uint32_t u = 0; u < kBatch; ++u) {
        consume(A[u], 2 * (q + u) + h, g0, hi, sh, xs, acc_a);
        if constexpr (Paired) consume(B[u], 2 * (q + u) + h, g0, hi, sh, xs, acc_b);
      }
    }
    for (; q < q1; ++q) {
      Tile A, B;
      load_tile<Fast>(codes_a + cs + size_t(q) * 2048, meta_a + ms + size_t(q) * 256, A);
      consume(A, 2 * q + h, g0, hi, sh, xs, acc_a);
      if constexpr (Paired) {
        load_tile<Fast>(codes_b + cs + size_t(q) * 2048, meta_b + ms + size_t(q) * 256, B);
        consume(B, 2 * q + h, g0, hi, sh, xs, acc_b);
      }
    }
    if (tail) {  // odd last tile: only lanes of tile 0 hold data
      const uint32_t kb = kbs - 1;
      const size_t ct = size_t(strip) * kbs * 1024 + size_t(kb) * 1024 + (lane & 31u) * 32;
      const size_t mt = size_t(strip) * kbs * 128 + size_t(kb) * 128 + (lane & 31u) * 4;
      Tile A, B;
      load_tile<Fast>(codes_a + ct, meta_a + mt, A);
      float pa = 0.f, pb = 0.f;
      consume(A, kb, g0, hi, sh, xs, pa);
      if constexpr (Paired) {
        load_tile<Fast>(codes_b + ct, meta_b + mt, B);
        consume(B, kb, g0, hi, sh, xs, pb);
      }
      if (h == 0) {
        acc_a += pa;
        acc_b += pb;
      }
    }
  }
  // a row's partials live in lanes {4r..4r+3} and {32+4r..32+4r+3}
  acc_a += __shfl_xor(acc_a, 1);
  acc_a += __shfl_xor(acc_a, 2);
  acc_a += __shfl_xor(acc_a, 32);
  if constexpr (Paired) {
    acc_b += __shfl_xor(acc_b, 1);
    acc_b += __shfl_xor(acc_b, 2);
    acc_b += __shfl_xor(acc_b, 32);
  }
  const uint32_t row = strip * 8 + r;
  const bool writer = (lane & 35u) == 0;
  if constexpr (WS > 1) {
    if (writer) {
      red[(wave * 2 + 0) * 8 + r] = acc_a;
      red[(wave * 2 + 1) * 8 + r] = acc_b;
    }
    __syncthreads();
    if (ks != 0) return;
    acc_a = acc_b = 0.f;
#pragma unroll
    for (int qq = 0; qq < WS; ++qq) {
      acc_a += red[((wave + qq) * 2 + 0) * 8 + r];
      acc_b += red[((wave + qq) * 2 + 1) * 8 + r];
    }
  }
  if (!live || !writer || row >= n) return;
  if (Paired && epi == QW38_DECODE_SWIGLU_BF16) {
    static_cast<uint16_t*>(out_a)[row] = f32_to_bf16_rne(silu(acc_a) * acc_b);
    return;
  }
  epilogue(epi, out_a, res_a, row, acc_a);
  if constexpr (Paired) epilogue(epi, out_b, res_b, row, acc_b);
}

template <bool Paired, bool Fast>
hipError_t launch_ws(const uint8_t* ca, const uint8_t* ma, const uint8_t* cb, const uint8_t* mb,
                     const uint16_t* x, uint32_t k, uint32_t pk, uint32_t n, uint32_t pn,
                     void* oa, void* ob, const float* ra, const float* rb, int epi,
                     hipStream_t s) {
  const uint32_t strips = pn / 8, kbs = pk / 256;
  int ws = 1;
  if (strips < 3072 && kbs >= 8) ws = 2;
  if (strips < 1536 && kbs >= 16) ws = 4;
  const size_t lds = size_t(pk) * 2 + 4 * 2 * 8 * 4;
#define QW38_BF16_LAUNCH(WSV)                                                                \
  hipLaunchKernelGGL((decode_bf16_kernel<Paired, Fast, WSV>),                                \
                     dim3((strips + (4 / WSV) - 1) / (4 / WSV)), dim3(256), lds, s, ca, ma, cb, mb, \
                     x, k, pk, n, strips, oa, ob, ra, rb, epi)
  if (ws == 4) QW38_BF16_LAUNCH(4);
  else if (ws == 2) QW38_BF16_LAUNCH(2);
  else QW38_BF16_LAUNCH(1);
#undef QW38_BF16_LAUNCH
  return hipGetLastError();
}

}  // namespace

hipError_t launch_decode_bf16(const WeightView& a, const WeightView* b, const uint16_t* x,
                              void* out_a, void* out_b, const float* res_a, const float* res_b,
                              int epilogue, hipStream_t s) {
  if (a.layout != QW38_LAYOUT_Q4K_CANDIDATE_V2) return hipErrorInvalidValue;
  auto aligned = [](const void* p, uintptr_t m) { return (reinterpret_cast<uintptr_t>(p) % m) == 0; };
  const bool fast = aligned(a.codes, 16) && aligned(a.scales, 4) &&
                    (!b || (aligned(b->codes, 16) && aligned(b->scales, 4)));
  const uint8_t* cb = b ? b->codes : nullptr;
  const uint8_t* mb = b ? b->scales : nullptr;
  if (b)
    return fast ? launch_ws<true, true>(a.codes, a.scales, cb, mb, x, a.k, a.pk, a.n, a.pn, out_a,
                                        out_b, res_a, res_b, epilogue, s)
                : launch_ws<true, false>(a.codes, a.scales, cb, mb, x, a.k, a.pk, a.n, a.pn, out_a,
                                         out_b, res_a, res_b, epilogue, s);
  return fast ? launch_ws<false, true>(a.codes, a.scales, cb, mb, x, a.k, a.pk, a.n, a.pn, out_a,
                                       out_b, res_a, res_b, epilogue, s)
              : launch_ws<false, false>(a.codes, a.scales, cb, mb, x, a.k, a.pk, a.n, a.pn, out_a,
                                        out_b, res_a, res_b, epilogue, s);
}

// ---------------------------------------------------------------------------
// The reference's other decode_mmv weight layouts (cuda/decode_mmv.cu:92-180):
//   Q4G64 (0x0201 / 0x020B): signed nibbles, one FP16 scale per 64 weights
//   Q8G32 (0x0202 / 0x020C): int8 codes, one FP16 scale per 32 weights
//   BF16 dense tile (0x0203): BF16 weights
// all in the 8-row x K256 tile order (tile_row = ((row/8) * K/256 + kb) * 8 +
// row % 8, so an 8-row strip is one contiguous run of tiles). Each weight is
// the BF16 operand  w = BF16_RNE(code * scale)  (code * scale is exact in FP32:
// an 11-bit significand times at most 8 bits), or the stored BF16 value.
// A zero scale gives a signed zero where the reference writes +0; no sum can
// tell them apart.
//
// Mapping: one wave64 streams one strip, 2 KB (Q4: a tile pair; Q8: one
// tile) or 4 KB (BF16: one tile) per iteration, every lane reading 32 or 64
// contiguous bytes:
//   Q4:   lane l -> tile l/32 of the pair, row (l%32)/4, 64 weights of group l%4
//   Q8:   lane l -> row l/8, 32 weights of group l%8
//   BF16: lane l -> row l/8, 32 weights at K offset (l%8)*32
// so each lane needs exactly one FP16 scale, and the lane-order scale entries
// of one iteration are contiguous (one 2 B load per lane).
// ---------------------------------------------------------------------------
namespace {

enum class DKind { Q4, Q8, Bf16 };

template <DKind K>
struct DUnit {
  static constexpr int kWords = K == DKind::Bf16 ? 16 : 8;
  uint32_t c[kWords];
  uint32_t s;  // FP16 scale bits (Q4, Q8)
};

template <DKind K>
struct DGeom {
  static constexpr uint32_t kTileBytes = K == DKind::Q4 ? 1024 : K == DKind::Q8 ? 2048 : 4096;
  static constexpr uint32_t kTileScales = K == DKind::Q4 ? 64 : 128;  // bytes per tile
  static constexpr uint32_t kTilesPerUnit = K == DKind::Q4 ? 2 : 1;
};

// Loads unit (first tile t0) of one lane; `half` limits a Q4 tail unit to its
// first tile (lanes of the missing second tile read nothing).
template <DKind K>
__device__ __forceinline__ void load_unit(const uint8_t* codes, const uint8_t* scales, size_t t0,
                                          uint32_t lane, bool half, DUnit<K>& u) {
  using G = DGeom<K>;
  const bool skip = half && lane >= 32;
  if (skip) {
#pragma unroll
    for (int i = 0; i < DUnit<K>::kWords; ++i) u.c[i] = 0;
    u.s = 0;
    return;
  }
  const uint4* cp = reinterpret_cast<const uint4*>(codes + t0 * G::kTileBytes +
                                                   lane * (K == DKind::Bf16 ? 64u : 32u));
#pragma unroll
  for (int i = 0; i < DUnit<K>::kWords / 4; ++i) {
    const uint4 v = cp[i];
    u.c[4 * i] = v.x; u.c[4 * i + 1] = v.y; u.c[4 * i + 2] = v.z; u.c[4 * i + 3] = v.w;
  }
  if constexpr (K != DKind::Bf16)
    u.s = *reinterpret_cast<const uint16_t*>(scales + t0 * G::kTileScales + lane * 2u);
}

// acc += sum over this lane's weights of w * x; k0 = K offset of the lane's first weight.
template <DKind K>
__device__ __forceinline__ void consume_unit(const DUnit<K>& u, uint32_t k0, const uint32_t* xs,
                                             float& acc) {
  const uint4* xp = reinterpret_cast<const uint4*>(xs + k0 / 2);
  if constexpr (K == DKind::Bf16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 xv = xp[i];
      const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
      for (int q = 0; q < 4; ++q)
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, u.c[4 * i + q]),
                                              __builtin_bit_cast(bf2, xw[q]), acc, false);
    }
  } else if constexpr (K == DKind::Q4) {
    // A signed nibble c is (c ^ 8) - 8 with c ^ 8 in 0..15, so every weight is
    // fma(s, u, -8 s) with u = (nibble ^ 8): exact, as c * s is (4 + 11
    // significant bits), hence the same BF16 after the RNE convert.
    const float s = f16_to_f32(u.s), n8 = -8.f * s;
#pragma unroll
    for (int i = 0; i < 8; ++i) {  // word i: bytes 4i..4i+3 = weights 8i..8i+7 (low nibble first)
      const uint32_t w = u.c[i] ^ 0x88888888u;
      uint32_t lo = w & 0x0f0f0f0fu, hv = (w >> 4) & 0x0f0f0f0fu;
      // Opaque to the optimizer, so each byte converts with one
      // v_cvt_f32_ubyte{0..3} instead of a bit-field extract and a convert.
      asm volatile("" : "+v"(lo), "+v"(hv));
      const uint4 xv = xp[i];
      const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float c0 = float((lo >> (8 * q)) & 0xffu);
        const float c1 = float((hv >> (8 * q)) & 0xffu);
        const fl2 wv = {fmaf(s, c0, n8), fmaf(s, c1, n8)};
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_convertvector(wv, bf2),
                                              __builtin_bit_cast(bf2, xw[q]), acc, false);
      }
    }
  } else {
    const float s = f16_to_f32(u.s);
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // words 2i, 2i+1: weights 8i..8i+7
      const uint4 xv = xp[i];
      const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t w = u.c[2 * i + (q >> 1)];
        const int c0 = __builtin_amdgcn_sbfe(int(w), 16 * (q & 1), 8);
        const int c1 = __builtin_amdgcn_sbfe(int(w), 16 * (q & 1) + 8, 8);
        const fl2 wv = {float(c0) * s, float(c1) * s};
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_convertvector(wv, bf2),
                                              __builtin_bit_cast(bf2, xw[q]), acc, false);
      }
    }
  }
}

template <DKind K, bool Paired, int WS>
__global__ __launch_bounds__(256) void decode_dense_kernel(
    const uint8_t* __restrict__ codes_a, const uint8_t* __restrict__ scales_a,
    const uint8_t* __restrict__ codes_b, const uint8_t* __restrict__ scales_b,
    const uint16_t* __restrict__ x, uint32_t k, uint32_t pk, uint32_t n, uint32_t strips,
    void* out_a, void* out_b, const float* res_a, const float* res_b, int epi) {
  using G = DGeom<K>;
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int SPB = 4 / WS;
  uint32_t* xs = reinterpret_cast<uint32_t*>(smem);
  float* red = reinterpret_cast<float*>(smem + size_t(pk) * 2);
  const uint32_t tiles_k = pk / 256;
  {
    uint16_t* x16 = reinterpret_cast<uint16_t*>(smem);
    for (uint32_t i = threadIdx.x; i < pk; i += 256) x16[i] = i < k ? x[i] : uint16_t(0);
  }
  __syncthreads();

  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t ks = wave % WS;
  const uint32_t strip = blockIdx.x * SPB + wave / WS;
  const bool live = strip < strips;
  // this lane's row in the strip and K offset within a unit
  const uint32_t r = K == DKind::Q4 ? (lane >> 2) & 7u : lane >> 3;
  const uint32_t koff = K == DKind::Q4 ? (lane >> 5) * 256 + (lane & 3u) * 64 : (lane & 7u) * 32;
  const uint32_t units = tiles_k / G::kTilesPerUnit;
  const bool tail = K == DKind::Q4 && (tiles_k & 1u) && ks == WS - 1;
  const uint32_t u0 = uint32_t(uint64_t(units) * ks / WS);
  const uint32_t u1 = uint32_t(uint64_t(units) * (ks + 1) / WS);

  float acc_a = 0.f, acc_b = 0.f;
  if (live) {
    const size_t tbase = size_t(strip) * tiles_k;
    // double-buffered: unit u+1 is in flight while unit u is consumed
    DUnit<K> A[2], B[Paired ? 2 : 1];
    uint32_t u = u0;
    if (u < u1) {
      load_unit<K>(codes_a, scales_a, tbase + u * G::kTilesPerUnit, lane, false, A[0]);
      if constexpr (Paired) load_unit<K>(codes_b, scales_b, tbase + u * G::kTilesPerUnit, lane, false, B[0]);
    }
    for (; u + 2 <= u1; u += 2) {
      load_unit<K>(codes_a, scales_a, tbase + (u + 1) * G::kTilesPerUnit, lane, false, A[1]);
      if constexpr (Paired) load_unit<K>(codes_b, scales_b, tbase + (u + 1) * G::kTilesPerUnit, lane, false, B[1]);
      consume_unit<K>(A[0], u * 256 * G::kTilesPerUnit + koff, xs, acc_a);
      if constexpr (Paired) consume_unit<K>(B[0], u * 256 * G::kTilesPerUnit + koff, xs, acc_b);
      if (u + 2 < u1) {
        load_unit<K>(codes_a, scales_a, tbase + (u + 2) * G::kTilesPerUnit, lane, false, A[0]);
        if constexpr (Paired) load_unit<K>(codes_b, scales_b, tbase + (u + 2) * G::kTilesPerUnit, lane, false, B[0]);
      }
      consume_unit<K>(A[1], (u + 1) * 256 * G::kTilesPerUnit + koff, xs, acc_a);
      if constexpr (Paired) consume_unit<K>(B[1], (u + 1) * 256 * G::kTilesPerUnit + koff, xs, acc_b);
    }
    if (u < u1) {
      consume_unit<K>(A[0], u * 256 * G::kTilesPerUnit + koff, xs, acc_a);
      if constexpr (Paired) consume_unit<K>(B[0], u * 256 * G::kTilesPerUnit + koff, xs, acc_b);
    }
    if (tail) {  // odd last Q4 tile: lanes of the first tile of the pair only
      const uint32_t t = tiles_k - 1;
      load_unit<K>(codes_a, scales_a, tbase + t, lane, true, A[0]);
      if (lane < 32) consume_unit<K>(A[0], t * 256 + koff, xs, acc_a);
      if constexpr (Paired) {
        load_unit<K>(codes_b, scales_b, tbase + t, lane, true, B[0]);
        if (lane < 32) consume_unit<K>(B[0], t * 256 + koff, xs, acc_b);
      }
    }
  }
  // row partials: Q4 lanes {4r..4r+3, 32+4r..32+4r+3}; Q8/BF16 lanes 8r..8r+7
  constexpr int kX3 = K == DKind::Q4 ? 32 : 4;
  acc_a += __shfl_xor(acc_a, 1);
  acc_a += __shfl_xor(acc_a, 2);
  acc_a += __shfl_xor(acc_a, kX3);
  if constexpr (Paired) {
    acc_b += __shfl_xor(acc_b, 1);
    acc_b += __shfl_xor(acc_b, 2);
    acc_b += __shfl_xor(acc_b, kX3);
  }
  const uint32_t row = strip * 8 + r;
  const bool writer = K == DKind::Q4 ? (lane & 35u) == 0 : (lane & 7u) == 0;
  if constexpr (WS > 1) {
    if (writer) {
      red[(wave * 2 + 0) * 8 + r] = acc_a;
      red[(wave * 2 + 1) * 8 + r] = acc_b;
    }
    __syncthreads();
    if (ks != 0) return;
    acc_a = acc_b = 0.f;
#pragma unroll
    for (int qq = 0; qq < WS; ++qq) {
      acc_a += red[((wave + qq) * 2 + 0) * 8 + r];
      acc_b += red[((wave + qq) * 2 + 1) * 8 + r];
    }
  }
  if (!live || !writer || row >= n) return;
  if (Paired && epi == QW38_DECODE_SWIGLU_BF16) {
    static_cast<uint16_t*>(out_a)[row] = f32_to_bf16_rne(silu(acc_a) * acc_b);
    return;
  }
  epilogue(epi, out_a, res_a, row, acc_a);
  if constexpr (Paired) epilogue(epi, out_b, res_b, row, acc_b);
}

template <DKind K, bool Paired>
hipError_t launch_dense_ws(const WeightView& a, const WeightView* b, const uint16_t* x, void* oa,
                           void* ob, const float* ra, const float* rb, int epi, hipStream_t s) {
  const uint32_t strips = a.pn / 8, tiles_k = a.pk / 256;
  const uint64_t strip_bytes = uint64_t(tiles_k) * DGeom<K>::kTileBytes;
  // enough waves in flight: split K when there are few strips of long K
  int ws = 1;
  if (strips < 6144 && strip_bytes >= 8192) ws = 2;
  if (strips < 1536 && strip_bytes >= 16384) ws = 4;
  const size_t lds = size_t(a.pk) * 2 + 4 * 2 * 8 * 4;
  const uint8_t* cb = b ? b->codes : nullptr;
  const uint8_t* sb = b ? b->scales : nullptr;
#define QW38_DENSE_LAUNCH(WSV)                                                                  \
  hipLaunchKernelGGL((decode_dense_kernel<K, Paired, WSV>),                                     \
                     dim3((strips + (4 / WSV) - 1) / (4 / WSV)), dim3(256), lds, s, a.codes,     \
                     a.scales, cb, sb, x, a.k, a.pk, a.n, strips, oa, ob, ra, rb, epi)
  if (ws == 4) QW38_DENSE_LAUNCH(4);
  else if (ws == 2) QW38_DENSE_LAUNCH(2);
  else QW38_DENSE_LAUNCH(1);
#undef QW38_DENSE_LAUNCH
  return hipGetLastError();
}

template <DKind K>
hipError_t launch_dense_kind(const WeightView& a, const WeightView* b, const uint16_t* x, void* oa,
                             void* ob, const float* ra, const float* rb, int epi, hipStream_t s) {
  return b ? launch_dense_ws<K, true>(a, b, x, oa, ob, ra, rb, epi, s)
           : launch_dense_ws<K, false>(a, b, x, oa, ob, ra, rb, epi, s);
}

}  // namespace

hipError_t launch_decode_dense(const WeightView& a, const WeightView* b, const uint16_t* x,
                               void* out_a, void* out_b, const float* res_a, const float* res_b,
                               int epilogue, hipStream_t s) {
  switch (a.layout) {
    case QW38_DECODE_LAYOUT_Q4G64_V0:
    case QW38_DECODE_LAYOUT_Q4G64_CANDIDATE_V1:
      return launch_dense_kind<DKind::Q4>(a, b, x, out_a, out_b, res_a, res_b, epilogue, s);
    case QW38_DECODE_LAYOUT_Q8G32_V0:
    case QW38_DECODE_LAYOUT_Q8G32_CANDIDATE_V1:
      return launch_dense_kind<DKind::Q8>(a, b, x, out_a, out_b, res_a, res_b, epilogue, s);
    case QW38_DECODE_LAYOUT_BF16_DENSE_TILE_V0:
      return launch_dense_kind<DKind::Bf16>(a, b, x, out_a, out_b, res_a, res_b, epilogue, s);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace qw38hip
