// Prefill MMQ for Q4_K layout 0x020D with direct global->LDS staging: the
// 256 x 128 tile of mmq_kernel (q4k_mmq.hip), restructured so that no VALU
// work and no VGPRs go into moving operands.
//
// Per-(row, token) arithmetic is that of mmq_kernel, operation for operation
// (cuda/q4k_q8.cu:140,245 reassociated as described there): one
// v_mfma_f32_16x16x32_f16 per K32 group gives P = s * dot exactly (A = s * w
// <= 945, B = z, every partial sum an integer below 2^24), X = a' P0 then
// X = fma(a', P, X) over the super-block's groups in order, the min term Y
// from two 16x16x16 MFMAs on the same hi / lo operands, acc = fma(-dmin, Y,
// fma(d, X, acc)), and out = acc * (1 / ts) (+ residual). The outputs are
// therefore bitwise equal to every mmq_kernel tile shape.
//
// What differs is the data movement:
// - A pre-pass (mmq_dma_prep_kernel) writes the activations once per call as
//   FP16 codes in the B-fragment order of the tile (chunk-major per K step, so
//   each 1 KB wave copy is one contiguous run), plus per (token, super-block)
//   the scaled a' = a * ts, the min-term operand hi / lo and 1 / ts. The
//   per-token scale ts is computed once there instead of in every block.
// - The block's 256 weight rows arrive as raw 0x020D bytes (1 KB per 8-row
//   tile and super-block, 16-byte chunks XOR-swizzled within a row so the
//   fragment reads are conflict-free) and each wave owns 32 rows x all 128 tokens: it
//   dequantizes its own A fragments straight from the raw bytes, so A never
//   makes an FP16 round trip through LDS.
// - An opt-in int8 form of the 256 x 128 tile (QW38_MMQ_I8=1) runs the same
//   arithmetic on v_mfma_i32_16x16x32_i8 (see mmq_dma_kernel's I8).
// - All staging is global_load_lds_dwordx4 (no VGPRs, no VALU). A ring of four
//   K-step slots for B and two super-block slots for A and the token data is
//   filled two steps ahead; one barrier per pair of K steps, with explicit
//   vmcnt waits (each wave waits for its own copies, the barrier publishes
//   them).
#include <algorithm>
#include <cstdlib>

#include "common.hpp"

namespace qw38hip {
namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));

// The pre-pass writes the activations in blocks of kPB = 128 tokens. Its token
// data block per (token block, super-block) is a' as [8 groups][128 tokens]
// fp32, then per token 32 B of min-term operands: hi of groups 0-3, lo of
// groups 0-3, hi of groups 4-7, lo of groups 4-7 (FP16), so a lane reads its
// hi and lo K-quarter with one 16-byte read.
constexpr uint32_t kPB = 128, kTSlot = 8192, kTokU = 4096;

// Tile geometry of the main kernel: NW waves of 32 rows x NJ 16-token tiles;
// 256 x 128 (NW = 8, NJ = 8) for the large grids, 128 x 32 (NW = 4, NJ = 2)
// for the tail rows and small M. LDS: a B ring of 4 K steps (BT tokens x
// 64 K, FP16), two super-block slots of raw codes (BR x 128 B), and two of
// metadata (BR x 16 B) + token data (a' [8][BT] fp32, min-term operands
// [BT][32 B]); metadata and token data of one super-block share a region
// (the compiler tracks at most eight regions of copies in flight).
template <int NW, int NJ, bool I8 = false>
struct Geo {
  static constexpr uint32_t BR = 32 * NW, BT = 16 * NJ;
  // B of one K step: 64 codes per token, FP16 (int8 in the I8 form)
  static constexpr uint32_t BSL = BT * (I8 ? 64 : 128), ASL = BR * 128, MSL = BR * 16, TSL = BT * 64;
  static constexpr uint32_t OffA = 4 * BSL, OffM = OffA + 2 * ASL, MTS = MSL + TSL;
  static constexpr uint32_t Lds = OffM + 2 * MTS;  // 155648 B for 256 x 128, 57344 B for 128 x 32
  static constexpr uint32_t TokU = 32 * BT;         // min-term operands in the tile's token data
};

__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }

// One 16-byte direct global->LDS copy per active lane: lane l's bytes land at
// lds + 16 l (lds wave-uniform).
__device__ __forceinline__ void dma16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

// Wait until at most N of this wave's vector memory operations are
// outstanding, then the workgroup barrier. The memory clobber keeps the
// compiler from moving LDS reads of the next step above it.
template <int N>
__device__ __forceinline__ void wait_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Calls f with the eight LDS regions of the tile (B step slots 0-3, A code
// super-block slots 0-1, metadata + token-data super-block slots 0-1) as pairwise disjoint
// __restrict__ pointers. Every LDS access of the main loop goes through them:
// that is what lets the compiler see that a copy in flight into one slot does
// not write the slot being read, so it adds no wait for the copies before
// each LDS read (the ring's waits are explicit, see wait_barrier).
template <class F>
__device__ __attribute__((always_inline)) inline void regions(
    uint8_t* __restrict__ b0, uint8_t* __restrict__ b1, uint8_t* __restrict__ b2, uint8_t* __restrict__ b3,
    uint8_t* __restrict__ a0, uint8_t* __restrict__ a1, uint8_t* __restrict__ mt0, uint8_t* __restrict__ mt1,
    F&& f) {
  f(b0, b1, b2, b3, a0, a1, mt0, mt1);
}

// A 16-byte LDS read that completes inside the asm statement (its own
// lgkmcnt wait), for reads the compiler would otherwise order behind every
// copy in flight.
__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
  const auto* lp = (__attribute__((address_space(3))) const uint8_t*)(p);
  return uint32_t(reinterpret_cast<uintptr_t>(lp));
}
__device__ __forceinline__ uint4 lds_read16_sync(const uint8_t* p) {
  uint4 v;
  const uint32_t a = lds_addr(p);
  asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
  return v;
}

// ---- pre-pass ----
// bq: [tb][step][chunk 8][token 128] 16-byte entries; chunk c = gsel * 4 + lk
//     holds the codes 32 g + 8 lk + {0, 2, 4, 6, 1, 3, 5, 7} of group
//     g = 2 step + gsel as FP16 (the slot order the A fragments unpack to).
// tq: [tb][kb] token data blocks (a' at 0, min-term operands at kTokU).
// ti: [mp] 1 / ts. Tokens m .. mp - 1 get zero codes and data, ti = 1.
// Block (x, y) covers tokens 64 x .. 64 x + 63. y < kbs: the codes of
// super-block y, transposed through LDS (row reads of 256 B per token, then
// each wave store one contiguous 1 KB run: 64 tokens x 16 B of one chunk).
// y = kbs .. kbs + 15: the token data (Q4_K: four tokens per block, one per
// wave; Q6_K: 64 tokens per block, lane = token).
__global__ __launch_bounds__(256) void mmq_dma_prep_kernel(const int8_t* __restrict__ xc,
                                                           const float* __restrict__ xa,
                                                           const int32_t* __restrict__ xs, uint32_t m,
                                                           uint32_t pk, uint8_t* __restrict__ bq,
                                                           uint8_t* __restrict__ tq, float* __restrict__ ti,
                                                           bool unit_scale, bool int8_b) {
  const uint32_t groups = pk / 32, kbs = pk / 256, steps = kbs * 4;
  const uint32_t t0 = blockIdx.x * 64, tid = threadIdx.x, lane = tid & 63u, w = tid >> 6;
  if (blockIdx.y < kbs) {
    const uint32_t kb = blockIdx.y;
    __shared__ uint32_t rows[64][65];  // 64 tokens x 256 codes (+1 dword pad)
#pragma unroll
    for (uint32_t r = 0; r < 4; ++r) {  // 16 tokens per pass: 16 threads x 16 B per token
      const uint32_t tl = r * 16 + tid / 16, part = tid % 16, t = t0 + tl;
      // unconditional load (clamped token), then a select: a conditional load
      // becomes a branch with its own wait
      uint4 v = *reinterpret_cast<const uint4*>(xc + size_t(min(t, m - 1)) * pk + kb * 256 + part * 16);
      if (t >= m) v = make_uint4(0u, 0u, 0u, 0u);
      rows[tl][part * 4] = v.x;
      rows[tl][part * 4 + 1] = v.y;
      rows[tl][part * 4 + 2] = v.z;
      rows[tl][part * 4 + 3] = v.w;
    }
    __syncthreads();
    const h2 off = {_Float16(-1152.f), _Float16(-1152.f)};
    const uint32_t t = t0 + lane, tb = t / kPB, tl = t % kPB;
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
      const uint32_t ch = w * 8 + i;  // 8-code chunk of the super-block (0..31)
      const uint32_t g = kb * 8 + ch / 4, lk = ch % 4, st = g / 2, c = (g % 2) * 4 + lk;
      if (int8_b) {  // the int8 form: the same slot order, 8 B per (chunk, token)
        const uint32_t z0 = rows[lane][ch * 2], z1 = rows[lane][ch * 2 + 1];
        *reinterpret_cast<uint2*>(bq + ((size_t(tb) * steps + st) * 8 + c) * (kPB * 8) + tl * 8) =
            make_uint2(perm(z1, z0, 0x06040200u), perm(z1, z0, 0x07050301u));  // z0 z2 z4 z6 | z1 z3 z5 z7
        continue;
      }
      const uint32_t u0 = rows[lane][ch * 2] ^ 0x80808080u, u1 = rows[lane][ch * 2 + 1] ^ 0x80808080u;
      uint4 o;
      o.x = as_u32(as_h2(perm(0x64646464u, u0, 0x04020400u)) + off);  // z0, z2
      o.y = as_u32(as_h2(perm(0x64646464u, u1, 0x04020400u)) + off);  // z4, z6
      o.z = as_u32(as_h2(perm(0x64646464u, u0, 0x04030401u)) + off);  // z1, z3
      o.w = as_u32(as_h2(perm(0x64646464u, u1, 0x04030401u)) + off);  // z5, z7
      *reinterpret_cast<uint4*>(bq + ((size_t(tb) * steps + st) * 8 + c) * (kPB * 16) + tl * 16) = o;
    }
    return;
  }
  // token data: ts = 2^e by mmq_kernel's rule (max_g |a| 2^12 ts in [2^13, 2^14)).
  // Loads are unconditional (clamped token) with a select after: a
  // conditional load becomes a branch with its own wait.
  const uint32_t j = blockIdx.y - kbs;
  if (!unit_scale) {
    // Q4_K: one wave per token (block j: tokens 4 j .. 4 j + 3), lanes over
    // the token's groups (7.4 us at M = 512, K = 5120)
    const uint32_t t = t0 + j * 4 + w, tb = t / kPB, tl = t % kPB, tc = min(t, m - 1);
    const bool real = t < m;
    float mx = 0.f;
    for (uint32_t g = lane; g < groups; g += 64) mx = fmaxf(mx, fabsf(xa[size_t(tc) * groups + g]));
#pragma unroll
    for (int sh = 32; sh >= 1; sh /= 2) mx = fmaxf(mx, __shfl_xor(mx, sh));
    const int ex = int(__float_as_uint(mx) >> 23);  // 0 for zero/subnormal, 255 for NaN/inf
    const int se = min(max(255 - ex, 1), 253);
    const float ts = __uint_as_float(uint32_t(se) << 23);
    if (lane == 0) ti[t] = real ? __uint_as_float(uint32_t(254 - se) << 23) : 1.f;
    for (uint32_t g = lane; g < groups; g += 64) {
      uint8_t* base = tq + (size_t(tb) * kbs + g / 8) * kTSlot;
      const uint32_t g8 = g % 8;
      const float av = xa[size_t(tc) * groups + g] * ts;
      const float v = av * float(xs[size_t(tc) * groups + g]);
      const _Float16 hv = _Float16(v);
      *reinterpret_cast<float*>(base + (g8 * kPB + tl) * 4) = real ? av : 0.f;
      // per token: hi of groups 0-3, lo of 0-3, hi of 4-7, lo of 4-7
      const uint32_t hpos = (g8 / 4) * 16 + (g8 % 4) * 2;
      *reinterpret_cast<_Float16*>(base + kTokU + tl * 32 + hpos) = real ? hv : _Float16(0);
      *reinterpret_cast<_Float16*>(base + kTokU + tl * 32 + hpos + 8) = real ? _Float16(v - float(hv)) : _Float16(0);
    }
    return;
  }
  // Q6_K (unit_scale: ts = 1, a' = a; its kernel reads no min-term
  // operands): wave w of block j writes the a' of super-blocks kb = 4 j + w,
  // 4 j + w + 64, ... with lane = token, coalesced per group (7.5 us at
  // M = 512, K = 17408, against 9.9 us with the Q4_K order's scattered stores)
  const uint32_t t = t0 + lane, tb = t / kPB, tl = t % kPB, tc = min(t, m - 1);
  const bool real = t < m;
  if (j == 0 && w == 0) ti[t] = 1.f;
  for (uint32_t kb = 4 * j + w; kb < kbs; kb += 64) {
    float* base = reinterpret_cast<float*>(tq + (size_t(tb) * kbs + kb) * kTSlot);
#pragma unroll
    for (uint32_t g8 = 0; g8 < 8; ++g8) {
      const float av = xa[size_t(tc) * groups + kb * 8 + g8];
      base[g8 * kPB + tl] = real ? av : 0.f;
    }
  }
}

// ---- main kernel: one 256 x 128 tile per block, 8 waves of 32 rows x 128 tokens ----
// Glu (fused gate + up, features [row0, row0 + 128) per tile): waves 0-3
// hold the gate rows of the tile's 128 features, waves 4-7 the up rows of the
// same features (codes2 / meta2); the epilogue applies SwiGLU -> BF16 -> Q8
// per K32 feature group with mmq_kernel's Glu arithmetic, so the codes equal
// swiglu_q8 of the two separate projections bit for bit.
struct GluDma {
  const uint8_t* codes2;
  const uint8_t* meta2;
  int8_t* qc;
  float* qa;
  int32_t* qs;
  int* failure;
};

// I8 (256 x 128, unfused; opt-in, QW38_MMQ_I8=1): the same per-(row, token)
// operations on the int8 matrix cores. The A operand is the raw codes (no
// dequantization), B the pre-pass's int8 codes in the same slot order, one
// v_mfma_i32_16x16x32_i8 per (row tile, token tile, group) gives the exact
// dot, and P = f32(s * dot) -- the value the FP16 form's MFMA returns -- goes
// into the same X chain, so the outputs are the same bits. It costs a
// multiply and a convert per output and group beyond the FP16 form.
template <int NW, int NJ, bool Glu, bool I8 = false>
__global__ __launch_bounds__(NW * 64) void mmq_dma_kernel(
    const uint8_t* __restrict__ codes, const uint8_t* __restrict__ meta, uint32_t n, uint32_t pn,
    uint32_t kbs, const uint8_t* __restrict__ bq, const uint8_t* __restrict__ tq,
    const float* __restrict__ ti, uint32_t m, float* __restrict__ out, const float* __restrict__ residual,
    uint32_t row_begin, uint32_t row_blocks, uint32_t tok_blocks, GluDma glu) {
  using G = Geo<NW, NJ, I8>;
  static_assert(!I8 || (!Glu && NJ == 8), "int8 form: the unfused 256 x 128 tile");
  constexpr uint32_t BR = G::BR, BT = G::BT, NH = NW / 2;
  extern __shared__ __align__(16) uint8_t lds[];
  const uint32_t tiles_n = row_blocks * tok_blocks;
  const uint32_t tile = (tiles_n % 8 == 0) ? (blockIdx.x % 8) * (tiles_n / 8) + blockIdx.x / 8 : blockIdx.x;
  const uint32_t rb = tile / tok_blocks, tb = tile % tok_blocks;
  constexpr uint32_t HR = Glu ? BR / 2 : BR;  // output rows (features) per tile
  const uint32_t row0 = row_begin + rb * HR;
  const uint32_t pb = tb * BT / kPB, toff = tb * BT % kPB;  // pre-pass token block and offset
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // scalar
  // the wave's 32 weight rows: first row and source arrays (wave-uniform)
  const uint32_t wrow0 = Glu ? row0 + (wave % NH) * 32 : row0 + wave * 32;
  const uint8_t* const wcodes = (Glu && wave >= NH) ? glu.codes2 : codes;
  const uint8_t* const wmeta = (Glu && wave >= NH) ? glu.meta2 : meta;
  const uint32_t lr = lane & 15u, lk = lane >> 4;
  const uint32_t steps = kbs * 4;
  const uint32_t last8 = pn / 8 - 1;

  // ---- copy issue (every wave issues 6 copies per super-block and 2 per K
  // step; past the end they re-read the last data into a slot
  // nobody reads, so the vmcnt arithmetic never changes) ----
  // A codes: block-local row R is 128 LDS bytes; within it, chunk position p
  // holds the row's chunk p ^ ((R / 2) % 8), so the fragment reads of 16
  // consecutive rows hit distinct banks. Copy u (0..3) of wave w is 8-row
  // tile T = 4 w + u: 1 KB contiguous in 0x020D, with lane l reading row
  // l / 8, chunk (l % 8) ^ (4 (T % 2) + l / 16) % 8 -- two lane offsets.
  // Metadata: the wave's 32 rows, 16 B each, half a wave copy (lane l < 32:
  // row l % 8 of the wave's 8-row tile l / 8).
  const uint32_t a_off0 = (lane >> 3) * 128 + (((lane & 7u) ^ ((lane >> 4) & 7u)) * 16);
  const uint32_t a_off1 = (lane >> 3) * 128 + (((lane & 7u) ^ ((4u + (lane >> 4)) & 7u)) * 16);
  auto issue_super = [&](uint32_t kb_in, uint8_t* wA, uint8_t* wM, uint8_t* wT) __attribute__((always_inline)) {
    const uint32_t kb = min(kb_in, kbs - 1);
#pragma unroll
    for (uint32_t u = 0; u < 4; ++u) {
      const uint32_t T = wave * 4 + u;
      const uint32_t r8 = min(wrow0 / 8 + u, last8);
      dma16(wcodes + ((r8 * kbs + kb) * 1024 + (u % 2 ? a_off1 : a_off0)), wA + T * 1024);
    }
    {
      const uint32_t r8 = min(wrow0 / 8 + ((lane & 31u) >> 3), last8);
      if (lane < 32) dma16(wmeta + ((r8 * kbs + kb) * 128 + (lane & 7u) * 16), wM + wave * 512);
    }
    {  // token data: 16-byte LDS positions p = P wave + lane of the tile's
       // a' [8][BT] then min-term operands [BT][32 B], gathered from the
       // pre-pass block at token offset toff
      constexpr uint32_t P = 4 * BT / NW;  // positions per wave (<= 64)
      const uint32_t pos = P * wave + lane;
      const uint8_t* blk = tq + (uint64_t(pb) * kbs + kb) * kTSlot;
      const uint8_t* src = pos < 2 * BT ? blk + (pos / (BT / 4)) * (kPB * 4) + (toff + (pos % (BT / 4)) * 4) * 4
                                        : blk + kTokU + (toff + (pos - 2 * BT) / 2) * 32 + ((pos - 2 * BT) % 2) * 16;
      if (P == 64 || lane < P) dma16(src, wT + P * wave * 16);
    }
  };
  // B of K step s: LDS [8 chunks][BT tokens][16 B]; wave w copies 1 KB runs
  // kc = CPW w .. CPW w + CPW - 1 of the slot (lane l: position 64 kc + l =
  // chunk, token), gathered from the pre-pass block's chunk rows.
  auto issue_step = [&](uint32_t s_in, uint8_t* wB) __attribute__((always_inline)) {
    constexpr uint32_t units = BT / 8, CPW = units / NW;  // 1 KB copies per step; per wave
    const uint32_t s = min(s_in, steps - 1);
    if constexpr (I8) {  // [8 chunks][BT tokens][8 B]: 64 16-byte positions per wave
      static_assert(BT * 4 == 64 * NW, "int8 B copy share");
      const uint8_t* row8 = bq + (uint64_t(pb) * steps + s) * 8 * (kPB * 8);
      const uint32_t pos = wave * 64 + lane, c = pos / (BT / 2), tp = (pos % (BT / 2)) * 2;
      dma16(row8 + c * (kPB * 8) + (toff + tp) * 8, wB + wave * 1024);
      return;
    }
    const uint8_t* row = bq + (uint64_t(pb) * steps + s) * 8 * (kPB * 16);
    if constexpr (CPW >= 1) {
#pragma unroll
      for (uint32_t k = 0; k < CPW; ++k) {
        const uint32_t pos = (CPW * wave + k) * 64 + lane, c = pos / BT, t = pos % BT;
        dma16(row + c * (kPB * 16) + (toff + t) * 16, wB + (CPW * wave + k) * 1024);
      }
    } else if (wave < units) {  // fewer units than waves (16-token tiles)
      const uint32_t pos = wave * 64 + lane, c = pos / BT, t = pos % BT;
      dma16(row + c * (kPB * 16) + (toff + t) * 16, wB + wave * 1024);
    }
  };

  float acc[2][NJ][4], X[2][NJ][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[i][j][v] = 0.f;

  // all ones in lanes lk < 2 (K 0..7 of the min-term MFMA), zero in the
  // padding lanes; opaque, so the compiler keeps an AND instead of branching
  uint32_t ymask = lk < 2 ? ~0u : 0u;
  asm volatile("" : "+v"(ymask));
  // per super-block row data of this lane's A rows (32 wave + 16 i + lr)
  uint32_t S[2][2];  // scale bytes of groups 0-3 and 4-7
  half4 mf[2];       // min-term A operand (m of groups 4 lk .. 4 lk + 3; zero for lk >= 2)
  // I8: the 6-bit scales of this lane's output rows 32 wave + 16 i + 4 lk + v,
  // groups 0-3 and 4-7 as bytes
  uint32_t Sx[I8 ? 2 : 1][I8 ? 4 : 1][2];

  auto compute = [&](auto qc, const uint8_t* Bs, const uint8_t* As, const uint8_t* Ms, const uint8_t* Ts) __attribute__((always_inline)) {
    constexpr uint32_t q = decltype(qc)::value;
    if constexpr (q == 0) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint4 mw = lds_read16_sync(Ms + (wave * 32 + i * 16 + lr) * 16);
        S[i][0] = mw.y & 0x3f3f3f3fu;
        S[i][1] = (mw.w & 0x0f0f0f0fu) | ((mw.y >> 2) & 0x30303030u);
        const uint32_t mlo = mw.z & 0x3f3f3f3fu;
        const uint32_t mhi = ((mw.w >> 4) & 0x0f0f0f0fu) | ((mw.z >> 2) & 0x30303030u);
        const uint32_t mm = lk == 0 ? mlo : mhi;
        const h2 k1024 = {_Float16(-1024.f), _Float16(-1024.f)};
        const h2 m01 = as_h2(perm(0x64646464u, mm, 0x04010400u)) + k1024;
        const h2 m23 = as_h2(perm(0x64646464u, mm, 0x04030402u)) + k1024;
        mf[i] = lk < 2 ? half4{m01.x, m01.y, m23.x, m23.y} : half4{0, 0, 0, 0};
      }
      if constexpr (I8) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          uint4 r4[4];
          const uint32_t a0 = lds_addr(Ms + (wave * 32 + i * 16 + lk * 4) * 16);
          asm volatile(
              "ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:16\n\tds_read_b128 %2, %4 offset:32\n\t"
              "ds_read_b128 %3, %4 offset:48\n\ts_waitcnt lgkmcnt(0)"
              : "=&v"(r4[0]), "=&v"(r4[1]), "=&v"(r4[2]), "=&v"(r4[3])
              : "v"(a0)
              : "memory");
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            Sx[i][v][0] = r4[v].y & 0x3f3f3f3fu;
            Sx[i][v][1] = (r4[v].w & 0x0f0f0f0fu) | ((r4[v].y >> 2) & 0x30303030u);
          }
        }
      }
    }
    // A fragments of row tiles 0, 1 for group g = 2 q + gsel: codes
    // 8 lk .. 8 lk + 7 in slot order {0, 2, 4, 6, 1, 3, 5, 7}, scaled by s
    // exactly ((1024 + c) s - 1024 s = c s <= 945).
    uint32_t wraw[2][2];
#pragma unroll
    for (uint32_t gsel = 0; gsel < 2; ++gsel)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint32_t g = 2 * q + gsel, R = wave * 32 + i * 16 + lr;
        wraw[gsel][i] = *reinterpret_cast<const uint32_t*>(As + R * 128 + ((g ^ (lr >> 1)) * 16) + lk * 4);
      }
    auto dequant = [&](uint32_t gsel, int i) __attribute__((always_inline)) {
      const uint32_t g = 2 * q + gsel, w = wraw[gsel][i];
      const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
      const uint32_t sel = 0x04000400u | ((g & 3u) << 16) | (g & 3u);
      const h2 s2 = as_h2(perm(0x64646464u, S[i][g >> 2], sel)) + h2{_Float16(-1024.f), _Float16(-1024.f)};
      const h2 b2 = s2 * h2{_Float16(-1024.f), _Float16(-1024.f)};
      const h2 p0 = __builtin_elementwise_fma(as_h2(perm(0x64646464u, lo, 0x04010400u)), s2, b2);
      const h2 p1 = __builtin_elementwise_fma(as_h2(perm(0x64646464u, lo, 0x04030402u)), s2, b2);
      const h2 p2 = __builtin_elementwise_fma(as_h2(perm(0x64646464u, hi, 0x04010400u)), s2, b2);
      const h2 p3 = __builtin_elementwise_fma(as_h2(perm(0x64646464u, hi, 0x04030402u)), s2, b2);
      return half8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
    };
    if constexpr (I8) {
      // The FP16 form's pipeline with int8 operands: A = the raw codes in the
      // slot order, B from the int8 pre-pass, D = the exact dot; the scaling
      // takes P = f32(s * D) (s * |D| < 2^22, so exact).
      auto bfrag8 = [&](int u) __attribute__((always_inline)) {
        return *reinterpret_cast<const long*>(Bs + (((u / NJ) * 4 + lk) * BT + (u % NJ) * 16 + lr) * 8);
      };
      auto afac8 = [&](int u) __attribute__((always_inline)) {
        return *reinterpret_cast<const float*>(Ts + ((2 * q + u / NJ) * BT + (u % NJ) * 16 + lr) * 4);
      };
      long a8[2][2];
#pragma unroll
      for (int gs = 0; gs < 2; ++gs)
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const uint32_t w = wraw[gs][i];
          a8[gs][i] = long((uint64_t((w >> 4) & 0x0f0f0f0fu) << 32) | (w & 0x0f0f0f0fu));
        }
      constexpr int kPF8 = 2;
      long b8_[kPF8 + 1];
      float a8q_[kPF8 + 1];
#pragma unroll
      for (int u = 0; u < kPF8; ++u) {
        b8_[u] = bfrag8(u);
        a8q_[u] = afac8(u);
      }
      v4i Dp[2];
      float ap = 0.f;
#pragma unroll
      for (int u = 0; u <= 2 * NJ; ++u) {
        v4i Dc[2];
        float ac = 0.f;
        if (u < 2 * NJ) {
          if (u + kPF8 < 2 * NJ) {
            b8_[(u + kPF8) % (kPF8 + 1)] = bfrag8(u + kPF8);
            a8q_[(u + kPF8) % (kPF8 + 1)] = afac8(u + kPF8);
          }
          const long bf = b8_[u % (kPF8 + 1)];
          ac = a8q_[u % (kPF8 + 1)];
#pragma unroll
          for (int i = 0; i < 2; ++i)
            Dc[i] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a8[u / NJ][i], bf, v4i{0, 0, 0, 0}, 0, 0, 0);
        }
        if (u > 0) {
          const int pu = u - 1, pj = pu % NJ;
          const uint32_t g = 2 * q + pu / NJ;
          const bool first = q == 0 && pu < NJ;  // the super-block's first group
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const int sv = int((Sx[i][v][g >> 2] >> (8 * (g & 3u))) & 0xffu);
              const float P = float(__mul24(sv, Dp[i][v]));
              X[i][pj][v] = first ? ap * P : fmaf(ap, P, X[i][pj][v]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        Dp[0] = Dc[0];
        Dp[1] = Dc[1];
        ap = ac;
      }
    } else {
    // Software pipeline over the step's 2 NJ items u = (group gsel = u / NJ,
    // token tile j = u % NJ): item u's MFMAs are issued after the B fragment
    // and a' of item u + kPF are requested and before item u - 1's results
    // are scaled; sched_barrier keeps the compiler from hoisting further
    // (the register budget is two waves per SIMD).
    constexpr int kPF = 2;
    auto bfrag = [&](int u) __attribute__((always_inline)) {
      return *reinterpret_cast<const half8*>(Bs + (((u / NJ) * 4 + lk) * BT + (u % NJ) * 16 + lr) * 16);
    };
    auto afac = [&](int u) __attribute__((always_inline)) {
      return *reinterpret_cast<const float*>(Ts + ((2 * q + u / NJ) * BT + (u % NJ) * 16 + lr) * 4);
    };
    half8 bq_[kPF + 1];
    float aq_[kPF + 1];
#pragma unroll
    for (int u = 0; u < kPF; ++u) {
      bq_[u] = bfrag(u);
      aq_[u] = afac(u);
    }
    half8 af[2][2];
    af[0][0] = dequant(0, 0);
    af[0][1] = dequant(0, 1);
    f4 Pp[2];
    float ap = 0.f;
#pragma unroll
    for (int u = 0; u <= 2 * NJ; ++u) {
      f4 Pc[2];
      float ac = 0.f;
      if (u < 2 * NJ) {
        if (u + kPF < 2 * NJ) {
          bq_[(u + kPF) % (kPF + 1)] = bfrag(u + kPF);
          aq_[(u + kPF) % (kPF + 1)] = afac(u + kPF);
        }
        if (u == (NJ >= 2 ? NJ - 2 : 0)) af[1][0] = dequant(1, 0);  // the second group's fragments,
        if (u == NJ - 1) af[1][1] = dequant(1, 1);                  // ready before its first item
        const half8 bf = bq_[u % (kPF + 1)];
        ac = aq_[u % (kPF + 1)];
#pragma unroll
        for (int i = 0; i < 2; ++i) Pc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[u / NJ][i], bf, f4{0, 0, 0, 0}, 0, 0, 0);
      }
      if (u > 0) {
        const int pu = u - 1, pj = pu % NJ;
        const bool first = q == 0 && pu < NJ;  // the super-block's first group
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int v = 0; v < 4; ++v) X[i][pj][v] = first ? ap * Pp[i][v] : fmaf(ap, Pp[i][v], X[i][pj][v]);
      }
      __builtin_amdgcn_sched_barrier(0);
      Pp[0] = Pc[0];
      Pp[1] = Pc[1];
      ap = ac;
    }
    }
    // Pin X: otherwise the compiler defers the scaling FMAs and keeps
    // (spills) the MFMA results.
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) asm volatile("" : "+v"(X[i][j][v]));
    // ---- end of super-block: acc += d X - dmin Y ----
    // The epilogue's LDS operands come through completing asm reads (the
    // compiler would otherwise order them behind every copy in flight).
    if constexpr (q == 3) {
      // d, -dmin of output rows 32 wave + 16 i + 4 lk + v
      uint32_t dw[8];
      {
        const uint32_t a0 = lds_addr(Ms + (wave * 32 + lk * 4) * 16);
        asm volatile(
            "ds_read_b32 %0, %8\n\tds_read_b32 %1, %8 offset:16\n\tds_read_b32 %2, %8 offset:32\n\t"
            "ds_read_b32 %3, %8 offset:48\n\tds_read_b32 %4, %8 offset:256\n\tds_read_b32 %5, %8 offset:272\n\t"
            "ds_read_b32 %6, %8 offset:288\n\tds_read_b32 %7, %8 offset:304\n\ts_waitcnt lgkmcnt(0)"
            : "=&v"(dw[0]), "=&v"(dw[1]), "=&v"(dw[2]), "=&v"(dw[3]), "=&v"(dw[4]), "=&v"(dw[5]), "=&v"(dw[6]),
              "=&v"(dw[7])
            : "v"(a0)
            : "memory");
      }
#pragma unroll
      for (int jh = 0; jh < (NJ + 3) / 4; ++jh) {
        // min-term operands of token tiles 4 jh .. 4 jh + 3; lanes lk >= 2
        // (K 8..15, the zero padding) read a valid address and are masked
        uint4 r[4];
        const uint32_t a0 = lds_addr(Ts + G::TokU + (jh * 64 + lr) * 32 + (lk & 1u) * 16);
        if constexpr (NJ % 4 == 0) {
          asm volatile(
              "ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:512\n\tds_read_b128 %2, %4 offset:1024\n\t"
              "ds_read_b128 %3, %4 offset:1536\n\ts_waitcnt lgkmcnt(0)"
              : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
              : "v"(a0)
              : "memory");
        } else if constexpr (NJ == 2) {
          asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %2 offset:512\n\ts_waitcnt lgkmcnt(0)"
                       : "=&v"(r[0]), "=&v"(r[1])
                       : "v"(a0)
                       : "memory");
        } else {
          static_assert(NJ == 1, "token tiles per wave: 1, 2 or a multiple of 4");
          asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(r[0]) : "v"(a0) : "memory");
        }
#pragma unroll
        for (int jj = 0; jj < (NJ < 4 ? NJ : 4); ++jj) {
          const int j = jh * 4 + jj;
          const half4 uh = __builtin_bit_cast(half4, make_uint2(r[jj].x & ymask, r[jj].y & ymask));
          const half4 ul = __builtin_bit_cast(half4, make_uint2(r[jj].z & ymask, r[jj].w & ymask));
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            f4 Y = __builtin_amdgcn_mfma_f32_16x16x16f16(mf[i], uh, f4{0, 0, 0, 0}, 0, 0, 0);
            Y = __builtin_amdgcn_mfma_f32_16x16x16f16(mf[i], ul, Y, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const uint32_t w0 = dw[i * 4 + v];
              acc[i][j][v] = fmaf(-f16_to_f32(w0 >> 16), Y[v], fmaf(f16_to_f32(w0 & 0xffffu), X[i][j][v], acc[i][j][v]));
            }
          }
        }
      }
      // Pin acc: the super-block's epilogue completes here, so X is dead
      // before the next super-block starts it again.
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int v = 0; v < 4; ++v) asm volatile("" : "+v"(acc[i][j][v]));
    }
  };

  using C0 = std::integral_constant<uint32_t, 0>;
  using C1 = std::integral_constant<uint32_t, 1>;
  using C2 = std::integral_constant<uint32_t, 2>;
  using C3 = std::integral_constant<uint32_t, 3>;
  // Step 4 kb + q of super-block kb in LDS slot SB = kb % 2. Steps run in
  // pairs (q = 0, 1 and q = 2, 3) with one barrier per pair: at q = 0 and
  // q = 2 each wave waits for all of its copies (the pair's B slots, issued
  // one pair earlier, and at q = 0 the super-block's data, issued one
  // super-block earlier), the barrier publishes them and retires the previous
  // pair's slots, which are refilled with the next pair (at q = 0 also
  // super-block kb + 1 into slot SB ^ 1).
  auto run = [&](uint8_t* B0, uint8_t* B1, uint8_t* B2, uint8_t* B3, uint8_t* A0, uint8_t* A1, uint8_t* MT0,
                 uint8_t* MT1) __attribute__((always_inline)) {
  uint8_t* const Bsl[4] = {B0, B1, B2, B3};
  uint8_t* const Asl[2] = {A0, A1};
  uint8_t* const Msl[2] = {MT0, MT1};
  uint8_t* const Tsl[2] = {MT0 + G::MSL, MT1 + G::MSL};
  auto step = [&](auto qc, auto sbc, uint32_t kb) __attribute__((always_inline)) {
    constexpr uint32_t q = decltype(qc)::value, SB = decltype(sbc)::value;
    if constexpr (q % 2 == 0) {
      wait_barrier<0>();
      if constexpr (q == 0) issue_super(kb + 1, Asl[SB ^ 1u], Msl[SB ^ 1u], Tsl[SB ^ 1u]);
      issue_step(4 * kb + q + 2, Bsl[(q + 2) & 3u]);
      issue_step(4 * kb + q + 3, Bsl[(q + 3) & 3u]);
    }
    compute(qc, Bsl[q], Asl[SB], Msl[SB], Tsl[SB]);
  };
  auto super_block = [&](uint32_t kb, auto sbc) __attribute__((always_inline)) {
    step(C0{}, sbc, kb);
    step(C1{}, sbc, kb);
    step(C2{}, sbc, kb);
    step(C3{}, sbc, kb);
  };
  // Prologue: super-block 0 and K steps 0, 1 in flight. kbs is even.
  issue_super(0, A0, Msl[0], Tsl[0]);
  issue_step(0, B0);
  issue_step(1, B1);
  for (uint32_t kb = 0; kb < kbs; kb += 2) {
    super_block(kb, C0{});
    super_block(kb + 1, C1{});
  }
  };
  regions(lds, lds + G::BSL, lds + 2 * G::BSL, lds + 3 * G::BSL, lds + G::OffA, lds + G::OffA + G::ASL,
          lds + G::OffM, lds + G::OffM + G::MTS, run);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no copy outlives the block

  if constexpr (Glu) {
    // ---- SwiGLU -> Q8 epilogue (mmq_kernel's Glu arithmetic). The gate
    // waves (the first NW / 2) park their unscaled g in LDS (the ring is free once every wave is
    // past its loop); up wave w holds u of the same features in the same
    // register positions. The wave's K32 feature group of token lr is row
    // tiles 0, 1 of lanes lr + 16 lk: eight values in each of 4 lanes. ----
    __syncthreads();
    float* gl = reinterpret_cast<float*>(lds);  // [HR features][BT tokens]
    const bool gate_wave = wave < NH;
    const uint32_t wq = wave % NH;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint32_t tok = min(tb * BT + j * 16 + lr, m - 1);
      const float inv = ti[tok];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[i][j][v] *= inv;
    }
    if (gate_wave) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int v = 0; v < 4; ++v) gl[(wq * 32 + i * 16 + lk * 4 + v) * BT + j * 16 + lr] = acc[i][j][v];
    }
    __syncthreads();
    if (gate_wave) return;
    const uint32_t groups_out = n / 32;
    const uint32_t f0 = row0 + wq * 32;  // first feature of the group
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint32_t tl = j * 16 + lr, tok = tb * BT + tl;
      float x[8];
      float peak = 0.f;
      int finite = 1;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float g = gl[(wq * 32 + h * 16 + lk * 4 + v) * BT + tl];
          const float y = swiglu_q8_value(g, acc[h][j][v]);
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
    return;
  }
  // ---- store: lane holds rows 4 lk .. 4 lk + 3 of token lr in each tile ----
  const bool vec = (n % 4 == 0) &&
                   ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(residual)) & 15u) == 0;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const uint32_t tok = tb * BT + j * 16 + lr;
    if (tok >= m) continue;
    const float inv = ti[tok];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t r4 = wrow0 + i * 16 + lk * 4;
      if (r4 >= n) continue;
      const size_t o = size_t(tok) * n + r4;
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[i][j][v] *= inv;
      if (vec) {
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
}

// ---- Q6_K (0x0241) direct-copy MMQ ----
// mmq_kernel's Q6_K arithmetic per (row, token), operation for operation:
// P = sum over the K32 group of sc (q - 32) z, exact (A split into FP16
// hi + lo, two chained 16x16x32 MFMAs, every partial sum an integer below
// 2^24), X = a P0 then X = fma(a, P, X) over the super-block's groups,
// acc = fma(d, X, acc), the fixed K segments of q6_seg_kb (a segment's sum
// starts from zero; the caller adds the sums in ascending order), and out =
// acc (+ residual). Each block runs one segment of one tile, so the outputs
// are bitwise equal to mmq_kernel's Q6_K tiles, split or not.
//
// NW waves of 16 rows x 128 tokens (160 x 128 for NW = 10, 80 x 128 for 5).
// Each wave dequantizes its own A fragments from the raw code planes: the
// 0x0241 tile of 8 rows stores a K step's two groups contiguously (256 B of
// low nibbles, 128 B of high pairs), so a wave's codes of one step are one
// 768 B copy. The step ring holds B (16 KB) and the NW waves' codes; a
// super-block slot holds the waves' scales and d and the tokens' a (fp32).
template <int NW, int NJ = 8>
struct Geo6 {
  static constexpr uint32_t BR = 16 * NW, BT = 16 * NJ;
  static constexpr uint32_t BSL = BT * 128, AW = 768, SSL = BSL + NW * AW;  // one K step
  static constexpr uint32_t MW = 288, TSL = 8 * BT * 4, MTS = NW * MW + TSL;  // one super-block
  static constexpr uint32_t OffM = 4 * SSL, Lds = OffM + 2 * MTS;
};

template <class F>
__device__ __attribute__((always_inline)) inline void q6_regions(uint8_t* __restrict__ b0, uint8_t* __restrict__ b1,
                                                                   uint8_t* __restrict__ b2, uint8_t* __restrict__ b3,
                                                                   uint8_t* __restrict__ mt0,
                                                                   uint8_t* __restrict__ mt1, F&& f) {
  f(b0, b1, b2, b3, mt0, mt1);
}

template <int NW, int NJ = 8>
__global__ __launch_bounds__(NW * 64) void q6_mmq_dma_kernel(
    const uint8_t* __restrict__ codes, const uint8_t* __restrict__ meta, uint32_t n, uint32_t pn,
    uint32_t kbs, const uint8_t* __restrict__ bq, const uint8_t* __restrict__ tq, uint32_t m,
    float* __restrict__ out, const float* __restrict__ residual, uint32_t row_blocks, uint32_t tok_blocks,
    uint32_t seg_kb, uint32_t segs, float* __restrict__ part) {
  using G = Geo6<NW, NJ>;
  constexpr uint32_t BT = G::BT;
  extern __shared__ __align__(16) uint8_t lds[];
  const uint32_t tiles_n = row_blocks * tok_blocks;
  // segs > 1: block b runs segment b / tiles_n and writes its sum to part
  const uint32_t sgm = blockIdx.x / tiles_n, bx = blockIdx.x % tiles_n;
  const uint32_t tile = (tiles_n % 8 == 0) ? (bx % 8) * (tiles_n / 8) + bx / 8 : bx;
  const uint32_t rb = tile / tok_blocks, tb = tile % tok_blocks;
  const uint32_t pb = tb * BT / kPB, toff = tb * BT % kPB;  // pre-pass token block and offset
  const uint32_t kb_lo = sgm * seg_kb, kb_hi = min(kbs, kb_lo + seg_kb);
  if (segs > 1) {
    out = part + size_t(sgm) * m * n;
    residual = nullptr;
  }
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t wrow0 = rb * G::BR + wave * 16;
  const uint32_t lr = lane & 15u, lk = lane >> 4;
  const uint32_t steps = kbs * 4, last8 = pn / 8 - 1;
  const uint64_t trows = uint64_t(pn) * kbs;  // tile rows: d follows the 16-byte scale rows

  // ---- copy issue ----
  // Super-block: lanes 0..15 the scale rows of the wave's two 8-row tiles,
  // lanes 16, 17 their d (8 x fp16 each); waves 0 .. BT / 32 - 1 also 1 KB
  // each of the tokens' a [8 groups][BT tokens], gathered from the pre-pass
  // block pb at token offset toff.
  auto issue_super = [&](uint32_t kb_in, uint8_t* MT) __attribute__((always_inline)) {
    const uint32_t kb = min(kb_in, kbs - 1);
    if (lane < 18) {
      const uint32_t t = lane < 16 ? lane >> 3 : lane - 16;
      const uint64_t tr = (uint64_t(min(wrow0 / 8 + t, last8)) * kbs + kb) * 8;
      const uint8_t* src = lane < 16 ? meta + (tr + (lane & 7u)) * 16 : meta + trows * 16 + tr * 2;
      dma16(src, MT + wave * G::MW);
    }
    if (wave < BT / 32) {
      const uint32_t p = wave * 64 + lane, g = p / (BT / 4), tp = p % (BT / 4);
      dma16(tq + (uint64_t(pb) * kbs + kb) * kTSlot + g * (kPB * 4) + (toff + tp * 4) * 4,
            MT + NW * G::MW + wave * 1024);
    }
  };
  // K step s: the wave's codes (lanes 0..31 low nibbles of tiles 0, 1 -- the
  // second tile's 16-byte chunks in the order p ^ 1, so the two tiles'
  // fragment reads use different banks -- lanes 32..47 the high pairs) and B
  // units k = wave, wave + NW, ... of 1 KB (64 tokens of one chunk of the
  // pre-pass block's K step [8 chunks][128 tokens][16 B]).
  auto issue_step = [&](uint32_t s_in, uint8_t* SL) __attribute__((always_inline)) {
    const uint32_t s = min(s_in, steps - 1), kb = s / 4, q = s % 4;
    if (lane < 48) {
      const uint32_t t = lane < 32 ? lane >> 4 : (lane - 32) >> 3;
      const uint8_t* base = codes + (uint64_t(min(wrow0 / 8 + t, last8)) * kbs + kb) * kQ6TileBytes;
      const uint8_t* src = lane < 32 ? base + q * 256 + (((lane & 15u) ^ t) * 16)
                                     : base + kQ6HiPlane + q * 128 + ((lane - 32) & 7u) * 16;
      dma16(src, SL + G::BSL + wave * G::AW);
    }
    const uint8_t* row = bq + (uint64_t(pb) * steps + s) * (8 * kPB * 16);
    constexpr uint32_t units = BT / 8, upc = BT / 64;  // 1 KB units per step, per chunk
#pragma unroll
    for (uint32_t k0 = 0; k0 < units; k0 += NW) {
      const uint32_t k = k0 + wave;
      if (k < units) dma16(row + (k / upc) * (kPB * 16) + (toff + (k % upc) * 64) * 16 + lane * 16, SL + k * 1024);
    }
  };

  float acc[NJ][4], X[NJ][4];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[j][v] = 0.f;
  uint32_t S[4];  // this lane's row: the super-block's 16 scale bytes, each + 128 (xor 0x80)
  // perm selectors of the lane's scale byte 2 gsel + lk / 2 of a step's dword
  const uint32_t sb0 = lk >> 1, sb1 = 2u + (lk >> 1);
  const uint32_t ssel0 = 0x04000400u | (sb0 << 16) | sb0, ssel1 = 0x04000400u | (sb1 << 16) | sb1;
  const uint32_t hsh = (lk & 1u) * 4;  // the lane's 2-bit fields within its high-pair bytes

  auto compute = [&](auto qc, const uint8_t* SL, const uint8_t* MT) __attribute__((always_inline)) {
    constexpr uint32_t q = decltype(qc)::value;
    const uint8_t* Bs = SL;
    const uint8_t* As = SL + G::BSL + wave * G::AW;
    const uint8_t* Ts = MT + NW * G::MW;
    if constexpr (q == 0) {
      const uint4 sw = lds_read16_sync(MT + wave * G::MW + (lr >> 3) * 128 + (lr & 7u) * 16);
      S[0] = sw.x ^ 0x80808080u;
      S[1] = sw.y ^ 0x80808080u;
      S[2] = sw.z ^ 0x80808080u;
      S[3] = sw.w ^ 0x80808080u;
    }
    // A fragments (hi, lo) of group g = 2 q + gsel: codes 8 lk .. 8 lk + 7 of
    // row lr in slot order {0, 2, 4, 6, 1, 3, 5, 7}
    const uint32_t t = lr >> 3, r = lr & 7u;
    uint32_t nib[2], hp[2];
#pragma unroll
    for (uint32_t gsel = 0; gsel < 2; ++gsel) {
      nib[gsel] = *reinterpret_cast<const uint32_t*>(As + t * 256 + (((2 * r + gsel) ^ t) * 16) + lk * 4);
      hp[gsel] = *reinterpret_cast<const uint32_t*>(As + 512 + t * 128 + (2 * r + gsel) * 8 + (lk >> 1) * 4);
    }
    auto dequant = [&](uint32_t gsel, half8& hi, half8& lo) __attribute__((always_inline)) {
      const uint32_t w = nib[gsel], xs = hp[gsel] >> hsh;
      const uint32_t q0 = (w & 0x0f0f0f0fu) | ((xs & 0x03030303u) << 4);         // codes 8 lk + 0..3
      const uint32_t q1 = ((w >> 4) & 0x0f0f0f0fu) | ((xs & 0x0c0c0c0cu) << 2);  // codes 8 lk + 4..7
      const h2 s2 = as_h2(perm(0x64646464u, S[q], gsel ? ssel1 : ssel0)) - h2{_Float16(1152.f), _Float16(1152.f)};
      const h2 k = {_Float16(1056.f), _Float16(1056.f)};  // 1024 + q -> q - 32, exact
      const h2 c0 = as_h2(perm(0x64646464u, q0, 0x04020400u)) - k;  // codes 0, 2
      const h2 c1 = as_h2(perm(0x64646464u, q1, 0x04020400u)) - k;  // 4, 6
      const h2 c2 = as_h2(perm(0x64646464u, q0, 0x04030401u)) - k;  // 1, 3
      const h2 c3 = as_h2(perm(0x64646464u, q1, 0x04030401u)) - k;  // 5, 7
      const h2 h0 = c0 * s2, h1 = c1 * s2, h2_ = c2 * s2, h3 = c3 * s2;  // RN(sc (q - 32))
      const h2 l0 = __builtin_elementwise_fma(c0, s2, -h0), l1 = __builtin_elementwise_fma(c1, s2, -h1);
      const h2 l2 = __builtin_elementwise_fma(c2, s2, -h2_), l3 = __builtin_elementwise_fma(c3, s2, -h3);
      hi = half8{h0.x, h0.y, h1.x, h1.y, h2_.x, h2_.y, h3.x, h3.y};
      lo = half8{l0.x, l0.y, l1.x, l1.y, l2.x, l2.y, l3.x, l3.y};
    };
    constexpr int kPF = 2;
    auto bfrag = [&](int u) __attribute__((always_inline)) {
      return *reinterpret_cast<const half8*>(Bs + (((u / NJ) * 4 + lk) * BT + (u % NJ) * 16 + lr) * 16);
    };
    auto afac = [&](int u) __attribute__((always_inline)) {
      return *reinterpret_cast<const float*>(Ts + ((2 * q + u / NJ) * BT + (u % NJ) * 16 + lr) * 4);
    };
    half8 bq_[kPF + 1];
    float aq_[kPF + 1];
#pragma unroll
    for (int u = 0; u < kPF; ++u) {
      bq_[u] = bfrag(u);
      aq_[u] = afac(u);
    }
    half8 ah[2], al[2];
    dequant(0, ah[0], al[0]);
    f4 Pp;
    float ap = 0.f;
#pragma unroll
    for (int u = 0; u <= int(2 * NJ); ++u) {
      f4 Pc;
      float ac = 0.f;
      if (u < int(2 * NJ)) {
        if (u + kPF < int(2 * NJ)) {
          bq_[(u + kPF) % (kPF + 1)] = bfrag(u + kPF);
          aq_[(u + kPF) % (kPF + 1)] = afac(u + kPF);
        }
        if (u == int(NJ) - 2) dequant(1, ah[1], al[1]);  // the second group's fragments
        const half8 bf = bq_[u % (kPF + 1)];
        ac = aq_[u % (kPF + 1)];
        Pc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[u / NJ], bf, f4{0, 0, 0, 0}, 0, 0, 0);
        Pc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[u / NJ], bf, Pc, 0, 0, 0);
      }
      if (u > 0) {
        const int pu = u - 1, pj = pu % NJ;
        const bool first = q == 0 && pu < int(NJ);  // the super-block's first group
#pragma unroll
        for (int v = 0; v < 4; ++v) X[pj][v] = first ? ap * Pp[v] : fmaf(ap, Pp[v], X[pj][v]);
      }
      __builtin_amdgcn_sched_barrier(0);
      Pp = Pc;
      ap = ac;
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) asm volatile("" : "+v"(X[j][v]));
    if constexpr (q == 3) {  // ---- end of super-block: acc += d X ----
      uint2 dw;
      {
        const uint32_t a0 = lds_addr(MT + wave * G::MW + 256 + lk * 8);
        asm volatile("ds_read_b64 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(dw) : "v"(a0) : "memory");
      }
      const float d[4] = {f16_to_f32(dw.x & 0xffffu), f16_to_f32(dw.x >> 16), f16_to_f32(dw.y & 0xffffu),
                          f16_to_f32(dw.y >> 16)};
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[j][v] = fmaf(d[v], X[j][v], acc[j][v]);
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) asm volatile("" : "+v"(acc[j][v]));
    }
  };

  using C0 = std::integral_constant<uint32_t, 0>;
  using C1 = std::integral_constant<uint32_t, 1>;
  using C2 = std::integral_constant<uint32_t, 2>;
  using C3 = std::integral_constant<uint32_t, 3>;
  // The ring discipline of mmq_dma_kernel: steps in pairs, one barrier per
  // pair after each wave's copies have landed, the next pair's steps (and at
  // q = 0 the next super-block) issued into the slots the barrier retired.
  // Super-block slots alternate from kb_lo; an odd range ends with one
  // super-block in slot 0.
  auto body = [&](uint8_t* B0, uint8_t* B1, uint8_t* B2, uint8_t* B3, uint8_t* MT0, uint8_t* MT1)
                 __attribute__((always_inline)) {
    uint8_t* const Ssl[4] = {B0, B1, B2, B3};
    uint8_t* const Msl[2] = {MT0, MT1};
    auto step = [&](auto qc, auto sbc, uint32_t kb) __attribute__((always_inline)) {
      constexpr uint32_t q = decltype(qc)::value, SB = decltype(sbc)::value;
      if constexpr (q % 2 == 0) {
        wait_barrier<0>();
        if constexpr (q == 0) issue_super(kb + 1, Msl[SB ^ 1u]);
        issue_step(4 * kb + q + 2, Ssl[(q + 2) & 3u]);
        issue_step(4 * kb + q + 3, Ssl[(q + 3) & 3u]);
      }
      compute(qc, Ssl[q], Msl[SB]);
    };
    auto super_block = [&](uint32_t kb, auto sbc) __attribute__((always_inline)) {
      step(C0{}, sbc, kb);
      step(C1{}, sbc, kb);
      step(C2{}, sbc, kb);
      step(C3{}, sbc, kb);
    };
    issue_super(kb_lo, MT0);
    issue_step(4 * kb_lo, B0);
    issue_step(4 * kb_lo + 1, B1);
    uint32_t kb = kb_lo;
    for (; kb + 1 < kb_hi; kb += 2) {
      super_block(kb, C0{});
      super_block(kb + 1, C1{});
    }
    if (kb < kb_hi) super_block(kb, C0{});
  };
  q6_regions(lds, lds + G::SSL, lds + 2 * G::SSL, lds + 3 * G::SSL, lds + G::OffM, lds + G::OffM + G::MTS, body);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no copy outlives the block

  // ---- store: lane holds rows 4 lk .. 4 lk + 3 of token lr in each tile ----
  const bool vec = (n % 4 == 0) &&
                   ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(residual)) & 15u) == 0;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const uint32_t tok = tb * BT + j * 16 + lr, r4 = wrow0 + lk * 4;
    if (tok >= m || r4 >= n) continue;
    const size_t o = size_t(tok) * n + r4;
    if (vec) {
      float4 y = make_float4(acc[j][0], acc[j][1], acc[j][2], acc[j][3]);
      if (residual) {
        const float4 rv = *reinterpret_cast<const float4*>(residual + o);
        y.x += rv.x; y.y += rv.y; y.z += rv.z; y.w += rv.w;
      }
      *reinterpret_cast<float4*>(out + o) = y;
    } else {
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (r4 + v < n) out[o + v] = acc[j][v] + (residual ? residual[o + v] : 0.f);
    }
  }
}

}  // namespace

// Scratch bytes the pre-pass needs for m tokens of padded width pk.
uint64_t mmq_dma_scratch_bytes(uint32_t m, uint32_t pk) {
  const uint64_t mp = (uint64_t(m) + kPB - 1) / kPB * kPB;
  return mp * pk * 2 + mp / kPB * (pk / 256) * kTSlot + mp * 4;
}

namespace {

template <int NW, int NJ, bool I8 = false>
hipError_t launch_dma_tiles(const WeightView& w, const Q8View& x, float* out, const float* residual, hipStream_t s,
                            uint32_t row_begin, uint32_t rows, const uint8_t* bq, const uint8_t* tq,
                            const float* ti, const WeightView* up, const GluDma& g) {
  using G = Geo<NW, NJ, I8>;
  const bool glu = up != nullptr;
  auto kern = mmq_dma_kernel<NW, NJ, false, I8>;
  if constexpr (!I8)
    if (glu) kern = mmq_dma_kernel<NW, NJ, true>;
  if (G::Lds > 64 * 1024) {
    const hipError_t e = set_max_lds(reinterpret_cast<const void*>(kern), int(G::Lds));
    if (e != hipSuccess) return e;
  }
  const uint32_t hr = glu ? G::BR / 2 : G::BR;
  const uint32_t row_blocks = (rows + hr - 1) / hr, tok_blocks = (x.m + G::BT - 1) / G::BT;
  hipLaunchKernelGGL(kern, dim3(row_blocks * tok_blocks), dim3(NW * 64), G::Lds, s, w.codes, w.scales, w.n, w.pn,
                     w.pk / 256, bq, tq, ti, x.m, out, residual, row_begin, row_blocks, tok_blocks, g);
  return hipGetLastError();
}

}  // namespace

// Output rows [0, rows) on 256 x 128 tiles and [rows, tail_end) on 128 x 32
// tiles (tail_nj = 2) or 128 x 16 tiles (tail_nj = 1; tail_end = rows: none) of a Q4_K 0x020D weight for all m tokens,
// after one activation pre-pass; rows a multiple of the big tile height (in
// features for the fused form), tail_end a multiple of the small one or the
// whole weight. scratch holds mmq_dma_scratch_bytes(m, pk). Codes and
// metadata must be 16-byte aligned. up != nullptr: fused gate + up over
// features (w is the gate, up the same geometry), writing the down
// projection's Q8 operand.
hipError_t launch_mmq_dma(const WeightView& w, const Q8View& x, float* out, const float* residual,
                          hipStream_t s, uint32_t rows, uint32_t tail_end, void* scratch, const WeightView* up,
                          int8_t* qc, float* qa, int32_t* qs, int* failure, int tail_nj) {
  const bool glu = up != nullptr;
  // QW38_MMQ_I8=1: the 256 x 128 tiles on the int8 matrix cores (same bits),
  // for unfused calls without a tail (the tail tiles read the FP16 pre-pass)
  static const bool i8_env = [] {
    const char* v = std::getenv("QW38_MMQ_I8");
    return v && std::atoi(v) == 1;
  }();
  const bool i8 = i8_env && !glu && tail_end == rows;
  if (w.layout != QW38_LAYOUT_Q4K_CANDIDATE_V2 || tail_end < rows || tail_end == 0 || x.pk != w.pk ||
      ((reinterpret_cast<uintptr_t>(w.codes) | reinterpret_cast<uintptr_t>(w.scales) |
        reinterpret_cast<uintptr_t>(x.codes) | reinterpret_cast<uintptr_t>(glu ? up->codes : nullptr) |
        reinterpret_cast<uintptr_t>(glu ? up->scales : nullptr)) % 16) != 0)
    return hipErrorInvalidValue;
  if (glu && (up->layout != w.layout || up->pn != w.pn || up->pk != w.pk || w.n % 32 != 0 || !qc || !qa ||
              !qs || !failure))
    return hipErrorInvalidValue;
  if ((w.pk / 256) % 2 != 0) return hipErrorNotReady;  // the main loop runs super-block pairs
  const uint32_t mp = (x.m + kPB - 1) / kPB * kPB;
  uint8_t* bq = static_cast<uint8_t*>(scratch);
  uint8_t* tq = bq + uint64_t(mp) * w.pk * 2;
  float* ti = reinterpret_cast<float*>(tq + uint64_t(mp / kPB) * (w.pk / 256) * kTSlot);
  hipLaunchKernelGGL(mmq_dma_prep_kernel, dim3(mp / 64, w.pk / 256 + 16), dim3(256), 0, s, x.codes, x.scales,
                     x.sums, x.m, x.pk, bq, tq, ti, false, i8);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const GluDma g{glu ? up->codes : nullptr, glu ? up->scales : nullptr, qc, qa, qs, failure};
  if (rows > 0)
    e = i8 ? launch_dma_tiles<8, 8, true>(w, x, out, residual, s, 0, rows, bq, tq, ti, up, g)
           : launch_dma_tiles<8, 8>(w, x, out, residual, s, 0, rows, bq, tq, ti, up, g);
  if (e == hipSuccess && tail_end > rows)
    e = tail_nj == 1 ? launch_dma_tiles<4, 1>(w, x, out, residual, s, rows, tail_end - rows, bq, tq, ti, up, g)
                     : launch_dma_tiles<4, 2>(w, x, out, residual, s, rows, tail_end - rows, bq, tq, ti, up, g);
  return e;
}

}  // namespace qw38hip

namespace qw38hip {

// Q6_K 0x0241 on the direct-copy tiles, NW = 10 (160 x 128, or 160 x 64 with
// nj = 4) or 5 (80 x 128):
// one block per (tile, fixed K segment). With several segments the tokens run
// in chunks of mc (a multiple of 128): the chunk's pre-pass and segment sums
// (one mc x n array per segment) share the scratch, and reduce(part, segs,
// mc, residual, out) adds them in ascending order (+ residual). scratch holds
// q6_mmq_dma_scratch_bytes(mc, n, pk).
uint64_t q6_mmq_dma_scratch_bytes(uint32_t mc, uint32_t n, uint32_t pk) {
  const uint32_t kbs = pk / 256, seg_kb = q6_seg_kb(kbs), segs = (kbs + seg_kb - 1) / seg_kb;
  const uint64_t prep = (mmq_dma_scratch_bytes(mc, pk) + 255) / 256 * 256;
  return prep + (segs > 1 ? uint64_t(segs) * mc * n * 4 : 0);
}

hipError_t launch_q6_mmq_dma(const WeightView& w, const Q8View& x, float* out, const float* residual,
                             hipStream_t s, void* scratch, int nw, int nj, uint32_t mc, Q6SegReduce reduce) {
  const uint32_t kbs = w.pk / 256, seg_kb = q6_seg_kb(kbs), segs = (kbs + seg_kb - 1) / seg_kb;
  if (w.layout != QW38_LAYOUT_Q6K_WAVE64 || x.pk != w.pk || w.pn % 8 != 0 ||
      !((nw == 10 && (nj == 8 || nj == 4)) || (nw == 5 && nj == 8)) ||
      mc == 0 || mc % kPB != 0 || x.m == 0 ||
      ((reinterpret_cast<uintptr_t>(w.codes) | reinterpret_cast<uintptr_t>(w.scales) |
        reinterpret_cast<uintptr_t>(x.codes)) % 16) != 0 ||
      (segs > 1 && !reduce))
    return hipErrorInvalidValue;
  const uint32_t groups = x.pk / 32;
  uint8_t* bq = static_cast<uint8_t*>(scratch);
  float* part = reinterpret_cast<float*>(bq + (mmq_dma_scratch_bytes(mc, w.pk) + 255) / 256 * 256);
  auto kern = nw == 5 ? q6_mmq_dma_kernel<5> : nj == 4 ? q6_mmq_dma_kernel<10, 4> : q6_mmq_dma_kernel<10>;
  const uint32_t br = nw == 10 ? Geo6<10>::BR : Geo6<5>::BR, bt = 16u * uint32_t(nj);
  const uint32_t lds_bytes = nw == 5 ? Geo6<5>::Lds : nj == 4 ? Geo6<10, 4>::Lds : Geo6<10>::Lds;
  hipError_t e = set_max_lds(reinterpret_cast<const void*>(kern), int(lds_bytes));
  for (uint32_t t0 = 0; e == hipSuccess && t0 < x.m; t0 += mc) {
    const uint32_t m = std::min(mc, x.m - t0), mp = (m + kPB - 1) / kPB * kPB;
    uint8_t* tq = bq + uint64_t(mp) * w.pk * 2;
    float* ti = reinterpret_cast<float*>(tq + uint64_t(mp / kPB) * kbs * kTSlot);
    hipLaunchKernelGGL(mmq_dma_prep_kernel, dim3(mp / 64, kbs + 16), dim3(256), 0, s, x.codes + size_t(t0) * x.pk,
                       x.scales + size_t(t0) * groups, x.sums + size_t(t0) * groups, m, x.pk, bq, tq, ti, true, false);
    e = hipGetLastError();
    if (e != hipSuccess) break;
    float* o = out + size_t(t0) * w.n;
    const float* res = residual ? residual + size_t(t0) * w.n : nullptr;
    const uint32_t row_blocks = (w.pn + br - 1) / br, tok_blocks = (m + bt - 1) / bt;
    hipLaunchKernelGGL(kern, dim3(row_blocks * tok_blocks * segs), dim3(nw * 64), lds_bytes, s, w.codes, w.scales,
                       w.n, w.pn, kbs, bq, tq, m, o, res, row_blocks, tok_blocks, seg_kb, segs, part);
    e = hipGetLastError();
    if (e == hipSuccess && segs > 1) e = reduce(part, segs, m, w.n, res, o, s);
  }
  return e;
}

}  // namespace qw38hip
