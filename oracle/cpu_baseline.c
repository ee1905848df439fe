/*
 * CPU baseline of the Q4_K / Q6_K x Q8 contraction -- TEST INFRASTRUCTURE.
 *
 * Timed by bench.py's cpu_baseline leg only (never by the product). It is the
 * reference's own closed-form oracle (tests/q4k_q8_test.cpp:121-131,
 * tests/q8_mlp_integration_test.cpp:21-45) as a plain FP32 CPU kernel:
 * exact int32 dot per (row, token, K32 group) straight from the packed GGML
 * blocks (144 B Q4_K, 210 B Q6_K; no unpacked code arrays), then the FP32
 * affine a * (d*s*dot - dmin*m*sum) (cuda/q4k_q8.cu:97,140) accumulated in
 * ascending K order. Built -O3 -march=native -fopenmp on the machine that
 * runs it, parallel over output rows, tokens innermost so each weight block is
 * read once per row for all M tokens.
 *
 * Q8 activations: codes int8 [m][pk], scales fp32 [m][pk/32], sums int32
 * [m][pk/32] (cuda/q4k_q8.hpp:16-21).
 */
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static float h2f(uint16_t h) {
  uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023, u;
  if (e == 0) {
    if (m == 0) {
      u = s;
    } else {
      e = 113;
      while (!(m & 1024)) { m <<= 1; --e; }
      u = s | (e << 23) | ((m & 1023) << 13);
    }
  } else if (e == 31) {
    u = s | 0x7f800000u | (m << 13);
  } else {
    u = s | ((e + 112) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* llama.cpp get_scale_min_k4 (third_party/llama.cpp-q4k/reference.hpp) */
static inline void scale_min(int j, const uint8_t* q, int* s, int* m) {
  if (j < 4) {
    *s = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *s = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

/* 32 nibbles (low or high half of 32 bytes) x 32 int8 codes, exact int32 */
static inline int32_t dot_nib(const uint8_t* qs, int shift, const int8_t* z) {
  int32_t acc = 0;
  for (int l = 0; l < 32; ++l) acc += (int32_t)((qs[l] >> shift) & 15) * (int32_t)z[l];
  return acc;
}

int cpub_q4k(const uint8_t* blocks, uint32_t n, uint32_t k, const int8_t* codes,
             const float* scales, const int32_t* sums, uint32_t m, float* out, int threads) {
  if (k % 256 || m == 0 || m > 64) return 1;
  const uint32_t kbs = k / 256, groups = k / 32;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
#endif
  for (int64_t r = 0; r < (int64_t)n; ++r) {
    float acc[64];
    for (uint32_t t = 0; t < m; ++t) acc[t] = 0.f;
    for (uint32_t kb = 0; kb < kbs; ++kb) {
      const uint8_t* b = blocks + ((uint64_t)r * kbs + kb) * 144;
      uint16_t dh, mh;
      memcpy(&dh, b, 2);
      memcpy(&mh, b + 2, 2);
      const float d = h2f(dh), dmin = h2f(mh);
      for (int g = 0; g < 8; ++g) {
        int s, mn;
        scale_min(g, b + 4, &s, &mn);
        const float ds = d * (float)s, dm = dmin * (float)mn;
        const uint8_t* qs = b + 16 + 32 * (g / 2);
        const int shift = (g & 1) * 4;
        for (uint32_t t = 0; t < m; ++t) {
          const uint64_t gi = (uint64_t)t * groups + kb * 8 + g;
          const int32_t dot = dot_nib(qs, shift, codes + gi * 32);
          acc[t] += scales[gi] * (ds * (float)dot - dm * (float)sums[gi]);
        }
      }
    }
    for (uint32_t t = 0; t < m; ++t) out[(uint64_t)t * n + r] = acc[t];
  }
  (void)threads;
  return 0;
}

int cpub_q6k(const uint8_t* blocks, uint32_t n, uint32_t k, const int8_t* codes,
             const float* scales, uint32_t m, float* out, int threads) {
  if (k % 256 || m == 0 || m > 64) return 1;
  const uint32_t kbs = k / 256, groups = k / 32;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
#endif
  for (int64_t r = 0; r < (int64_t)n; ++r) {
    float acc[64];
    for (uint32_t t = 0; t < m; ++t) acc[t] = 0.f;
    for (uint32_t kb = 0; kb < kbs; ++kb) {
      const uint8_t* b = blocks + ((uint64_t)r * kbs + kb) * 210;
      const int8_t* sc = (const int8_t*)(b + 192);
      uint16_t dh;
      memcpy(&dh, b + 208, 2);
      const float d = h2f(dh);
      int8_t q[256]; /* q - 32 of the block, ggml block_q6_K order */
      for (int half = 0; half < 2; ++half) {
        const uint8_t* ql = b + 64 * half;
        const uint8_t* qh = b + 128 + 32 * half;
        int8_t* y = q + 128 * half;
        for (int l = 0; l < 32; ++l) {
          y[l] = (int8_t)(((ql[l] & 15) | (((qh[l] >> 0) & 3) << 4)) - 32);
          y[l + 32] = (int8_t)(((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32);
          y[l + 64] = (int8_t)(((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
          y[l + 96] = (int8_t)(((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
        }
      }
      for (int g = 0; g < 8; ++g) {
        const float d0 = d * (float)sc[2 * g], d1 = d * (float)sc[2 * g + 1];
        for (uint32_t t = 0; t < m; ++t) {
          const uint64_t gi = (uint64_t)t * groups + kb * 8 + g;
          const int8_t* z = codes + gi * 32;
          int32_t s0 = 0, s1 = 0;
          for (int l = 0; l < 16; ++l) s0 += (int32_t)q[32 * g + l] * z[l];
          for (int l = 0; l < 16; ++l) s1 += (int32_t)q[32 * g + 16 + l] * z[16 + l];
          acc[t] += scales[gi] * (d0 * (float)s0 + d1 * (float)s1);
        }
      }
    }
    for (uint32_t t = 0; t < m; ++t) out[(uint64_t)t * n + r] = acc[t];
  }
  (void)threads;
  return 0;
}
