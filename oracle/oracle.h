/*
 * CPU oracle for the Q4_K / Q6_K x Q8 projection path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline). The product path in qw38_amd/ never links,
 * loads or falls back to it.
 *
 * Every function restates the reference algorithm it names (file:line in the
 * reference tree) in plain C; the header of oracle.c lists how each one is
 * pinned (golden vectors, the compiled pinned llama.cpp header, closed forms).
 */
#ifndef QW38_ORACLE_H
#define QW38_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions ------------------------------------------------ */
float orc_fp16_to_fp32(uint16_t h);
uint16_t orc_fp32_to_fp16(float f);
float orc_bf16_to_fp32(uint16_t h);
uint16_t orc_fp32_to_bf16_rne(float x);
int orc_nearest_int(float x);
float orc_expf(float x);

/* ---- Q8 activation producers ------------------------------------------- */
/* BF16 [m][k] -> codes int8 [m][pk], scales f32 [m][pk/32], sums i32.
 * Returns 1 when any group was nonfinite (the device failure flag). */
int orc_pack_q8(const uint16_t* bf16, uint32_t m, uint32_t k, uint32_t pk,
                int8_t* codes, float* scales, int32_t* sums);
/* Same producer over FP32 values already rounded by the caller. */
int orc_pack_q8_f32(const float* x, uint32_t m, uint32_t k, uint32_t pk,
                    int8_t* codes, float* scales, int32_t* sums);
/* Zero-centred RMS (1+gamma)*x/rms -> BF16 -> Q8, hidden width 5120. */
int orc_rms_q8(const float* residual, const uint16_t* gamma, float eps,
               uint32_t m, int8_t* codes, float* scales, int32_t* sums,
               uint16_t* bf16_out /* may be NULL */);
/* BF16(SiLU(g)*u) -> Q8 over [m][n]; n % 256 == 0. */
int orc_swiglu_q8(const float* gate, const float* up, uint32_t m, uint32_t n,
                  int8_t* codes, float* scales, int32_t* sums,
                  uint16_t* bf16_out /* may be NULL */);

/* ---- Q4_K quantizer and layouts ----------------------------------------- */
/* 256 floats -> codes[256] in 0..15 and meta[16] (d, dmin, 12 packed bytes).
 * Returns 0, or 1 (nonfinite) / 2 (unrepresentable) as the reference does. */
int orc_quantize_q4k_block(const float* x, uint8_t* codes, uint8_t* meta);
/* Row-major [n][k] (k % 256 == 0) -> logical codes [n][k], meta [n][k/256][16]. */
int orc_quantize_q4k_rows(const float* x, uint64_t n, uint64_t k,
                          uint8_t* codes, uint8_t* meta, int threads);
void orc_q4k_logical_to_ggml(const uint8_t* codes, const uint8_t* meta,
                             uint64_t blocks, uint8_t* ggml /* 144 B each */);
void orc_q4k_ggml_to_logical(const uint8_t* ggml, uint64_t blocks,
                             uint8_t* codes, uint8_t* meta);
void orc_q4k_scale_min(const uint8_t* meta, unsigned g, unsigned* s, unsigned* m);
/* Logical [n][pk] -> physical tiles. layout 0x020D: sequential nibbles;
 * layout 0x0240: wave64 nibble order. codes_out: padded_n*pk/2 bytes,
 * meta_out: padded_n*(pk/256)*16 bytes. */
int orc_pack_q4k_layout(uint16_t layout, const uint8_t* codes, const uint8_t* meta,
                        uint32_t n, uint32_t pk, uint8_t* codes_out, uint8_t* meta_out);
int orc_unpack_q4k_layout(uint16_t layout, const uint8_t* codes_in, const uint8_t* meta_in,
                          uint32_t n, uint32_t pk, uint8_t* codes, uint8_t* meta);

/* ---- Q6_K quantizer and layouts ----------------------------------------- */
/* 256 floats -> q[256] in 0..63, sc[16] int8, d fp16 bits. */
void orc_quantize_q6k_block(const float* x, uint8_t* q, int8_t* sc, uint16_t* d);
float orc_q6k_fit_subblock(const float* x, uint8_t* L);
int orc_quantize_q6k_rows(const float* x, uint64_t n, uint64_t k, uint8_t* q,
                          int8_t* sc, uint16_t* d, int threads);
void orc_q6k_logical_to_ggml(const uint8_t* q, const int8_t* sc, const uint16_t* d,
                             uint64_t blocks, uint8_t* ggml /* 210 B each */);
void orc_q6k_ggml_to_logical(const uint8_t* ggml, uint64_t blocks, uint8_t* q,
                             int8_t* sc, uint16_t* d);
/* layout 0x0241: codes = padded_n*kbs*192 B, scales = padded_n*kbs*18 B. */
int orc_pack_q6k_layout(const uint8_t* q, const int8_t* sc, const uint16_t* d,
                        uint32_t n, uint32_t pk, uint8_t* codes_out, uint8_t* meta_out);
int orc_unpack_q6k_layout(const uint8_t* codes_in, const uint8_t* meta_in,
                          uint32_t n, uint32_t pk, uint8_t* q, int8_t* sc, uint16_t* d);

/* ---- contractions ------------------------------------------------------- */
/* out64[t][r] = sum_g a*(ds*dot - dm*sum) in double (closed form);
 * out32[t][r] = the same expression in FP32, ascending-K order (reference
 * K32 order); dots[t][r][g] = exact per-group int32 dots (any may be NULL). */
void orc_q4k_q8_contract(const uint8_t* codes, const uint8_t* meta, uint32_t n,
                         uint32_t pk, const int8_t* z, const float* a,
                         const int32_t* sums, uint32_t m, double* out64,
                         float* out32, int32_t* dots, int threads);
/* Q6_K: per K32 group I = sc0*sum16((q-32)z) + sc1*sum16((q-32)z);
 * out += a * (d * I). dots[t][r][g] = I. */
void orc_q6k_q8_contract(const uint8_t* q, const int8_t* sc, const uint16_t* d,
                         uint32_t n, uint32_t pk, const int8_t* z, const float* a,
                         const int32_t* sums, uint32_t m, double* out64,
                         float* out32, int32_t* dots, int threads);

/* ---- BF16-activation decode (decode_mmv Q4_K branch) -------------------- */
/* Reconstructed BF16 weight operand for one logical element. */
float orc_q4k_bf16_weight(const uint8_t* meta_block, unsigned code, unsigned g);
/* y[r] = sum_k W[r][k]*x[k] with W reconstructed as the BF16 operand;
 * out64 in double. */
void orc_q4k_bf16_gemv(const uint8_t* codes, const uint8_t* meta, uint32_t n,
                       uint32_t pk, uint32_t k, const uint16_t* x, double* out64,
                       int threads);

/* ---- decode_mmv dense layouts (Q4G64 0x0201/0x020B, Q8G32 0x0202/0x020C,
 * BF16 dense tile 0x0203) ---------------------------------------------------- */
/* Logical codes [n][k] and FP16 scale bits [n][k/group] -> tiled codes/scales. */
int orc_pack_dense_layout(uint16_t layout, const int8_t* codes, const uint16_t* scales,
                          uint32_t n, uint32_t k, uint8_t* co, uint8_t* so);
/* Row-major BF16 [n][k] -> BF16 dense tiles. */
int orc_pack_bf16_tile(const uint16_t* w, uint32_t n, uint32_t k, uint8_t* co);
/* BF16 operand bits of every padded element, out[pn][pk]. */
void orc_dense_operands(uint16_t layout, const uint8_t* co, const uint8_t* so, uint32_t pn,
                        uint32_t pk, uint16_t* out);

/* ---- FP8 (OCP E4M3FN) path (cuda/fp8.cu) ---------------------------------- */
float orc_e4m3_to_fp32(uint8_t c);
uint8_t orc_fp32_to_e4m3(float x);
/* BF16 [m][k] -> codes [pm][pk], scales [pk/128][pm] (pm, pk padded to 128). */
void orc_pack_fp8(const uint16_t* x, uint32_t m, uint32_t k, uint8_t* codes, float* scales);
/* y[n] and per-row sum of |products| (l1, may be NULL) in double. */
void orc_fp8_gemv(const uint8_t* codes, const float* wscales, uint32_t n, uint32_t k,
                  const uint16_t* x, double* out, double* l1);
/* y[m][n] and l1 [m][n] (may be NULL) in double; xs is [k/128][m]. */
void orc_fp8_gemm(const uint8_t* wc, const float* ws, uint32_t n, uint32_t k, const uint8_t* xc,
                  const float* xs, uint32_t m, double* out, double* l1);

/* ---- NVFP4 (src/format/nvfp4.cpp, cuda/nvfp4.cu) --------------------------- */
float orc_e2m1_value(uint8_t c);
float orc_ue4m3_value(uint8_t c);
uint8_t orc_nvfp4_nearest(float v, int scale);
uint64_t orc_nvfp4_sf_index(uint64_t row, uint64_t block, uint64_t pk);
void orc_pack_nvfp4(const uint16_t* x, uint32_t m, uint32_t k, uint8_t* codes, uint8_t* scales);
int orc_quantize_nvfp4(const uint16_t* w, uint32_t n, uint32_t k, uint8_t* codes, uint8_t* scales);
void orc_nvfp4_gemv(const uint8_t* codes, const uint8_t* scales, uint32_t n, uint32_t pk,
                    const uint16_t* x, uint32_t k, double* out, double* l1);
void orc_nvfp4_gemm(const uint8_t* wc, const uint8_t* ws, uint32_t n, uint32_t pk, const uint8_t* xc,
                    const uint8_t* xs, uint32_t m, double* out, double* l1);


#ifdef __cplusplus
}
#endif
#endif
