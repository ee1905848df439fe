/*
 * qw38_hip.h -- C-ABI boundary of the MI355X (gfx950) Q4_K_M x Q8 projection
 * path. Plain pointers, sizes and a HIP stream handle passed as void*; no C++
 * or torch types. Every entry point validates all operands before launching
 * anything and returns a qw38_status; the details of the last failure on the
 * calling thread are available from qw38_last_error().
 *
 * Each declaration names the reference interface it replaces (paths are in the
 * Enucatl/qw38 tree). The C++ mirror of those interfaces (namespace
 * qw38::cuda, headers under qw38_amd/cpp/cuda/, sources under
 * qw38_amd/cpp/src/) is implemented on top of this ABI.
 */
#ifndef QW38_HIP_H
#define QW38_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: mirror qw38::cuda::ErrorCode (cuda/error.hpp:13-17). */
enum qw38_status {
  QW38_OK = 0,
  QW38_STATUS = 1,           /* HIP runtime failure (hip status in last error) */
  QW38_INVALID_ARGUMENT = 2, /* contract violation, rejected before launch */
  QW38_OVERFLOW = 3          /* size/address arithmetic overflow */
};

/* Layout / quantizer wire IDs. 0x020D/0x0105 are the reference's
 * (cuda/decode_mmv.hpp:195,205); 0x0240/0x0241/0x0140 are this build's
 * repacked layouts (lossless byte reorders of GGML super-blocks). */
#define QW38_LAYOUT_Q4K_CANDIDATE_V2 0x020D /* sequential nibbles, 8-row tiles */
#define QW38_LAYOUT_Q4K_WAVE64 0x0240       /* 0x020D tiles, wave64 nibble order */
#define QW38_LAYOUT_Q6K_WAVE64 0x0241       /* Q6_K 8-row tiles */
#define QW38_QUANTIZER_Q4K 0x0105
#define QW38_QUANTIZER_Q6K 0x0140

/* Matrix operand: field-for-field cuda::PrefillWeight (cuda/prefill.hpp:33-44). */
typedef struct qw38_weight {
  const void* codes;
  const void* scales;
  uint16_t layout;
  uint16_t quantizer;
  uint32_t n;
  uint32_t k;
  uint32_t padded_n;
  uint32_t padded_k;
  uint64_t codes_bytes;
  uint64_t scales_bytes;
} qw38_weight;

/* Q8 activation pack: cuda::Q8Input (cuda/q4k_q8.hpp:16-21) with each span as
 * pointer + element count. codes int8 [m][padded_k], scales f32 and sums i32
 * [m][padded_k/32]. */
typedef struct qw38_q8_input {
  int8_t* codes;
  uint64_t codes_len;
  float* scales;
  uint64_t scales_len;
  int32_t* sums;
  uint64_t sums_len;
  uint32_t m;
  uint32_t k;
  uint32_t padded_k;
} qw38_q8_input;

/* Limits (cuda/q4k_q8.hpp:23-25 and the larger shapes this build supports). */
#define QW38_Q4K_Q8_DOT_BOUND (32 * 15 * 127)
#define QW38_Q8_SUM_BOUND (32 * 127)
#define QW38_Q8_MLP_MAX_TOKENS 512u
#define QW38_PROJECT_MAX_TOKENS 4096u
#define QW38_PROJECT_MAX_K 65536u
#define QW38_PROJECT_MAX_N (1u << 20)

/* Last failure on this thread: returns its status; copies the failing
 * operation name and detail (NUL-terminated, truncated to the capacities). */
int qw38_last_error(int* hip_status, char* operation, size_t operation_cap,
                    char* detail, size_t detail_cap);

/* Replaces qw38::cuda::pack_q8 (cuda/q4k_q8.hpp:32-34, cuda/q4k_q8.cu:318-330).
 * BF16 rows [m][k] -> Q8 pack; *failure is set to 1 on a nonfinite group
 * (that group's scale becomes NaN and its codes 0). failure_len must be 1. */
int qw38_pack_q8(const uint16_t* input, uint64_t input_len, const qw38_q8_input* output,
                 int* failure, uint64_t failure_len, void* stream);

/* Replaces qw38::cuda::q4k_q8_project (cuda/q4k_q8.hpp:35-37,
 * cuda/q4k_q8.cu:332-345). out [m][n] fp32 = W x^T (+ residual). Accepts
 * layouts 0x020D and 0x0240 (Q4_K) and 0x0241 (Q6_K). residual may be NULL
 * with residual_len 0. M <= 8 runs the HBM-streaming GEMV; larger M the MFMA
 * MMQ kernels. */
int qw38_q4k_q8_project(const qw38_weight* weight, const qw38_q8_input* input,
                        float* output, uint64_t output_len, const float* residual,
                        uint64_t residual_len, void* stream);

/* The gate + up half of q4k_q8_mlp (cuda/q4k_q8.cu:378-385: two
 * q4k_q8_project calls, then the SwiGLU->Q8 producer of cuda/q4k_q8.cu:52-61)
 * as ONE launch: output = Q8 pack of BF16(SiLU(gate x) * (up x)), written by
 * the projection's epilogue (no FP32 [m][n] intermediates). Bit-identical to
 * the unfused chain. gate/up: Q4_K (0x020D or 0x0240), same layout and
 * geometry, n % 32 == 0; output: m x n Q8 operand; *failure is set to 1 on a
 * nonfinite group (failure_len must be 1). m == 1 on layout 0x020D runs the
 * streaming decode GEMV's arithmetic, every other case the MFMA MMQ's; each
 * equals the unfused chain at the m where q4k_q8_project runs the same
 * kernel family. q4k_q8_mlp uses it wherever it applies (m > 8, or m == 1 on
 * 0x020D). No reference counterpart as an entry point. */
int qw38_q4k_q8_gate_up_swiglu(const qw38_weight* gate, const qw38_weight* up,
                               const qw38_q8_input* input, const qw38_q8_input* output,
                               int* failure, uint64_t failure_len, void* stream);

/* Replaces cuda::q8_mlp_workspace_bytes (cuda/q4k_q8.hpp:28-30). */
uint64_t qw38_q8_mlp_workspace_bytes(uint32_t m);

/* Replaces qw38::cuda::q4k_q8_mlp (cuda/q4k_q8.hpp:44-49, cuda/q4k_q8.cu:
 * 347-398): RMS->Q8, gate, up, SwiGLU->Q8, down + residual. *submitted is 0
 * on prelaunch rejection and 1 once device work was enqueued. With
 * pending_failure NULL the call waits and reports a nonfinite producer as
 * QW38_INVALID_ARGUMENT ("q8.producer"); otherwise it only enqueues and the
 * caller reads the sticky flag. */
int qw38_q4k_q8_mlp(const qw38_weight* gate, const qw38_weight* up, const qw38_weight* down,
                    const float* residual, const uint16_t* gamma, float eps, float* output,
                    uint32_t m, void* workspace, uint64_t workspace_bytes, void* stream,
                    int* submitted, int* pending_failure);

/* No counterpart in the reference: an allocation-free qw38_q4k_q8_mlp for
 * callers that cannot allocate or pass device memory (code under HIP graph
 * capture, tight serving loops). Same operands, semantics and errors as
 * qw38_q4k_q8_mlp, but the workspace is a static device array of the library
 * (qw38_q8_mlp_static_scratch_bytes(), held on each GPU until the process
 * ends), so m <= QW38_Q8_MLP_STATIC_MAX_TOKENS; larger m is rejected with
 * QW38_INVALID_ARGUMENT before any launch. Every call on one GPU shares that
 * GPU's scratch, so calls must be serialized per device: a call made while
 * another is running on the host, or while an earlier call's device work on
 * another stream has not completed, is rejected with QW38_INVALID_ARGUMENT
 * before any launch (calls on one stream are ordered by the stream and
 * accepted). Work captured into a graph is not tracked: replays of captured
 * calls on several streams must be serialized by the caller. Without
 * pending_failure the internal failure flag is cleared by a kernel on each
 * call; a caller-supplied pending_failure is never cleared (the caller zeroes
 * it), as in qw38_q4k_q8_mlp. */
#define QW38_Q8_MLP_STATIC_MAX_TOKENS 64u
uint64_t qw38_q8_mlp_static_scratch_bytes(void);
int qw38_q4k_q8_mlp_static(const qw38_weight* gate, const qw38_weight* up, const qw38_weight* down,
                           const float* residual, const uint16_t* gamma, float eps, float* output,
                           uint32_t m, void* stream, int* submitted, int* pending_failure);

/* Replaces launch_hidden_rms_q8 (cuda/activation.hpp:11-14,
 * cuda/activation.cu:536-548): zero-centred RMS over hidden 5120 ->
 * BF16 -> Q8 pack. codes [m][5120], scales/sums [m][160]. */
int qw38_hidden_rms_q8(const float* residual, const uint16_t* gamma, float eps, uint32_t m,
                       int8_t* codes, float* scales, int32_t* sums, int* failure,
                       void* stream);

/* The SwiGLU->Q8 producer used inside q4k_q8_mlp (cuda/q4k_q8.cu:52-61),
 * exposed on its own: BF16(SiLU(gate)*up) -> Q8 over [m][n], n % 256 == 0. */
int qw38_swiglu_q8(const float* gate, const float* up, uint32_t m, uint32_t n,
                   int8_t* codes, float* scales, int32_t* sums, int* failure, void* stream);

/* Parity aid with no reference counterpart: the exact per-(token, row, K32
 * group) int32 dots [m][n][padded_k/32] computed by the same device dot
 * routines the projection kernels use (for Q6_K: sc0*dot0 + sc1*dot1). */
int qw38_q8_group_dots(const qw38_weight* weight, const qw38_q8_input* input, int32_t* dots,
                       uint64_t dots_len, void* stream);

/* Load-time repack replacing the untyped cuda::upload of pre-tiled bytes
 * (cuda/upload.hpp:16-17, cuda/upload.cpp:6-27) for GGML-order weights:
 * n*(k/256) super-blocks (144 B Q4_K / 210 B Q6_K, row-major) already in
 * device memory -> the tiled layout (0x020D or 0x0240 for Q4_K, 0x0241 for
 * Q6_K). Lossless: only the byte order changes. k % 256 == 0. */
int qw38_repack_q4k_blocks(const void* blocks, uint64_t blocks_bytes, uint32_t n, uint32_t k,
                           uint16_t layout, void* codes, uint64_t codes_bytes, void* scales,
                           uint64_t scales_bytes, void* stream);
int qw38_repack_q6k_blocks(const void* blocks, uint64_t blocks_bytes, uint32_t n, uint32_t k,
                           void* codes, uint64_t codes_bytes, void* scales,
                           uint64_t scales_bytes, void* stream);

/* On-device fitting of FP32 rows [n][k] (k % 256 == 0) into GGML-order
 * super-blocks, replacing the offline compiler's quantize_bf16 / quantize_q4k_block
 * (src/compiler/quantization/quantizer.cpp:173-183, q4k.cpp:186-278; Q6_K from
 * llama.cpp quantize_row_q6_K_ref). Output bytes equal the pinned CPU fitter's.
 * Q4_K: *failure is set to 1 for nonfinite or unrepresentable blocks (those
 * blocks are left unwritten). Follow with qw38_repack_*_blocks. */
int qw38_quantize_q4k_blocks(const float* x, uint64_t x_len, uint32_t n, uint32_t k,
                             void* blocks, uint64_t blocks_bytes, int* failure, void* stream);
int qw38_quantize_q6k_blocks(const float* x, uint64_t x_len, uint32_t n, uint32_t k,
                             void* blocks, uint64_t blocks_bytes, void* stream);

/* ---- BF16-activation decode GEMV (cuda/decode_mmv.hpp) -------------------
 * Field-for-field mirrors of DecodeOperandView, DecodeMmvDesc and the enums
 * (cuda/decode_mmv.hpp:25-134). Validation follows the reference's contract
 * (cuda/decode_mmv.cu:245-560): typed views, padded geometry, exact byte
 * counts, alignment, writability and non-overlap, all before any launch.
 * This build implements the Q4_K layout 0x020D (quantizer 0x0105), Q4G64
 * (0x0201, 0x020B), Q8G32 (0x0202, 0x020C), BF16 dense tiles (0x0203), FP8
 * (0x020F, single and ranged launches) and NVFP4 (0x020E: single and paired
 * launches; ranged launches are rejected, cuda/decode_mmv.cu:796-799). */
#define QW38_DECODE_LAYOUT_Q4G64_V0 0x0201
#define QW38_DECODE_LAYOUT_Q8G32_V0 0x0202
#define QW38_DECODE_LAYOUT_BF16_DENSE_TILE_V0 0x0203
#define QW38_DECODE_LAYOUT_BF16_VECTOR_V0 0x0205
#define QW38_DECODE_LAYOUT_FP32_VECTOR_V0 0x020A
#define QW38_DECODE_LAYOUT_Q4G64_CANDIDATE_V1 0x020B
#define QW38_DECODE_LAYOUT_Q8G32_CANDIDATE_V1 0x020C
#define QW38_DECODE_LAYOUT_NVFP4_V1 0x020E
#define QW38_DECODE_LAYOUT_FP8_V1 0x020F
#define QW38_DECODE_QUANTIZER_NONE 0x0100
#define QW38_DECODE_QUANTIZER_Q4G64_V0 0x0101
#define QW38_DECODE_QUANTIZER_Q8G32_V0 0x0102
#define QW38_DECODE_QUANTIZER_Q4G64_CANDIDATE_V1 0x0103
#define QW38_DECODE_QUANTIZER_Q8G32_CANDIDATE_V1 0x0104
#define QW38_DECODE_QUANTIZER_NVFP4_V1 0x0106
#define QW38_DECODE_QUANTIZER_FP8_V1 0x0107
#define QW38_DECODE_MAX_K 17408u

/* DecodeEpilogue */
#define QW38_DECODE_STORE_BF16 1
#define QW38_DECODE_STORE_FP32 2
#define QW38_DECODE_RESIDUAL_ADD_FP32 3
#define QW38_DECODE_SWIGLU_BF16 4
/* DecodeMemorySpace */
#define QW38_DECODE_SPACE_DEVICE 1
#define QW38_DECODE_SPACE_HOST 2
/* DecodeDtype */
#define QW38_DECODE_DTYPE_Q4 1
#define QW38_DECODE_DTYPE_Q8 2
#define QW38_DECODE_DTYPE_BF16 3
#define QW38_DECODE_DTYPE_FP16 4
#define QW38_DECODE_DTYPE_FP32 5
#define QW38_DECODE_DTYPE_NVFP4 6
#define QW38_DECODE_DTYPE_FP8 7
/* DecodeActivationPolicy */
#define QW38_DECODE_ACTIVATION_BF16 1

typedef struct qw38_decode_view {
  void* pointer;
  uint8_t space;
  uint8_t dtype;
  uint16_t layout;
  uint32_t logical_n;
  uint32_t logical_k;
  uint32_t padded_n;
  uint32_t padded_k;
  uint64_t bytes;
  uint32_t alignment;
  uint8_t writable;
} qw38_decode_view;

typedef struct qw38_decode_desc {
  uint16_t layout;
  uint16_t quantizer;
  uint8_t activation_policy;
  uint32_t n;
  uint32_t k;
  uint32_t padded_n;
  uint32_t padded_k;
  qw38_decode_view codes;
  qw38_decode_view scales;
  qw38_decode_view input;
  qw38_decode_view output;
  qw38_decode_view residual;
  uint8_t epilogue;
} qw38_decode_desc;

/* Replaces qw38::cuda::launch_decode_mmv (cuda/decode_mmv.hpp:205-206,
 * cuda/decode_mmv.cu:755-766). y[n] = W x, x BF16 [k], FP32 accumulation of
 * the rebuilt BF16 weights, then the epilogue. */
int qw38_decode_mmv(const qw38_decode_desc* desc, void* stream);
/* Replaces launch_decode_mmv_paired (cuda/decode_mmv.hpp:208-209,
 * cuda/decode_mmv.cu:768-779): gate/up sharing K and input, separate outputs
 * or SwiGLU -> BF16 into a's output. */
int qw38_decode_mmv_paired(const qw38_decode_desc* a, const qw38_decode_desc* b, void* stream);
/* Replaces launch_decode_mmv_ranges (cuda/decode_mmv.hpp:216-217,
 * cuda/decode_mmv.cu:781-853): two or three BF16-store projections sharing
 * layout, K and input. */
int qw38_decode_mmv_ranges(const qw38_decode_desc* ranges, uint32_t count, void* stream);
/* Replaces launch_decode_ab_bf16 (cuda/decode_mmv.hpp:211-213,
 * cuda/decode_mmv.cu:781-800): two BF16 dense-tile matrices (the GDN a/b
 * projections) sharing K and input, FP32 outputs, one launch. */
int qw38_decode_ab_bf16(const qw38_decode_desc* a, const qw38_decode_desc* b, void* stream);
/* ---- FP8 (OCP E4M3FN) projections (cuda/fp8.hpp) -------------------------
 * Fp8Weight / Fp8Input (cuda/fp8.hpp:13-22): E4M3 codes row-major with padded
 * extents that are multiples of 128, FP32 scales per 128-column block: weights
 * [k/128][n/128] (128 x 128 blocks), activations [k/128][m] (1 x 128 blocks). */
typedef struct qw38_fp8_weight {
  const uint8_t* codes;
  uint64_t codes_len; /* elements (bytes) */
  const float* scales;
  uint64_t scales_len; /* elements */
  uint32_t n, k;
} qw38_fp8_weight;
typedef struct qw38_fp8_input {
  const uint8_t* codes;
  uint64_t codes_len;
  const float* scales;
  uint64_t scales_len;
  uint32_t m, k;
} qw38_fp8_input;
/* Replaces cuda::pack_fp8 (cuda/fp8.hpp:29-31, cuda/fp8.cu:172-183): BF16
 * [m][k] (m <= 1024, k <= 17408) -> codes [pm][pk], scales [pk/128][pm],
 * absmax/448 per (row, 128 block), NaN scale for a nonfinite block. */
int qw38_pack_fp8(const uint16_t* input, uint64_t input_len, uint32_t m, uint32_t k,
                  uint8_t* codes, uint64_t codes_len, float* scales, uint64_t scales_len,
                  void* stream);
/* Replaces cuda::fp8_gemv (cuda/fp8.hpp:35-37, cuda/fp8.cu:195-203): y[n] FP32
 * from BF16 x[k]. */
int qw38_fp8_gemv(const qw38_fp8_weight* weight, const uint16_t* x, uint64_t x_len, float* y,
                  uint64_t y_len, void* stream);
/* Replaces cuda::fp8_gemm (cuda/fp8.hpp:32-34, cuda/fp8.cu:137-160): y[m][n]
 * FP32, m a multiple of 128 up to 1024. The workspace and SM count are
 * accepted for interface parity and must be non-empty / positive; the kernel
 * needs no workspace. */
int qw38_fp8_gemm(const qw38_fp8_weight* weight, const qw38_fp8_input* input, float* y,
                  uint64_t y_len, void* workspace, uint64_t workspace_bytes, int sm_count,
                  void* stream);
/* Replaces the FP8 branch of PrefillEngine::project for M > 1
 * (cuda/prefill.cu:565-593: fp8_gemm into an FP32 scratch, then
 * epilogue_kernel at cuda/prefill.cu:116-134). Here the epilogue is fused into
 * the GEMM's store and no scratch is used. input is the pack_fp8 operand of
 * the tokens (m = tokens rounded up to 128); output [tokens][n] is BF16
 * (QW38_DECODE_STORE_BF16) or FP32 (_STORE_FP32, _RESIDUAL_ADD_FP32:
 * output = residual + product, residual [tokens][n] not aliasing output).
 * Weight geometry: n <= 12288, n % 128 == 0, k <= 6144, k % 256 == 0
 * (cuda/prefill.cu:218-219). */
int qw38_fp8_project(const qw38_fp8_weight* weight, const qw38_fp8_input* input, uint32_t tokens,
                     void* output, const float* residual, int epilogue, void* stream);
/* ---- NVFP4 (cuda/nvfp4.hpp, cuda/nvfp4.cu) --------------------------------
 * Elements are E2M1 nibbles, row-major [rows][pk/2] with element 2j in the
 * low nibble of byte j; every 16 elements share a UE4M3 scale byte placed by
 * the CUTLASS SM1xx swizzle over 128-row stripes (src/format/nvfp4.hpp:
 * 9-18). Weights prepend a 256-byte header whose first 4 bytes are the FP32
 * global factor. */
/* Replaces launch_pack_nvfp4 (cuda/nvfp4.hpp:17-19, cuda/nvfp4.cu:72-82):
 * BF16 [m][k] -> codes [m][pk/2] and scales of pad128(m) rows (padding
 * rows' scales 0). The byte sizes are checked against m, pad_k(k). */
int qw38_pack_nvfp4(const uint16_t* input, uint32_t m, uint32_t k, uint8_t* codes,
                    uint64_t codes_bytes, uint8_t* scales, uint64_t scales_bytes, void* stream);
/* Replaces launch_hidden_rms_nvfp4 (cuda/activation.hpp:20-22,
 * cuda/activation.cu:507-520): the RMS of hidden 5120 packed straight to
 * NVFP4 (codes [m][2560], scales of pad128(m) rows). */
int qw38_hidden_rms_nvfp4(const float* residual, const uint16_t* gamma, float eps, uint32_t m,
                          uint8_t* codes, uint8_t* scales, void* stream);
/* Replaces launch_hidden_rms_fp8 (cuda/activation.hpp:16-19,
 * cuda/activation.cu:522-534): the RMS of hidden 5120 packed to FP8 (codes
 * [pad128(m)][5120], scales [40][pad128(m)]); companion, when non-null,
 * receives the BF16 row [m][5120]. */
int qw38_hidden_rms_fp8(const float* residual, const uint16_t* gamma, float eps, uint32_t m,
                        uint16_t* companion, uint8_t* codes, float* scales, void* stream);
/* Replaces nvfp4_gemm_tile (cuda/nvfp4.hpp:12-16, cuda/nvfp4.cu:83-116):
 * output FP32 [m][n] = factor * activation . weight rows row_start ..
 * row_start + n - 1 (m <= 1024, n <= 17408, n % 8 == 0, k <= 5120,
 * k % 256 == 0, row_start % 128 == 0). No workspace is needed. */
int qw38_nvfp4_gemm_tile(const void* codes, const void* scales, const uint8_t* activation,
                         const uint8_t* activation_scales, uint32_t m, uint32_t n, uint32_t k,
                         uint32_t row_start, float* output, void* stream);
/* Scratch of the NVFP4 prefill entries for `tokens` rows: packed codes and
 * scales, and the FP32 gate projection of the paired SwiGLU. */
uint64_t qw38_nvfp4_workspace_bytes(uint32_t tokens);
/* Replaces the NVFP4 branch of PrefillEngine::project (cuda/prefill.cu:
 * 598-628): pack the BF16 input, W4A4 GEMM, prefill epilogue fused into the
 * store. Weight: layout 0x020E, quantizer 0x0106, K <= 5120, K % 256 == 0,
 * N <= 17408, N % 8 == 0 (cuda/prefill.cu:220-221). The packed part of
 * the workspace (up to the gate region) is required. */
int qw38_nvfp4_project(const qw38_weight* weight, const uint16_t* input, uint32_t tokens,
                       void* output, const float* residual, int epilogue, void* workspace,
                       uint64_t workspace_bytes, void* stream);
/* Replaces the NVFP4 branch of PrefillEngine::paired_swiglu (cuda/prefill.cu:
 * 680-715): one pack, gate GEMM to FP32 scratch, up GEMM storing
 * BF16(SiLU(gate) * up). */
int qw38_nvfp4_paired_swiglu(const qw38_weight* gate, const qw38_weight* up,
                             const uint16_t* normalized, uint16_t* swiglu, uint32_t tokens,
                             void* workspace, uint64_t workspace_bytes, void* stream);
/* Replaces cuda::fp8_store_bf16 (cuda/fp8.hpp:27-28, cuda/fp8.cu:161-171). */
int qw38_fp8_store_bf16(const float* x, uint16_t* y, uint64_t count, void* stream);
/* Replaces cuda::prepare_fp8_gemm (cuda/fp8.hpp:26, cuda/fp8.cu:113-123):
 * compute units of the stream's device. */
int qw38_fp8_prepare(void* stream, int* sm_count);

/* ---- BF16 prefill projections (cuda/prefill.hpp) -------------------------
 * Stateless C-ABI under qw38::cuda::PrefillEngine (cuda/prefill.hpp:72-160):
 * BF16 token-major activations [tokens][k] times a Q4_K 0x020D weight whose
 * operands are rebuilt as BF16 exactly as decode_mmv does, FP32 accumulation
 * on the matrix cores. Epilogue IDs are PrefillEpilogue's (cuda/prefill.hpp:
 * 46-50): QW38_DECODE_STORE_BF16 / _STORE_FP32 / _RESIDUAL_ADD_FP32. Weights
 * with other layouts are rejected as not implemented on this build. */
#define QW38_PREFILL_MAX_K 17408u

/* Replaces PrefillEngine::project (cuda/prefill.cu:510-628) for Q4_K. output
 * [tokens][n] BF16 or FP32; residual [tokens][n] FP32 only with the residual
 * epilogue. */
int qw38_prefill_project(const qw38_weight* weight, const uint16_t* input, uint32_t tokens,
                         void* output, const float* residual, int epilogue, void* stream);
/* Replaces PrefillEngine::paired_swiglu (cuda/prefill.cu:630-715): swiglu
 * [tokens][n] BF16 = BF16(SiLU(X gate^T) * (X up^T)). */
int qw38_prefill_paired_swiglu(const qw38_weight* gate, const qw38_weight* up,
                               const uint16_t* normalized, uint16_t* swiglu, uint32_t tokens,
                               void* stream);
/* Replaces launch_hidden_rms (cuda/activation.hpp, cuda/activation.cu:477-
 * 500): the zero-centred RMS of hidden 5120 written as BF16 [m][5120]. */
int qw38_hidden_rms_bf16(const float* residual, const uint16_t* gamma, float eps, uint32_t m,
                         uint16_t* output, void* stream);
/* Workspace of qw38_prefill_mlp: BF16 normalized [tokens][5120] and SwiGLU
 * [tokens][17408] (the PrefillEngine's normalized_/swiglu_ buffers,
 * cuda/prefill.cu:388-397), then the NVFP4 scratch of
 * qw38_nvfp4_workspace_bytes(tokens) used when gate/up are NVFP4. */
uint64_t qw38_prefill_mlp_workspace_bytes(uint32_t tokens);
/* Replaces PrefillEngine::mlp (cuda/prefill.cu:717-779): RMS -> BF16, paired
 * gate/up SwiGLU, down projection + residual into next_h [tokens][5120].
 * NVFP4 gate/up (layout 0x020E) take the fused RMS -> NVFP4 producer and the
 * W4A4 pair (cuda/prefill.cu:766-772); down is Q4_K 0x020D. */
int qw38_prefill_mlp(const qw38_weight* gate, const qw38_weight* up, const qw38_weight* down,
                     const float* h_mid, const uint16_t* gamma, float eps, float* next_h,
                     uint32_t tokens, void* workspace, uint64_t workspace_bytes, void* stream);

/* Measurement aid with no reference counterpart: one wave per SIMD on every
 * CU runs `iterations` x 4 independent v_mfma_i32_32x32x32_i8; ticks (device
 * memory, 3 x uint64) receives the shader-clock cycles and the 100 MHz
 * real-time ticks wave 0 spent in its loop; *blocks the grid size. Used by the
 * bench to recompute the int8 MFMA dense peak at the measured sclk. */
int qw38_mfma_clock_probe(uint32_t iterations, uint64_t* ticks, uint32_t* blocks, void* stream);

/* No counterpart in the reference: a diagnostic. Writes the library scratch
 * requests on the current device since the process started: stats[0]
 * granted, stats[1] refused because the request exceeded the 64 MB array,
 * stats[2] refused because the array was in use (another thread, or earlier
 * work on another stream). Refused requests run the path without scratch
 * (same bits, more time); tests use the counts to confirm which path ran. */
int qw38_scratch_stats(uint64_t* stats);

/* No counterpart in the reference: a measurement aid. Reads `bytes` (a
 * multiple of 1024, 16-byte aligned device memory) once with no arithmetic
 * beyond an XOR fold: mode 0 grid-stride 16-byte loads, modes 1 / 2 one
 * contiguous range per wave streamed 1 KB per load instruction with 8 / 16
 * loads in flight; blocks_per_cu x CUs
 * blocks of 256 threads. `sink` (>= that many uint32) is written only by a
 * block whose fold hits a fixed 32-bit value. The pure-read ceiling the
 * decode GEMVs are compared against. */
int qw38_read_probe(const void* buf, uint64_t bytes, uint32_t mode, uint32_t blocks_per_cu,
                    uint32_t* sink, uint64_t sink_len, void* stream);

/* No counterpart in the reference: a measurement aid. Eight waves per CU
 * (two per SIMD) run `iterations` of a register-only loop: mode 0 sixteen
 * independent v_mfma_f32_16x16x32_f16, mode 1 sixty-four independent FP32
 * FMAs, mode 2 both interleaved one MFMA to four FMAs, mode 3 eight MFMAs
 * interleaved one to eight FMAs, mode 4 one MFMA-only and one FMA-only wave
 * per SIMD (16 MFMAs and 64 FMAs per SIMD and iteration), modes 5 / 6
 * sixteen independent v_mfma_i32_16x16x32_i8 / 16x16x64_i8 alone. ticks[0] (device memory) receives the
 * s_memtime ticks wave 0 spent in its loop; `sink` (device, >= 1 float)
 * is written only on a value the loop never produces. Shows how far the
 * VALU and the matrix core overlap on one SIMD. */
int qw38_issue_probe(uint32_t mode, uint32_t iterations, uint64_t* ticks, float* sink, void* stream);

/* Replaces qw38::runtime::profiling::enabled (src/runtime/profiling.hpp:9-10):
 * turns the calling thread's roctx ranges ("qw38:op name=q4k_project ...",
 * the reference's NVTX strings) on or off. QW38_PROFILE=1 in the environment
 * turns them on for every thread. */
void qw38_set_profiling(int enabled);

/* Byte sizes of a tiled weight (cuda/decode_mmv.hpp:330-369 for 0x020D,
 * extended with this build's layouts). 0 for an unknown layout. */
uint64_t qw38_code_bytes(uint16_t layout, uint32_t padded_n, uint32_t padded_k);
uint64_t qw38_scale_bytes(uint16_t layout, uint32_t padded_n, uint32_t padded_k);

/* Device allocation with the reference's instrumentation counters
 * (cuda/alloc.hpp:9-15, cuda/buffer.hpp:212-215). */
int qw38_device_malloc(void** pointer, uint64_t bytes);
int qw38_device_free(void* pointer, uint64_t bytes);
uint64_t qw38_malloc_count(void);
uint64_t qw38_free_count(void);
uint64_t qw38_live_bytes(void);
uint64_t qw38_peak_live_bytes(void);
/* Accounting of allocations made outside qw38_device_malloc
 * (cuda::record_malloc / record_free, cuda/alloc.hpp:15-16). */
void qw38_record_malloc(uint64_t bytes);
void qw38_record_free(uint64_t bytes);

#ifdef __cplusplus
}
#endif
#endif
