// Thin C-ABI shim over the reference's vendored, pinned llama.cpp Q4_K header
// (third_party/llama.cpp-q4k/reference.hpp in the reference tree), compiled in
// place from /root/reference by oracle/Makefile into oracle/_ref/. Test
// infrastructure only: it checks the oracle's Q4_K quantizer and FP16 helpers.
#include "third_party/llama.cpp-q4k/reference.hpp"

extern "C" {
void ref_quantize_row_q4_K(const float* x, void* blocks, long long k) {
  pinned_llama_q4k::quantize_row_q4_K_ref(
      x, static_cast<pinned_llama_q4k::block_q4_K*>(blocks), k);
}
void ref_dequantize_row_q4_K(const void* blocks, float* y, long long k) {
  pinned_llama_q4k::dequantize_row_q4_K(
      static_cast<const pinned_llama_q4k::block_q4_K*>(blocks), y, k);
}
float ref_fp16_to_fp32(unsigned short h) {
  return pinned_llama_q4k::ggml_compute_fp16_to_fp32(h);
}
unsigned short ref_fp32_to_fp16(float f) {
  return pinned_llama_q4k::ggml_compute_fp32_to_fp16(f);
}
int ref_nearest_int(float f) { return pinned_llama_q4k::nearest_int(f); }
}
