// ling_gemm.hpp: the C++ face of libling_gemm.so, shaped like ling-engine's `ling::kernels` quantized GEMM
// functions (reference src/core/kernels.cuh:162-295) so an engine written against them recompiles with HIP.
// Each function forwards to the C ABI (ling_gemm.h) and throws std::runtime_error with the library's message
// on failure; the messages follow the reference's texts ("stream_gemm: K must be a multiple of 128", ...).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>

#include "ling_gemm.h"

namespace ling::kernels {

inline void lq_check(int rc) {
  if (rc != LQ_OK) throw std::runtime_error(lq_last_error());
}

constexpr int kMaxStreamRows = LQ_MAX_STREAM_ROWS;
constexpr int kScaleCodes = 64;

// kernels.cuh:281-287
struct StreamTarget {
  const uint8_t* w;
  const uint8_t* wscale;  // NVFP4: a coded blob's scale-code table; nullptr for a raw blob and for FP8
  float scale;            // NVFP4 global scale, or the FP8 per-tensor scale
  float* y;
  int N;
};

// ---- tiled layout (kernels.cuh:162-188) ----
// The skinny GEMMs' split-K workspace in caller-owned device memory (nullptr: the library's own again).
inline size_t stream_workspace_bytes(int max_rows) { return lq_stream_workspace_bytes(max_rows); }
inline void set_workspace(void* buffer, size_t bytes) { lq_check(lq_set_workspace(buffer, bytes)); }
inline size_t tiled_bytes_nvfp4(int N, int K) { return lq_tiled_bytes_nvfp4(N, K); }
inline size_t tiled_bytes_fp8(int N, int K) { return lq_tiled_bytes_fp8(N, K); }
inline size_t tiled_bytes_nvfp4_coded(int N, int K) { return lq_tiled_bytes_nvfp4_coded(N, K); }
inline void retile_nvfp4(const uint8_t* w, const uint8_t* wscale, uint8_t* out, int N, int K, hipStream_t s) {
  lq_check(lq_retile_nvfp4(w, wscale, out, N, K, s));
}
inline void retile_fp8(const uint8_t* w, uint8_t* out, int N, int K, hipStream_t s) {
  lq_check(lq_retile_fp8(w, out, N, K, s));
}
inline bool scale_code_table(const uint8_t* scales, size_t n, uint8_t (&table)[kScaleCodes], uint8_t (&code_of)[256]) {
  return lq_scale_code_table(scales, n, table, code_of) == 1;
}
inline void retile_nvfp4_coded(const uint8_t* w, const uint8_t* wscale, const uint8_t* code_of_dev, uint8_t* out,
                               uint8_t* raw_scales, int N, int K, hipStream_t s) {
  lq_check(lq_retile_nvfp4_coded(w, wscale, code_of_dev, out, raw_scales, N, K, s));
}
inline void dequant_tiled_nvfp4(const uint8_t* tw, float scale2, uint16_t* out_bf16, int N, int K, hipStream_t s,
                                const uint8_t* raw_scales = nullptr) {
  lq_check(lq_dequant_tiled_nvfp4(tw, scale2, out_bf16, N, K, s, raw_scales));
}
inline void dequant_tiled_fp8(const uint8_t* tw, float wscale, uint16_t* out_bf16, int N, int K, hipStream_t s) {
  lq_check(lq_dequant_tiled_fp8(tw, wscale, out_bf16, N, K, s));
}

// ---- rows path (kernels.cuh:266-295) ----
inline void to_half_rows(const float* x, int M, int K, __half* out, float* xinv, hipStream_t s) {
  lq_check(lq_to_half_rows(x, M, K, reinterpret_cast<uint16_t*>(out), xinv, s));
}
inline void bf16_to_half_rows(const uint16_t* x_bf16, int M, int K, __half* out, float* xinv, hipStream_t s) {
  lq_check(lq_bf16_to_half_rows(x_bf16, M, K, reinterpret_cast<uint16_t*>(out), xinv, s));
}
inline void rmsnorm_half(const float* x, const uint16_t* w_bf16, float* out, __half* xh, float* xinv, int rows, int H,
                         float eps, bool gemma, hipStream_t s) {
  lq_check(lq_rmsnorm_half(x, w_bf16, out, reinterpret_cast<uint16_t*>(xh), xinv, rows, H, eps, gemma ? 1 : 0, s));
}
inline void stream_gemm_nvfp4(const __half* x, const float* xinv, int M, const uint8_t* w, const uint8_t* wscale,
                              float scale2, float* y, int N, int K, hipStream_t s) {
  lq_check(lq_stream_gemm_nvfp4(reinterpret_cast<const uint16_t*>(x), xinv, M, w, wscale, scale2, y, N, K, s));
}
inline void stream_gemm_fp8(const __half* x, const float* xinv, int M, const uint8_t* w, float wscale, float* y, int N,
                            int K, hipStream_t s) {
  lq_check(lq_stream_gemm_fp8(reinterpret_cast<const uint16_t*>(x), xinv, M, w, wscale, y, N, K, s));
}
inline void stream_gemm_multi(bool nvfp4, const __half* x, const float* xinv, int M, const StreamTarget* t, int n, int K,
                              hipStream_t s) {
  lq_stream_target c[4];
  if (n < 1 || n > 4 || !t) throw std::runtime_error("stream_gemm: 1 to 4 matrices per launch");
  for (int i = 0; i < n; ++i) c[i] = lq_stream_target{t[i].w, t[i].wscale, t[i].scale, t[i].y, t[i].N};
  lq_check(lq_stream_gemm_multi(nvfp4 ? 1 : 0, reinterpret_cast<const uint16_t*>(x), xinv, M, c, n, K, s));
}

inline void stream_gemm_gather_nvfp4(const uint16_t* xh, const float* xinv, int M, const uint8_t* w,
                                     const uint8_t* raw_scales, float scale2, const int* rows, const int* nrows,
                                     int cap, float* y, int K, int N, hipStream_t s) {
  lq_check(lq_stream_gemm_gather_nvfp4(xh, xinv, M, w, raw_scales, scale2, rows, nrows, cap, y, K, N, s));
}

inline void l2_prefetch_weights(const uint8_t* w, bool fp4, bool coded, int N, int K, size_t bytes, hipStream_t s) {
  lq_check(lq_l2_prefetch_weights(w, fp4 ? 1 : 0, coded ? 1 : 0, N, K, bytes, s));
}

// ---- rows path, BF16 formats (additive) ----
inline void stream_fp8_pc(const uint16_t* x, int M, const uint8_t* w, const float* wscale_n, uint16_t* y, int N, int K,
                          hipStream_t s) {
  lq_check(lq_stream_fp8_pc(x, M, w, wscale_n, y, N, K, s));
}
inline void stream_fp8_pc_silu_mul(const uint16_t* x, int M, const uint8_t* w_gate, const float* s_gate,
                                   const uint8_t* w_up, const float* s_up, uint16_t* h, int N, int K, hipStream_t s) {
  lq_check(lq_stream_fp8_pc_silu_mul(x, M, w_gate, s_gate, w_up, s_up, h, N, K, s));
}
inline void stream_fp8_pc_residual(const uint16_t* x, int M, const uint8_t* w, const float* wscale_n,
                                   const uint16_t* resid, uint16_t* y, int N, int K, hipStream_t s) {
  lq_check(lq_stream_fp8_pc_residual(x, M, w, wscale_n, resid, y, N, K, s));
}
inline void stream_fp8_pc_ffn(const uint16_t* x, int M, const uint8_t* w_gate, const float* s_gate,
                              const uint8_t* w_up, const float* s_up, const uint8_t* w_down, const float* s_down,
                              const uint16_t* resid, uint16_t* h, uint16_t* y, int I, int H, hipStream_t s) {
  lq_check(lq_stream_fp8_pc_ffn(x, M, w_gate, s_gate, w_up, s_up, w_down, s_down, resid, h, y, I, H, s));
}
inline void stream_nvfp4_bf16(const uint16_t* x, int M, const uint8_t* w, const uint8_t* table, float scale2,
                              uint16_t* y, int N, int K, hipStream_t s) {
  lq_check(lq_stream_nvfp4_bf16(x, M, w, table, scale2, y, N, K, s));
}

// ---- prefill, NVFP4 (kernels.cuh:207-221) ----
inline void prefill_gemm_nvfp4(const uint8_t* xq, const uint8_t* xs, int M, const uint8_t* w, float alpha, float* y,
                               int ldy, int N, int K, bool accumulate, hipStream_t s, const uint8_t* wsf = nullptr) {
  lq_check(lq_prefill_gemm_nvfp4(xq, xs, M, w, alpha, y, ldy, N, K, accumulate ? 1 : 0, s, wsf));
}
inline void prefill_swiglu_nvfp4(const uint8_t* xq, const uint8_t* xs, int M, const uint8_t* gate, float alpha_gate,
                                 const uint8_t* up, float alpha_up, int N, int K, float out_input_scale, uint8_t* q_out,
                                 uint8_t* sf_out, hipStream_t s, const uint8_t* gate_sf = nullptr,
                                 const uint8_t* up_sf = nullptr) {
  lq_check(lq_prefill_swiglu_nvfp4(xq, xs, M, gate, alpha_gate, up, alpha_up, N, K, out_input_scale, q_out, sf_out, s,
                                   gate_sf, up_sf));
}

// ---- prefill activation producers (kernels.cuh:190-206) ----
inline void quant_act_nvfp4(const float* x, int M, int K, float input_scale, uint8_t* q, uint8_t* sf, hipStream_t s) {
  lq_check(lq_quant_act_nvfp4(x, M, K, input_scale, q, sf, s));
}
inline void silu_mul_quant_nvfp4(const float* g, const float* u, int M, int K, float input_scale, uint8_t* q,
                                 uint8_t* sf, hipStream_t s) {
  lq_check(lq_silu_mul_quant_nvfp4(g, u, M, K, input_scale, q, sf, s));
}
inline void rmsnorm_quant(const float* x, const uint16_t* w, float* out, int M, int H, float eps, bool nvfp4,
                          float input_scale, uint8_t* q, uint8_t* sf, hipStream_t s) {
  lq_check(lq_rmsnorm_quant(x, w, out, M, H, eps, nvfp4 ? 1 : 0, input_scale, q, sf, s));
}
// kernels.cuh:234-235 (BF16 as uint16_t bits)
inline void rmsnorm_quant_bf16(const float* x, const uint16_t* w, uint16_t* out, int M, int H, float eps, bool nvfp4,
                               float input_scale, uint8_t* q, uint8_t* sf, hipStream_t s) {
  lq_check(lq_rmsnorm_quant_bf16(x, w, out, M, H, eps, nvfp4 ? 1 : 0, input_scale, q, sf, s));
}

// ---- prefill (block-scaled FP8; kernels.cuh:190-221 for the reference's per-tensor forms) ----
inline void quant_act_fp8_g128(const uint16_t* x_bf16, int M, int K, uint8_t* q, float* scale, hipStream_t s) {
  lq_check(lq_quant_act_fp8_g128(x_bf16, M, K, q, scale, s));
}
inline void quant_act_fp8(const float* x, int M, int K, float input_scale, uint8_t* q, hipStream_t s) {
  lq_check(lq_quant_act_fp8(x, M, K, input_scale, q, s));
}
// kernels.cuh:237
inline void quant_act_fp8_bf16in(const uint16_t* x_bf16, int M, int K, float input_scale, uint8_t* q, hipStream_t s) {
  lq_check(lq_quant_act_fp8_bf16in(x_bf16, M, K, input_scale, q, s));
}
// DeltaNet / attention FP8 producers (kernels.cuh:205-207, 244-246)
inline void gated_rmsnorm_fp8(const float* x, const float* z, const uint16_t* w, int rows, int D, float eps,
                              float input_scale, uint8_t* q, hipStream_t s) {
  lq_check(lq_gated_rmsnorm_fp8(x, z, w, rows, D, eps, input_scale, q, s));
}
inline void gated_rmsnorm_fp8_bf16(const uint16_t* x, const uint16_t* z, const uint16_t* w, int rows, int D, float eps,
                                   float input_scale, uint8_t* q, hipStream_t s) {
  lq_check(lq_gated_rmsnorm_fp8_bf16(x, z, w, rows, D, eps, input_scale, q, s));
}
inline void sigmoid_mul_fp8(const float* x, const float* gate, size_t n, float input_scale, uint8_t* q, hipStream_t s) {
  lq_check(lq_sigmoid_mul_fp8(x, gate, n, input_scale, q, s));
}
inline void prefill_gemm_fp8(const uint8_t* xq, int M, const uint8_t* w, float alpha, float* y, int ldy, int N, int K,
                             bool accumulate, hipStream_t s) {
  lq_check(lq_prefill_gemm_fp8(xq, M, w, alpha, y, ldy, N, K, accumulate ? 1 : 0, s));
}
inline void prefill_gemm_fp8_bf16out(const uint8_t* xq, int M, const uint8_t* w, float alpha, uint16_t* y_bf16, int ldy,
                                     int N, int K, hipStream_t s) {
  lq_check(lq_prefill_gemm_fp8_bf16out(xq, M, w, alpha, y_bf16, ldy, N, K, s));
}
inline void prefill_gemm_fp8_block(const uint8_t* xq, const float* xs, int M, const uint8_t* w, const float* ws,
                                   uint16_t* y_bf16, int ldy, int N, int K, hipStream_t s) {
  lq_check(lq_prefill_fp8_block(xq, xs, M, w, ws, y_bf16, ldy, N, K, s));
}

// ---- host weight quantizers (CPU threads; model.cu:188-249 quantize_nvfp4, and the configs' FP8 recipes) ----
// Returns g (scale2); rel_sq_err may be null.
inline float quantize_nvfp4(const uint16_t* w_bf16, int N, int K, uint8_t* values, uint8_t* scales,
                            double* rel_sq_err = nullptr) {
  float g = 0.f;
  lq_check(lq_quantize_nvfp4(w_bf16, N, K, values, scales, &g, rel_sq_err));
  return g;
}
inline void quantize_fp8_channel(const void* w, int dtype, int N, int K, uint8_t* q, float* scale) {
  lq_check(lq_quantize_fp8_channel(w, dtype, N, K, q, scale));
}
inline void quantize_fp8_block128(const void* w, int dtype, int N, int K, uint8_t* q, float* scale) {
  lq_check(lq_quantize_fp8_block128(w, dtype, N, K, q, scale));
}

}  // namespace ling::kernels
