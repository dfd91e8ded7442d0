// Activation producers of the prefill GEMMs, fused with their quantization (reference
// src/core/prefill_gemm.cu:378-494, 607-665): the NVFP4 activation quantizer, the same on silu(g) * u, the
// Gemma RMSNorm straight into FP8 or NVFP4, the DeltaNet gated output norm and the attention's sigmoid gate into
// FP8. Every value is rounded to BF16 first (production's activations are
// BF16), as the reference does.
//
// NVFP4 (reference put_nvfp4, prefill_gemm.cu:382-394): per block of 16 consecutive values along K,
//   g = 1 / input_scale, sc = E4M3_rne_satfinite(g * (amax * (1/6))), os = sv != 0 ? 1 / (sv * (1/g)) : 0
//   (sv = the E4M3 value of sc), codes = E2M1 round-to-nearest-even, saturating, sign kept (a small negative
//   value gives code 8), low nibble first.
// One thread per 16-value block: 64 bytes in, 9 bytes out; consecutive threads read consecutive blocks.
#include "lq_common.hpp"

#include <string>

namespace lq {
namespace {

// E4M3, round to nearest even, saturating to +-448 (NaN stays NaN).
__device__ __forceinline__ uint32_t e4m3_sat(float v) {
  return __builtin_amdgcn_cvt_pk_fp8_f32(isnan(v) ? v : fminf(fmaxf(v, -448.f), 448.f), 0.f, 0, false) & 0xffu;
}

__device__ __forceinline__ float bf16_round(float x) { return bf16_to_f32(f32_to_bf16(x)); }

__device__ __forceinline__ float silu_ref(float x) { return x / (1.f + __expf(-x)); }

// Block b's 16 values (already BF16-rounded) -> 8 code bytes and the scale byte.
__device__ __forceinline__ void put_nvfp4_block(const float (&v)[16], float g, uint8_t* q8, uint8_t* sfb) {
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
  const uint32_t sc = e4m3_sat(g * (amax * (1.f / 6.f)));
  const float sv = e4m3_to_f32(sc);
  const float os = sv != 0.f ? 1.f / (sv * (1.f / g)) : 0.f;
  uint32_t w[2] = {0u, 0u};
#pragma unroll
  for (int i = 0; i < 16; i += 2) {
    const uint32_t byte = e2m1x2_rne(v[i] * os, v[i + 1] * os);
    w[i >> 3] |= byte << (8 * ((i >> 1) & 3));
  }
  *reinterpret_cast<u32x2*>(q8) = u32x2{w[0], w[1]};
  *sfb = static_cast<uint8_t>(sc);
}

template <bool SILU>
__global__ void __launch_bounds__(256) quant_nvfp4_kernel(const float* __restrict__ x, const float* __restrict__ u,
                                                          size_t blocks, float g, uint8_t* __restrict__ q,
                                                          uint8_t* __restrict__ sf) {
  for (size_t b = blockIdx.x * static_cast<size_t>(256) + threadIdx.x; b < blocks;
       b += static_cast<size_t>(gridDim.x) * 256) {
    float v[16];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const f32x4 f = reinterpret_cast<const f32x4*>(x)[b * 4 + k];
      f32x4 uu = f32x4{1.f, 1.f, 1.f, 1.f};
      if constexpr (SILU) uu = reinterpret_cast<const f32x4*>(u)[b * 4 + k];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[4 * k + e] = bf16_round(SILU ? silu_ref(f[e]) * uu[e] : f[e]);
    }
    put_nvfp4_block(v, g, q + b * 8, sf + b);
  }
}

// One workgroup per row, one thread per 16-value block (NB <= 4 blocks per thread when the row has more than 1024,
// so H <= 65536), the row held in registers from a single read: the sum of squares (each thread's values in
// order, then the wave, then the waves in order), rstd = 1 / sqrt(sum / H + eps), v = x * rstd * (1 + w)
// (written to `out` when given), then the thread quantizes its blocks of BF16(v): NVFP4, or FP8
// E4M3(BF16(v) * (1 / input_scale)).
// BF16OUT: `out` is BF16, the values rounded as the quantizer rounds them (reference rmsnorm_quant_bf16,
// prefill_gemm.cu:640-645, the norm_quant_kernel's OutT = BF16 form).
template <bool FP4, int NB, bool BF16OUT>
__global__ void __launch_bounds__(1024) rmsnorm_quant_kernel(const float* __restrict__ x, const uint16_t* __restrict__ w,
                                                             void* __restrict__ out, int H, float eps, float g,
                                                             uint8_t* __restrict__ q, uint8_t* __restrict__ sf) {
  __shared__ float red[16];
  const size_t r = blockIdx.x;
  const int nblk = H / 16, T = static_cast<int>(blockDim.x);
  const float* row = x + r * H;
  f32x4 f[NB][4];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int blk = static_cast<int>(threadIdx.x) + j * T;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      f[j][k] = blk < nblk ? reinterpret_cast<const f32x4*>(row)[blk * 4 + k] : f32x4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int e = 0; e < 4; ++e) ss = __builtin_fmaf(f[j][k][e], f[j][k][e], ss);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
  for (int i = 0; i < T / 64; ++i) tot += red[i];
  const float rstd = 1.f / sqrtf(tot / static_cast<float>(H) + eps);
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int blk = static_cast<int>(threadIdx.x) + j * T;
    if (blk >= nblk) continue;
    const u32x4 w0 = reinterpret_cast<const u32x4*>(w)[blk * 2], w1 = reinterpret_cast<const u32x4*>(w)[blk * 2 + 1];
    const uint32_t wp[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
    float v[16];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int h = 4 * k + e;
        const uint32_t wb = (h & 1) ? wp[h >> 1] >> 16 : wp[h >> 1] & 0xffff;
        v[h] = f[j][k][e] * rstd * (1.f + bf16_to_f32(wb));
      }
      if (out && !BF16OUT)
        reinterpret_cast<f32x4*>(static_cast<float*>(out) + r * H)[blk * 4 + k] =
            f32x4{v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
    }
    uint32_t ob[8];
#pragma unroll
    for (int i = 0; i < 16; i += 2) ob[i >> 1] = f32_to_bf16(v[i]) | (uint32_t(f32_to_bf16(v[i + 1])) << 16);
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = bf16_round(v[i]);
    if (out && BF16OUT) {
      u32x4* o = reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) + r * H + static_cast<size_t>(blk) * 16);
      o[0] = u32x4{ob[0], ob[1], ob[2], ob[3]};
      o[1] = u32x4{ob[4], ob[5], ob[6], ob[7]};
    }
    const size_t b = r * nblk + blk;
    if constexpr (FP4) {
      put_nvfp4_block(v, g, q + b * 8, sf + b);
    } else {
      uint32_t wq[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        wq[k] = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) wq[k] |= e4m3_sat(v[4 * k + e] * g) << (8 * e);
      }
      reinterpret_cast<u32x4*>(q)[b] = u32x4{wq[0], wq[1], wq[2], wq[3]};
    }
  }
}

template <bool FP4, bool BF16OUT>
void rmsnorm_launch(int M, int H, hipStream_t s, const float* x, const uint16_t* w, void* out, float eps, float g,
                    uint8_t* q, uint8_t* sf) {
  const int nblk = H / 16;
  const int T = nblk < 1024 ? nblk : 1024;  // H % 1024 == 0: a multiple of 64
  const int nb = (nblk + T - 1) / T;
  if (nb == 1)
    hipLaunchKernelGGL((rmsnorm_quant_kernel<FP4, 1, BF16OUT>), dim3(M), dim3(T), 0, s, x, w, out, H, eps, g, q, sf);
  else if (nb == 2)
    hipLaunchKernelGGL((rmsnorm_quant_kernel<FP4, 2, BF16OUT>), dim3(M), dim3(T), 0, s, x, w, out, H, eps, g, q, sf);
  else hipLaunchKernelGGL((rmsnorm_quant_kernel<FP4, 4, BF16OUT>), dim3(M), dim3(T), 0, s, x, w, out, H, eps, g, q, sf);
}

int rmsnorm_quant_any(const char* name, const float* x, const uint16_t* w, void* out, bool bf16out, int M, int H,
                      float eps, int nvfp4, float input_scale, uint8_t* q, uint8_t* sf, void* stream) {
  const std::string nm(name);
  if (M < 1) return fail(LQ_ERR_SHAPE, nm + ": M must be positive");
  if (H <= 0 || H % 1024 != 0) return fail(LQ_ERR_SHAPE, nm + ": H % 1024 must be 0");
  if (H > 65536) return fail(LQ_ERR_SHAPE, nm + ": H must be at most 65536 (the row is held in registers)");
  if (!x || !w || !q || (nvfp4 && !sf)) return fail(LQ_ERR_ARG, nm + ": null pointer");
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(out) |
       reinterpret_cast<uintptr_t>(q)) % 16 != 0)
    return fail(LQ_ERR_ARG, nm + ": x, w, out and q must be 16-byte aligned");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const float g = 1.f / input_scale;
  if (nvfp4) {
    if (bf16out) rmsnorm_launch<true, true>(M, H, s, x, w, out, eps, g, q, sf);
    else rmsnorm_launch<true, false>(M, H, s, x, w, out, eps, g, q, sf);
  } else {
    if (bf16out) rmsnorm_launch<false, true>(M, H, s, x, w, out, eps, g, q, nullptr);
    else rmsnorm_launch<false, false>(M, H, s, x, w, out, eps, g, q, nullptr);
  }
  return check_launch(name);
}

// FP8 E4M3 of four BF16-rounded values times inv_scale, saturating, packed low byte first (reference put_fp8x4,
// prefill_gemm.cu:396-402).
__device__ __forceinline__ uint32_t fp8x4(const float (&v)[4], float inv_scale) {
  uint32_t w = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) w |= e4m3_sat(v[k] * inv_scale) << (8 * k);
  return w;
}

__device__ __forceinline__ f32x4 load4(const float* p, size_t i) { return reinterpret_cast<const f32x4*>(p)[i]; }
__device__ __forceinline__ f32x4 load4(const uint16_t* p, size_t i) {
  const u32x2 u = reinterpret_cast<const u32x2*>(p)[i];
  return f32x4{__uint_as_float(u[0] << 16), __uint_as_float(u[0] & 0xffff0000u), __uint_as_float(u[1] << 16),
               __uint_as_float(u[1] & 0xffff0000u)};
}

// The DeltaNet output norm over heads of D = 128 (reference gated_norm_fp8_kernel, prefill_gemm.cu:461-482):
// v = BF16(x * rstd * w * silu(z)), q = E4M3_sat(v * inv_scale). One row per half wave (32 lanes, four values
// each), so a 64-wide wave finishes two rows from two 512-byte FP32 reads per operand. The sum of squares is
// the reference's order: per lane fma(x3, x3, fma(x2, x2, fma(x1, x1, x0 * x0))), then the xor butterfly over
// lane distances 16, 8, 4, 2, 1 inside the half wave (every lane ends with the same tree sum);
// rstd = 1 / sqrt(ss / 128 + eps), both operations rounded correctly.
template <typename InT>
__global__ void __launch_bounds__(256) gated_norm_fp8_kernel(const InT* __restrict__ x, const InT* __restrict__ z,
                                                             const uint16_t* __restrict__ w, size_t rows, float eps,
                                                             float inv_scale, uint8_t* __restrict__ q) {
  const size_t r = blockIdx.x * static_cast<size_t>(8) + (threadIdx.x >> 5);
  if (r >= rows) return;
  const int lane = threadIdx.x & 31;
  const f32x4 f = load4(x, r * 32 + lane);
  const f32x4 g = load4(z, r * 32 + lane);
  float ss = f[0] * f[0];
  ss = __builtin_fmaf(f[1], f[1], ss);
  ss = __builtin_fmaf(f[2], f[2], ss);
  ss = __builtin_fmaf(f[3], f[3], ss);
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 32);
  const float rstd = 1.f / sqrtf(ss / 128.f + eps);
  const f32x4 wv = load4(w, lane);
  float v[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) v[k] = bf16_round(f[k] * rstd * wv[k] * silu_ref(g[k]));
  reinterpret_cast<uint32_t*>(q)[r * 32 + lane] = fp8x4(v, inv_scale);
}

// x * sigmoid(gate) into FP8 (reference sigmoid_mul_fp8_kernel, prefill_gemm.cu:484-494): v = BF16(x / (1 +
// e^-gate)), q = E4M3_sat(v * inv_scale); four values per thread, grid-stride.
__global__ void __launch_bounds__(256) sigmoid_mul_fp8_kernel(const float* __restrict__ x, const float* __restrict__ gate,
                                                              size_t quads, float inv_scale, uint8_t* __restrict__ q) {
  for (size_t i = blockIdx.x * static_cast<size_t>(256) + threadIdx.x; i < quads;
       i += static_cast<size_t>(gridDim.x) * 256) {
    const f32x4 f = load4(x, i), g = load4(gate, i);
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = bf16_round(f[k] / (1.f + __expf(-g[k])));
    reinterpret_cast<uint32_t*>(q)[i] = fp8x4(v, inv_scale);
  }
}

template <typename InT>
int gated_norm_launch(const char* name, const InT* x, const InT* z, const uint16_t* w, int rows, int D, float eps,
                      float input_scale, uint8_t* q, void* stream) {
  const std::string nm(name);
  if (D != 128) return fail(LQ_ERR_SHAPE, nm + ": D must be 128");
  if (rows < 0) return fail(LQ_ERR_SHAPE, nm + ": rows must not be negative");
  if (rows == 0) return LQ_OK;
  if (!x || !z || !w || !q) return fail(LQ_ERR_ARG, nm + ": null pointer");
  const uintptr_t a = sizeof(InT) * 4;
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(z)) % a != 0 ||
      (reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(q)) % 8 != 0)
    return fail(LQ_ERR_ARG, nm + ": x and z must be " + std::to_string(a) + "-byte, w and q 8-byte aligned");
  hipLaunchKernelGGL(gated_norm_fp8_kernel<InT>, dim3((rows + 7) / 8), dim3(256), 0, static_cast<hipStream_t>(stream),
                     x, z, w, static_cast<size_t>(rows), eps, 1.f / input_scale, q);
  return check_launch(name);
}

unsigned grid_for(size_t items) {
  const size_t b = (items + 255) / 256;
  return static_cast<unsigned>(b < 8192 ? (b ? b : 1) : 8192);
}

}  // namespace
}  // namespace lq

using namespace lq;

extern "C" {

int lq_quant_act_nvfp4(const float* x, int M, int K, float input_scale, uint8_t* q, uint8_t* sf, void* stream) {
  if (M < 1 || K <= 0 || K % 16 != 0) return fail(LQ_ERR_SHAPE, "quant_act_nvfp4: M >= 1 and K % 16 == 0");
  if (!x || !q || !sf) return fail(LQ_ERR_ARG, "quant_act_nvfp4: null pointer");
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(q) % 8 != 0)
    return fail(LQ_ERR_ARG, "quant_act_nvfp4: x must be 16-byte and q 8-byte aligned");
  const size_t blocks = static_cast<size_t>(M) * K / 16;
  hipLaunchKernelGGL(quant_nvfp4_kernel<false>, dim3(grid_for(blocks)), dim3(256), 0, static_cast<hipStream_t>(stream), x,
                     nullptr, blocks, 1.f / input_scale, q, sf);
  return check_launch("quant_act_nvfp4");
}

int lq_silu_mul_quant_nvfp4(const float* g, const float* u, int M, int K, float input_scale, uint8_t* q, uint8_t* sf,
                            void* stream) {
  if (M < 1 || K <= 0 || K % 16 != 0) return fail(LQ_ERR_SHAPE, "silu_mul_quant_nvfp4: M >= 1 and K % 16 == 0");
  if (!g || !u || !q || !sf) return fail(LQ_ERR_ARG, "silu_mul_quant_nvfp4: null pointer");
  if ((reinterpret_cast<uintptr_t>(g) | reinterpret_cast<uintptr_t>(u)) % 16 != 0 || reinterpret_cast<uintptr_t>(q) % 8 != 0)
    return fail(LQ_ERR_ARG, "silu_mul_quant_nvfp4: g and u must be 16-byte and q 8-byte aligned");
  const size_t blocks = static_cast<size_t>(M) * K / 16;
  hipLaunchKernelGGL(quant_nvfp4_kernel<true>, dim3(grid_for(blocks)), dim3(256), 0, static_cast<hipStream_t>(stream), g,
                     u, blocks, 1.f / input_scale, q, sf);
  return check_launch("silu_mul_quant_nvfp4");
}

int lq_rmsnorm_quant(const float* x, const uint16_t* w, float* out, int M, int H, float eps, int nvfp4,
                     float input_scale, uint8_t* q, uint8_t* sf, void* stream) {
  return rmsnorm_quant_any("rmsnorm_quant", x, w, out, false, M, H, eps, nvfp4, input_scale, q, sf, stream);
}

int lq_rmsnorm_quant_bf16(const float* x, const uint16_t* w, uint16_t* out, int M, int H, float eps, int nvfp4,
                          float input_scale, uint8_t* q, uint8_t* sf, void* stream) {
  return rmsnorm_quant_any("rmsnorm_quant_bf16", x, w, out, true, M, H, eps, nvfp4, input_scale, q, sf, stream);
}

int lq_gated_rmsnorm_fp8(const float* x, const float* z, const uint16_t* w, int rows, int D, float eps,
                         float input_scale, uint8_t* q, void* stream) {
  return gated_norm_launch("gated_rmsnorm_fp8", x, z, w, rows, D, eps, input_scale, q, stream);
}

int lq_gated_rmsnorm_fp8_bf16(const uint16_t* x, const uint16_t* z, const uint16_t* w, int rows, int D, float eps,
                              float input_scale, uint8_t* q, void* stream) {
  return gated_norm_launch("gated_rmsnorm_fp8_bf16", x, z, w, rows, D, eps, input_scale, q, stream);
}

int lq_sigmoid_mul_fp8(const float* x, const float* gate, size_t n, float input_scale, uint8_t* q, void* stream) {
  if (n % 4 != 0) return fail(LQ_ERR_SHAPE, "sigmoid_mul_fp8: n % 4 must be 0");
  if (n == 0) return LQ_OK;
  if (!x || !gate || !q) return fail(LQ_ERR_ARG, "sigmoid_mul_fp8: null pointer");
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(gate)) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(q) % 4 != 0)
    return fail(LQ_ERR_ARG, "sigmoid_mul_fp8: x and gate must be 16-byte and q 4-byte aligned");
  hipLaunchKernelGGL(sigmoid_mul_fp8_kernel, dim3(grid_for(n / 4)), dim3(256), 0, static_cast<hipStream_t>(stream), x,
                     gate, n / 4, 1.f / input_scale, q);
  return check_launch("sigmoid_mul_fp8");
}

}  // extern "C"
