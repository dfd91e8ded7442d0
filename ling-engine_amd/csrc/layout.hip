// The tiled ("kernel-order") weight layout on the device: retile from the checkpoint's row-major codes and
// dequantize back (reference src/core/stream_gemm.cu:705-820, kernels.cuh:162-188). Byte-identical to the
// reference's layout: FP8 block (tile, chunk) is 2048 bytes whose 16-byte piece ((h*2+q)*8+g)*4+t holds
// W[16 tile + g + 8h][128 chunk + 32t + 16q, +16); NVFP4 block is 1152 bytes whose slot r*4+t holds the
// 16 value bytes of W[16 tile + r][128 chunk + 32t, +32) with its 2 E4M3 scales at 1024 + 2 slot.
// One thread per 16-byte piece; the grid strides over the blob. These run once per weight at load time
// (and in tests), so they are written for clarity, with coalesced 16-byte stores.
#include "lq_common.hpp"

#include <algorithm>
#include <string>

namespace lq {
namespace {

int grid_of(size_t n) { return static_cast<int>(std::min<size_t>((n + 255) / 256, size_t(1) << 20)); }

__global__ void retile_fp8_kernel(const uint8_t* __restrict__ w, uint8_t* __restrict__ out, int N, int K) {
  const int C = K / kChunk;
  const size_t pieces = static_cast<size_t>(N / 16) * C * 128;
  for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < pieces; i += size_t(gridDim.x) * blockDim.x) {
    const size_t blk = i >> 7;
    const int p = static_cast<int>(i & 127);
    const int t = p & 3, g = (p >> 2) & 7, q = (p >> 5) & 1, h = p >> 6;
    const size_t n = (blk / C) * 16 + g + 8 * h;
    const size_t k = (blk % C) * kChunk + 32 * t + 16 * q;
    *reinterpret_cast<u32x4*>(out + i * 16) = *reinterpret_cast<const u32x4*>(w + n * K + k);
  }
}

__global__ void retile_nvfp4_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ sc,
                                    uint8_t* __restrict__ out, int N, int K) {
  const int C = K / kChunk;
  const size_t slots = static_cast<size_t>(N / 16) * C * 64;
  for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < slots; i += size_t(gridDim.x) * blockDim.x) {
    const size_t blk = i >> 6;
    const int s = static_cast<int>(i & 63), r = s >> 2, t = s & 3;
    const size_t n = (blk / C) * 16 + r, c = blk % C;
    uint8_t* b = out + blk * kTileBytesFp4;
    *reinterpret_cast<u32x4*>(b + s * 16) = *reinterpret_cast<const u32x4*>(w + n * (K / 2) + c * 64 + t * 16);
    const uint8_t* ss = sc + n * (K / 16) + c * 8 + t * 2;
    b[1024 + s * 2] = ss[0];
    b[1024 + s * 2 + 1] = ss[1];
  }
}

// The coded blob: values at the 1024-byte block stride (one thread per slot), then each block's 96 code
// bytes and its raw scales (one thread per block).
__global__ void retile_nvfp4_coded_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ sc,
                                          const uint8_t* __restrict__ code_of, uint8_t* __restrict__ out,
                                          uint8_t* __restrict__ raw, int N, int K) {
  const int C = K / kChunk;
  const size_t blocks = static_cast<size_t>(N / 16) * C;
  for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < blocks * 64; i += size_t(gridDim.x) * blockDim.x) {
    const size_t blk = i >> 6;
    const int s = static_cast<int>(i & 63), r = s >> 2, t = s & 3;
    const size_t n = (blk / C) * 16 + r, c = blk % C;
    *reinterpret_cast<u32x4*>(out + blk * kValueBytesFp4 + s * 16) =
        *reinterpret_cast<const u32x4*>(w + n * (K / 2) + c * 64 + t * 16);
    const uint8_t* ss = sc + n * (K / 16) + c * 8 + t * 2;
    raw[blk * 128 + s * 2] = ss[0];
    raw[blk * 128 + s * 2 + 1] = ss[1];
    // slot s's 12-bit code pair (first scale low); slot s < 32 -> byte 2s and the low nibble of 64 + s,
    // slot 32 + L -> byte 2L + 1 and the high nibble of 64 + L
    const uint32_t f = uint32_t(code_of[ss[0]]) | (uint32_t(code_of[ss[1]]) << 6);
    uint8_t* cd = out + blocks * kValueBytesFp4 + blk * kCodeBytesFp4;
    const int L = s & 31, hi = s >> 5;
    cd[2 * L + hi] = static_cast<uint8_t>(f & 0xff);
    // two slots share the nibble byte: the low-half slot writes it after reading its partner's code
    if (hi == 0) {
      const uint8_t* sp = sc + ((blk / C) * 16 + ((s + 32) >> 2)) * (K / 16) + c * 8 + ((s + 32) & 3) * 2;
      const uint32_t f2 = uint32_t(code_of[sp[0]]) | (uint32_t(code_of[sp[1]]) << 6);
      cd[64 + L] = static_cast<uint8_t>((f >> 8) | ((f2 >> 8) << 4));
    }
  }
}

// dequant: one thread per element (FP8) or per value pair (NVFP4); the product order of the reference's
// dequant_tiled_* (stream_gemm.cu:797-818): FP8 e4m3 * wscale, NVFP4 e2m1 * (e4m3 * scale2).
template <bool F32OUT>
__global__ void dequant_fp8_kernel(const uint8_t* __restrict__ tw, const float* __restrict__ svec, float wscale,
                                   void* __restrict__ out, int N, int K) {
  const int C = K / kChunk;
  const size_t total = static_cast<size_t>(N) * K;
  for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < total; i += size_t(gridDim.x) * blockDim.x) {
    const int n = static_cast<int>(i / K), k = static_cast<int>(i % K);
    const int r = n & 15, kk = k & 127;
    const int p = (((r >> 3) * 2 + ((kk >> 4) & 1)) * 8 + (r & 7)) * 4 + (kk >> 5);
    const uint8_t b = tw[(static_cast<size_t>(n >> 4) * C + (k >> 7)) * kTileBytesFp8 + p * 16 + (kk & 15)];
    const float v = e4m3_to_f32(b) * (svec ? svec[n] : wscale);
    if (F32OUT) reinterpret_cast<float*>(out)[i] = v;
    else reinterpret_cast<uint16_t*>(out)[i] = f32_to_bf16(v);
  }
}

__device__ __forceinline__ float e2m1_to_f32(uint32_t nib) {
  const float mag[8] = {0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};
  const float v = mag[nib & 7];
  return (nib & 8) ? -v : v;
}

template <bool F32OUT>
__global__ void dequant_nvfp4_kernel(const uint8_t* __restrict__ tw, float scale2, void* __restrict__ out, int N, int K,
                                     const uint8_t* __restrict__ raw) {
  const int C = K / kChunk;
  const size_t pairs = static_cast<size_t>(N) * K / 2;
  for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < pairs; i += size_t(gridDim.x) * blockDim.x) {
    const int n = static_cast<int>(i / (K / 2)), k = static_cast<int>(i % (K / 2)) * 2;
    const int r = n & 15, kk = k & 127, s = r * 4 + (kk >> 5);
    const size_t blk = static_cast<size_t>(n >> 4) * C + (k >> 7);
    const uint8_t* base = tw + blk * (raw ? kValueBytesFp4 : kTileBytesFp4);
    const uint8_t b = base[s * 16 + ((kk & 31) >> 1)];
    const uint8_t scb = raw ? raw[blk * 128 + s * 2 + ((kk & 31) >> 4)] : base[1024 + s * 2 + ((kk & 31) >> 4)];
    const float sv = e4m3_to_f32(scb) * scale2;
    const float v0 = e2m1_to_f32(b & 15) * sv, v1 = e2m1_to_f32(b >> 4) * sv;
    const size_t o = static_cast<size_t>(n) * K + k;
    if (F32OUT) {
      reinterpret_cast<float*>(out)[o] = v0;
      reinterpret_cast<float*>(out)[o + 1] = v1;
    } else {
      reinterpret_cast<uint16_t*>(out)[o] = f32_to_bf16(v0);
      reinterpret_cast<uint16_t*>(out)[o + 1] = f32_to_bf16(v1);
    }
  }
}

int check_shape(int N, int K, const char* what) {
  if (N <= 0 || K <= 0 || N % 16 != 0 || K % kChunk != 0)
    return fail(LQ_ERR_SHAPE, std::string(what) + ": N % 16 and K % 128 must be 0");
  return LQ_OK;
}

}  // namespace
}  // namespace lq

using namespace lq;

extern "C" {

size_t lq_tiled_bytes_fp8(int N, int K) { return static_cast<size_t>(N) * K; }
size_t lq_tiled_bytes_nvfp4(int N, int K) { return static_cast<size_t>(N) * K / 2 + static_cast<size_t>(N) * K / 16; }
size_t lq_tiled_bytes_nvfp4_coded(int N, int K) {
  return static_cast<size_t>(N / 16) * (K / kChunk) * (kValueBytesFp4 + kCodeBytesFp4);
}

int lq_retile_fp8(const uint8_t* w, uint8_t* out, int N, int K, void* stream) {
  if (int rc = check_shape(N, K, "retile_fp8")) return rc;
  if (!w || !out) return fail(LQ_ERR_ARG, "retile_fp8: null pointer");
  hipLaunchKernelGGL(retile_fp8_kernel, dim3(grid_of(size_t(N) * K / 16)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     w, out, N, K);
  return check_launch("retile_fp8");
}

int lq_retile_nvfp4(const uint8_t* w, const uint8_t* wscale, uint8_t* out, int N, int K, void* stream) {
  if (int rc = check_shape(N, K, "retile_nvfp4")) return rc;
  if (!w || !wscale || !out) return fail(LQ_ERR_ARG, "retile_nvfp4: null pointer");
  hipLaunchKernelGGL(retile_nvfp4_kernel, dim3(grid_of(size_t(N) * K / 32)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), w, wscale, out, N, K);
  return check_launch("retile_nvfp4");
}

int lq_scale_code_table(const uint8_t* scales, size_t n, uint8_t* table, uint8_t* code_of) {
  if (!scales || !table || !code_of) return fail(LQ_ERR_ARG, "scale_code_table: null pointer");
  size_t count[256] = {};
  for (size_t i = 0; i < n; ++i) ++count[scales[i]];
  int distinct = 0;
  for (int v = 0; v < 256; ++v) distinct += count[v] > 0;
  if (distinct > 64) return 0;
  for (int i = 0; i < 64; ++i) table[i] = 0;
  for (int v = 0; v < 256; ++v) code_of[v] = 0xff;
  int next = 0;
  for (int v = 0; v < 256; ++v)
    if (count[v]) {
      code_of[v] = static_cast<uint8_t>(next);
      table[next++] = static_cast<uint8_t>(v);
    }
  return 1;
}

int lq_retile_nvfp4_coded(const uint8_t* w, const uint8_t* wscale, const uint8_t* code_of_dev, uint8_t* out,
                          uint8_t* raw_scales, int N, int K, void* stream) {
  if (int rc = check_shape(N, K, "retile_nvfp4_coded")) return rc;
  if (!w || !wscale || !code_of_dev || !out || !raw_scales) return fail(LQ_ERR_ARG, "retile_nvfp4_coded: null pointer");
  hipLaunchKernelGGL(retile_nvfp4_coded_kernel, dim3(grid_of(size_t(N) * K / 32)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), w, wscale, code_of_dev, out, raw_scales, N, K);
  return check_launch("retile_nvfp4_coded");
}

int lq_dequant_tiled_fp8(const uint8_t* tw, float wscale, uint16_t* out, int N, int K, void* stream) {
  if (int rc = check_shape(N, K, "dequant_tiled_fp8")) return rc;
  if (!tw || !out) return fail(LQ_ERR_ARG, "dequant_tiled_fp8: null pointer");
  hipLaunchKernelGGL(dequant_fp8_kernel<false>, dim3(grid_of(size_t(N) * K)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), tw, nullptr, wscale, out, N, K);
  return check_launch("dequant_tiled_fp8");
}

int lq_dequant_tiled_fp8_pc_f32(const uint8_t* tw, const float* wscale_n, float* out, int N, int K, void* stream) {
  if (int rc = check_shape(N, K, "dequant_tiled_fp8_pc_f32")) return rc;
  if (!tw || !wscale_n || !out) return fail(LQ_ERR_ARG, "dequant_tiled_fp8_pc_f32: null pointer");
  hipLaunchKernelGGL(dequant_fp8_kernel<true>, dim3(grid_of(size_t(N) * K)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), tw, wscale_n, 0.f, out, N, K);
  return check_launch("dequant_tiled_fp8_pc_f32");
}

int lq_dequant_tiled_nvfp4(const uint8_t* tw, float scale2, uint16_t* out, int N, int K, void* stream,
                           const uint8_t* raw_scales) {
  if (int rc = check_shape(N, K, "dequant_tiled_nvfp4")) return rc;
  if (!tw || !out) return fail(LQ_ERR_ARG, "dequant_tiled_nvfp4: null pointer");
  hipLaunchKernelGGL(dequant_nvfp4_kernel<false>, dim3(grid_of(size_t(N) * K / 2)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), tw, scale2, out, N, K, raw_scales);
  return check_launch("dequant_tiled_nvfp4");
}

int lq_dequant_tiled_nvfp4_f32(const uint8_t* tw, float scale2, float* out, int N, int K, void* stream,
                               const uint8_t* raw_scales) {
  if (int rc = check_shape(N, K, "dequant_tiled_nvfp4_f32")) return rc;
  if (!tw || !out) return fail(LQ_ERR_ARG, "dequant_tiled_nvfp4_f32: null pointer");
  hipLaunchKernelGGL(dequant_nvfp4_kernel<true>, dim3(grid_of(size_t(N) * K / 2)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), tw, scale2, out, N, K, raw_scales);
  return check_launch("dequant_tiled_nvfp4_f32");
}

}  // extern "C"
