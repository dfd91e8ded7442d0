// Shared device/host helpers for the gfx950 quantized GEMM library: vector types, exact FP8/FP4
// conversions on CDNA4's conversion instructions, MFMA wrappers, the per-thread error state of the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "ling_gemm.h"

namespace lq {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
typedef __attribute__((ext_vector_type(8))) int i32x8;

constexpr int kChunk = 128;                       // K values per tiled block
constexpr int kTileBytesFp8 = 16 * 128;           // one (16-row tile, 128-value chunk) FP8 block
constexpr int kTileBytesFp4 = 16 * 64 + 16 * 8;   // NVFP4 values then E4M3 scales
constexpr int kValueBytesFp4 = 16 * 64;           // coded NVFP4: value block
constexpr int kCodeBytesFp4 = 96;                 // coded NVFP4: 6-bit scale codes per block
constexpr int kWave = 64;

// ---- error state of the C ABI (per host thread) ----
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

// ---- exact conversions (CDNA4 v_cvt_scalef32_* with scale 1.0: every FP8 / FP4 code is exact) ----
// Four E4M3 bytes of `v` -> four BF16 (byte 0 first).
__device__ __forceinline__ u32x2 fp8x4_to_bf16x4(uint32_t v) {
  const bf16x2 lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v, 1.0f, false);
  const bf16x2 hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v, 1.0f, true);
  return u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
}
__device__ __forceinline__ u32x2 fp8x4_to_f16x4(uint32_t v) {
  const f16x2 lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(v, 1.0f, false);
  const f16x2 hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(v, 1.0f, true);
  return u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
}
// Byte `sel` of v (two E2M1 codes, low nibble first) -> two FP16 (exact).
template <int SEL>
__device__ __forceinline__ f16x2 fp4x2_to_f16x2(uint32_t v) {
  return __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, 1.0f, SEL);
}
// Two values to E2M1 codes, the first in the low nibble: nearest, ties to the even code (values 0, .5, 1, 1.5, 2, 3,
// 4, 6), saturating at 6, the sign kept (a negative value that rounds to zero is code 8). The hardware conversion at
// scale 1, tested bit for bit against the oracle's encoding at every rounding midpoint and its BF16 neighbours (it
// replaced seven compares per value: the NVFP4 activation quantizers 16-23 % faster).
__device__ __forceinline__ uint32_t e2m1x2_rne(float lo, float hi) {
  return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, lo, hi, 1.0f, 0) & 0xffu;
}

__device__ __forceinline__ float e4m3_to_f32(uint32_t byte) {
  return __builtin_amdgcn_cvt_f32_fp8(byte, 0);
}

__device__ __forceinline__ f32x4 mfma16x16x32(const u32x4& a, const u32x4& b, const f32x4& c, bool f16) {
  if (f16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }
// Round to nearest even (NaN kept quiet).
// FP32 -> BF16, round to nearest even (gfx950's v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16(float x) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x)); }

__device__ __forceinline__ u32x4 load_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x4 load16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

__host__ __device__ constexpr int cdiv(int a, int b) { return (a + b - 1) / b; }

// Per-device facts the launchers need (CU count), read once per device.
int device_cus(int dev);

}  // namespace lq
