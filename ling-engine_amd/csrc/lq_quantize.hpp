// Host weight quantizers shared by the C ABI (quantize.cpp) and the weight-file compiler (weight_file.cpp).
#pragma once

#include <cstddef>
#include <cstdint>

#include "ling_gemm.h"

namespace lq {
namespace hostq {

uint8_t e4m3_encode(float x);  // OCP E4M3FN, round to nearest even, saturating to +-448; NaN -> 0x7f
float e4m3_decode(uint8_t c);
float bf16_to_f32(uint16_t b);
uint16_t f32_to_bf16(float x);  // round to nearest even
float f16_to_f32(uint16_t h);
// element i of a [N][K] weight of type dtype (LQ_DT_*) as FP32 (exact); dtype | kRoundBf16: the element rounded
// to BF16 (nearest even) on the fly, so a caller needs no BF16 copy of an F16 / F32 weight
constexpr int kRoundBf16 = 0x100;
float element(const void* w, int dtype, size_t i);

// NVFP4 round-to-nearest in two passes: the global scale g (returned) and the E4M3 block scales [N][K/16]; then
// the packed E2M1 values [N][K/2] (low nibble first), returning the relative squared error.
float nvfp4_scales(const void* w, int dtype, int N, int K, uint8_t* scales);
double nvfp4_values(const void* w, int dtype, int N, int K, float g, const uint8_t* scales, uint8_t* values);
// FP8 per output channel: q [N][K], scale [N].
void fp8_channel(const void* w, int dtype, int N, int K, uint8_t* q, float* scale);
// FP8 in 128 x 128 blocks: q [N][K], scale [ceil(N/128)][ceil(K/128)].
void fp8_block128(const void* w, int dtype, int N, int K, uint8_t* q, float* scale);

}  // namespace hostq
}  // namespace lq
