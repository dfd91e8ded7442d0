/*
 * CPU oracle for the fused quantized GEMM path: TEST INFRASTRUCTURE ONLY.
 *
 * This library is the checker. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it, and only to compute expected values or to time the reference CPU path. The product (the HIP
 * library under ling-engine_amd/) never links, loads or calls anything here.
 *
 * It restates, in plain C, the arithmetic of ling-engine's quantized GEMM path (file:line citations are
 * relative to the reference repository):
 *   - OCP FP8 E4M3FN and FP4 E2M1 codecs, BF16 / FP16 round-to-nearest-even;
 *   - the weight quantizers: per-channel FP8 (bench/quant/drafter_variants.py:77-81, `fake_fp8`),
 *     NVFP4 RTN (src/core/model.cu:188-249, `quantize_nvfp4`), 128x128 / 1x128 FP8 block scaling;
 *   - the tiled ("kernel-order") weight layout (src/core/stream_gemm.cu:705-780) and its dequantizers
 *     (src/core/stream_gemm.cu:782-820);
 *   - the FP16 activation copy with a power-of-two row scale (src/core/stream_gemm.cu:480-566);
 *   - the reference GEMM: dequantize to FP32, accumulate in FP32 (k ascending), then the epilogues
 *     (SiLU * mul, src/core/kernels.cu:38,308-312; residual add, src/core/kernels.cu:303-306), rounded
 *     to BF16 once, round-to-nearest-even.
 *
 * Parity pins (tests/test_oracle.py): every codec is checked exhaustively against torch's independent
 * float8_e4m3fn / bfloat16 / float16 casts; the NVFP4 quantizer against the reference's hand-made block
 * (tests/stream_tests.cu:1093-1107) and Gaussian error band (:1111-1119); the tiled layout against
 * literal byte positions from the reference's layout comments plus a retile/untile round trip; the GEMM
 * against a float64 numpy product on the same dequantized operands.
 */
#ifndef LING_ORACLE_H
#define LING_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- portable seeded generator: splitmix64 -> uniform double -> Box-Muller (double) ---- */
typedef struct { uint64_t s; int have; double spare; } or_rng;
void or_rng_init(or_rng* r, uint64_t seed);
uint64_t or_rng_next(or_rng* r);
double or_rng_normal(or_rng* r);
/* n floats ~ N(0, sigma), float32 */
void or_fill_normal(uint64_t seed, float sigma, float* out, size_t n);
/* n BF16 (bit patterns) ~ N(0, sigma), rounded to nearest even */
void or_fill_normal_bf16(uint64_t seed, float sigma, uint16_t* out, size_t n);

/* ---- codecs ---- */
float or_e4m3_decode(uint8_t c);           /* OCP E4M3FN: bias 7, no inf, S.1111.111 = NaN */
uint8_t or_e4m3_encode(float x);           /* RNE, saturating to +-448 (satfinite); NaN -> 0x7f */
float or_e2m1_decode(uint8_t nibble);      /* {0,.5,1,1.5,2,3,4,6} with sign bit 8 */
uint8_t or_e2m1_encode_weight(float y);    /* model.cu:225-229: nearest, ties to the smaller magnitude, sign only if != 0 */
uint8_t or_e2m1_encode_rne(float y);       /* activations: nearest, ties to even code, saturating, sign kept */
uint16_t or_bf16_bits(float x);            /* RNE; NaN -> quiet NaN */
float or_bf16_float(uint16_t b);
uint16_t or_f16_bits(float x);             /* IEEE binary16, RNE, with subnormals and overflow to inf */
float or_f16_float(uint16_t h);

/* ---- weight quantizers ---- */
/* fake_fp8 (drafter_variants.py:77-81): s_n = max(amax_n / 448, 1e-12); q = E4M3(w / s_n). w FP32 [N][K]. */
void or_quant_fp8_per_channel(const float* w, int N, int K, uint8_t* q, float* scale);
/* quantize_nvfp4 (model.cu:188-249) on BF16 [N][K]: values [N][K/2] (low nibble first), E4M3 scales
 * [N][K/16], returns scale2 and (optionally) the relative squared error. */
float or_quant_nvfp4(const uint16_t* w_bf16, int N, int K, uint8_t* values, uint8_t* scales, double* rel_sq_err);
/* FP8 in 128x128 blocks: s[nb][kb] = amax / 448 (1 for an all-zero block); q = E4M3(w / s). N, K % 128 == 0. */
void or_quant_fp8_block128(const float* w, int N, int K, uint8_t* q, float* scale);
/* FP8 activations in 1x128 groups of BF16 x [M][K]: s[m][kb] = amax / 448 (1 if zero); q = E4M3(x / s). */
void or_quant_act_fp8_g128(const uint16_t* x_bf16, int M, int K, uint8_t* q, float* scale);

/* ---- the tiled layout (stream_gemm.cu:39-46,705-780); N % 16 == 0, K % 128 == 0 ---- */
size_t or_tiled_bytes_fp8(int N, int K);
size_t or_tiled_bytes_nvfp4(int N, int K);
size_t or_tiled_bytes_nvfp4_coded(int N, int K);
void or_retile_fp8(const uint8_t* w, uint8_t* out, int N, int K);
void or_untile_fp8(const uint8_t* tiled, uint8_t* w, int N, int K);
void or_retile_nvfp4(const uint8_t* values, const uint8_t* scales, uint8_t* out, int N, int K);
void or_untile_nvfp4(const uint8_t* tiled, uint8_t* values, uint8_t* scales, int N, int K);
/* scale_code_table (stream_gemm.cu:1804-1819): returns 0 when more than 64 distinct scale bytes. */
int or_scale_code_table(const uint8_t* scales, size_t n, uint8_t* table64, uint8_t* code_of256);
/* retile_nvfp4_coded (stream_gemm.cu:740-780): the coded blob and the raw scale copy (128 B per block). */
void or_retile_nvfp4_coded(const uint8_t* values, const uint8_t* scales, const uint8_t* code_of256, uint8_t* out,
                           uint8_t* raw_scales, int N, int K);

/* ---- dequantization (row-major, from row-major codes) ---- */
/* FP32: e4m3(q) * s_n */
void or_dequant_fp8_pc(const uint8_t* q, const float* scale, int N, int K, float* out);
/* FP32: e2m1(c) * (e4m3(sc) * scale2)  (dequant_tiled_nvfp4_kernel's product order, stream_gemm.cu:797-800) */
void or_dequant_nvfp4(const uint8_t* values, const uint8_t* scales, float scale2, int N, int K, float* out);
/* FP32: e4m3(q) * s[n/128][k/128] */
void or_dequant_fp8_block128(const uint8_t* q, const float* scale, int N, int K, float* out);

/* ---- activations ---- */
/* to_half_rows (stream_gemm.cu:480-566): e = frexp(max|x_row|) (0 if zero or non-finite), xh = f16_rn(x*2^(15-e)),
 * xinv = 2^(e-15). x FP32 [M][K]. */
void or_to_half_rows(const float* x, int M, int K, uint16_t* xh, float* xinv);

/* ---- reference GEMMs: y = x . Wdeq^T, FP32 accumulation in k order; threads = 0 -> all cores ---- */
/* x FP32 [M][K], wdeq FP32 [N][K] (row-major), y FP32 [M][N] */
void or_gemm_f32(const float* x, const float* wdeq, int M, int N, int K, float* y, int threads);
/* Epilogue helpers (elementwise, FP32 in, BF16 bits out). */
float or_silu(float v);                           /* v / (1 + expf(-v)) */
void or_epi_bf16(const float* acc, size_t n, uint16_t* out);
void or_epi_silu_mul_bf16(const float* g, const float* u, size_t n, uint16_t* out);
void or_epi_residual_bf16(const float* acc, const uint16_t* resid, size_t n, uint16_t* out);

/* Whole-path helpers used by the CPU baseline (one call = dequantize + GEMM + epilogue):
 * FP8 per-channel skinny GEMM with BF16 x [M][K] and row-major q [N][K]; out BF16 [M][N]. Rows of y are
 * computed only for the output-channel range [n0, n1) (a bounded sample); pass 0, N for all. */
void or_stream_fp8_pc_bf16(const uint16_t* x, int M, const uint8_t* q, const float* scale, int N, int K,
                           int n0, int n1, uint16_t* y, int threads);
/* The prefill reference on a row subset: y[r][n] for rows `rows[r]`, from FP8 block-scaled operands. */
void or_prefill_fp8_rows(const uint8_t* xq, const float* xs, const int* rows, int R, const uint8_t* wq,
                         const float* ws, int N, int K, float* y, int threads);

/* RMSNorm rows (FP32 out) and their FP16 copy with row scales, as rmsnorm_half makes them. */
void or_rmsnorm_half(const float* x, const uint16_t* w, int rows, int H, float eps, int gemma, float* out,
                     uint16_t* xh, float* xinv);
/* Per-tensor FP8 activations: E4M3_satfinite(bf16(x) * (1 / input_scale)). */
void or_quant_act_fp8(const float* x, size_t n, float input_scale, uint8_t* q);
/* prefill activation producers (reference src/core/prefill_gemm.cu:382-459, 607-637) */
void or_quant_act_nvfp4(const float* x, int M, int K, float input_scale, uint8_t* q, uint8_t* sf);
void or_silu_mul_quant_nvfp4(const float* g, const float* u, int M, int K, float input_scale, uint8_t* q, uint8_t* sf);
void or_rmsnorm_quant(const float* x, const uint16_t* w, float* out, int M, int H, float eps, int nvfp4,
                      float input_scale, uint8_t* q, uint8_t* sf);
/* DeltaNet gated output norm (D = 128) and attention sigmoid gate into FP8 (prefill_gemm.cu:461-494) */
void or_gated_rmsnorm_fp8(const float* x, const float* z, const uint16_t* w, int rows, float eps, float input_scale,
                          uint8_t* q);
void or_sigmoid_mul_fp8(const float* x, const float* gate, size_t n, float input_scale, uint8_t* q);

int or_hardware_threads(void);

#ifdef __cplusplus
}
#endif
#endif
