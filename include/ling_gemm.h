/*
 * ling_gemm.h: the C ABI of the MI355X (gfx950) fused quantized GEMM library, libling_gemm.so.
 *
 * It is the drop-in for ling-engine's `ling::kernels` quantized GEMM path (reference src/core/kernels.cuh).
 * Every pointer is caller-owned device memory unless stated; every call is asynchronous on `stream` (a
 * hipStream_t, NULL = the default stream) and never synchronizes the host. Calls return LQ_OK (0) or an
 * error code; lq_last_error() then holds the message (per host thread). include/ling_gemm.hpp rethrows
 * these as std::runtime_error with the reference's message texts.
 *
 * Weights are read in the reference's tiled ("kernel-order") layout, byte for byte (reference
 * src/core/stream_gemm.cu:39-46,705-780): a (16-row tile, 128-value chunk) block is contiguous, blocks in
 * (tile, chunk) order; FP8 blocks are 2048 bytes, NVFP4 blocks 1024 value bytes + 128 E4M3 scale bytes.
 *
 * Activations: BF16 [M][K] (row-major, 16-bit patterns) for the BF16 entry points; FP16 [M][K] with a
 * power-of-two row scale xinv[M] (to_half_rows) for the reference-compatible ones.
 *
 * Scratch: the skinny GEMMs split K across workgroups and reduce the partial sums in a fixed order inside
 * the kernel; the partials and arrival counters live in a per-device workspace the library allocates on
 * first use (lq_init allocates it up front so that later calls can be graph-captured). Calls that overlap
 * on one device (two streams) must not share it: serialize them.
 */
#ifndef LING_GEMM_H
#define LING_GEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  LQ_OK = 0,
  LQ_ERR_SHAPE = 1,  /* a shape the kernels do not take (K % 128, N % 16, M out of range, ...) */
  LQ_ERR_ARG = 2,    /* a null pointer or an invalid argument */
  LQ_ERR_LAUNCH = 3, /* the HIP runtime reported an error at launch */
  LQ_ERR_DEVICE = 4, /* device query or workspace allocation failed */
  LQ_ERR_IO = 5      /* a file is missing, unreadable or not in the expected format */
};

/* Largest row count of the skinny (stream) GEMMs: 5 groups of 16 (4 sequences x 17 verify rows = 68 fit).
 * The reference takes 32 (kernels.cuh:107, kMaxStreamRows). */
#define LQ_MAX_STREAM_ROWS 80

/* Message of the last failed call on this host thread ("" if none). */
const char* lq_last_error(void);
/* Allocates the current device's workspace now (otherwise on first use). No reference counterpart. */
int lq_init(void);
/* Library version string. */
const char* lq_version(void);
/* Bytes of a caller-owned workspace that serves every skinny (stream) GEMM entry point with M <= max_rows on
 * the current device (0 for max_rows outside [1, 80]). */
size_t lq_stream_workspace_bytes(int max_rows);
/* Make buffer (device memory of the current device, 256-byte aligned, `bytes` long) that device's workspace for
 * the skinny GEMMs: split-K partial sums, arrival counters, the one-launch FFN's flags. The library frees its
 * own and allocates nothing more for them; a launch that needs more than the buffer holds fails with LQ_ERR_ARG.
 * buffer = NULL returns to the library's own workspace. Call outside graph capture, with no launch in flight
 * that uses the current workspace; the buffer must stay allocated while it is set. The reference's split-K
 * buffer is a function-static grow-only allocation (src/core/stream_gemm.cu:581-590); this is the
 * caller-provided form of it. The prefill's tail-split scratch stays library-owned. */
int lq_set_workspace(void* buffer, size_t bytes);

/* ---------------- tiled layout (reference src/core/kernels.cuh:162-188) ---------------- */
size_t lq_tiled_bytes_fp8(int N, int K);          /* kernels.cuh:167 tiled_bytes_fp8 */
size_t lq_tiled_bytes_nvfp4(int N, int K);        /* kernels.cuh:166 tiled_bytes_nvfp4 */
size_t lq_tiled_bytes_nvfp4_coded(int N, int K);  /* kernels.cuh:182 tiled_bytes_nvfp4_coded */
/* Row-major FP8 [N][K] -> tiled. kernels.cuh:169 retile_fp8 */
int lq_retile_fp8(const uint8_t* w, uint8_t* out, int N, int K, void* stream);
/* Row-major NVFP4 values [N][K/2] + E4M3 scales [N][K/16] -> tiled. kernels.cuh:168 retile_nvfp4 */
int lq_retile_nvfp4(const uint8_t* w, const uint8_t* wscale, uint8_t* out, int N, int K, void* stream);
/* Host: the 6-bit scale-code table (0: more than 64 distinct scales). kernels.cuh:181 scale_code_table */
int lq_scale_code_table(const uint8_t* scales, size_t n, uint8_t* table64, uint8_t* code_of256);
/* The coded NVFP4 blob plus a raw scale copy (128 B per block). code_of_dev: device [256].
 * kernels.cuh:183-184 retile_nvfp4_coded */
int lq_retile_nvfp4_coded(const uint8_t* w, const uint8_t* wscale, const uint8_t* code_of_dev, uint8_t* out,
                          uint8_t* raw_scales, int N, int K, void* stream);
/* Tiled -> BF16 row-major [N][K]: bf16(e4m3 * wscale). kernels.cuh:188 dequant_tiled_fp8 */
int lq_dequant_tiled_fp8(const uint8_t* tw, float wscale, uint16_t* out, int N, int K, void* stream);
/* Tiled -> BF16: bf16(e2m1 * (e4m3 * scale2)); raw_scales: a coded blob's raw copy, or NULL.
 * kernels.cuh:186-187 dequant_tiled_nvfp4 */
int lq_dequant_tiled_nvfp4(const uint8_t* tw, float scale2, uint16_t* out, int N, int K, void* stream,
                           const uint8_t* raw_scales);
/* Additive: tiled FP8 -> FP32 with per-channel scales, e4m3 * wscale_n[n] (the bit-exact dequant check). */
int lq_dequant_tiled_fp8_pc_f32(const uint8_t* tw, const float* wscale_n, float* out, int N, int K, void* stream);
/* Additive: tiled NVFP4 -> FP32, e2m1 * (e4m3 * scale2). */
int lq_dequant_tiled_nvfp4_f32(const uint8_t* tw, float scale2, float* out, int N, int K, void* stream,
                               const uint8_t* raw_scales);

/* ---------------- rows path, reference-compatible (reference src/core/kernels.cuh:266-295) ------------- */
/* FP32 x [M][K] -> FP16 with a power-of-two row scale (largest magnitude in [2^14, 2^15)); xinv[m] undoes it.
 * kernels.cuh:270 to_half_rows */
int lq_to_half_rows(const float* x, int M, int K, uint16_t* xh, float* xinv, void* stream);
/* The same from BF16 x. kernels.cuh:546-547 bf16_to_half_rows */
int lq_bf16_to_half_rows(const uint16_t* x, int M, int K, uint16_t* xh, float* xinv, void* stream);
/* RMSNorm of each row: out = x * rstd * w' (FP32 [rows][H]; rstd = 1 / sqrt(mean(x^2) + eps), w' = 1 + w when
 * gemma, else w; w BF16 [H]) and the FP16 row copy of out with its row scales, as to_half_rows makes them.
 * kernels.cuh:267-268 rmsnorm_half */
int lq_rmsnorm_half(const float* x, const uint16_t* w, float* out, uint16_t* xh, float* xinv, int rows, int H, float eps,
                    int gemma, void* stream);
/* y[M][N] (FP32) = (wscale * xh . W^T) * xinv[m], W tiled FP8. kernels.cuh:276-277 stream_gemm_fp8 */
int lq_stream_gemm_fp8(const uint16_t* xh, const float* xinv, int M, const uint8_t* w, float wscale, float* y, int N,
                       int K, void* stream);
/* y = (scale2 * xh . W^T) * xinv[m], W tiled NVFP4 (table: a coded blob's scale-code table, device [64], or
 * NULL for a raw blob). kernels.cuh:273-274 stream_gemm_nvfp4 */
int lq_stream_gemm_nvfp4(const uint16_t* xh, const float* xinv, int M, const uint8_t* w, const uint8_t* table,
                         float scale2, float* y, int N, int K, void* stream);
/* kernels.cuh:281-287 StreamTarget */
typedef struct {
  const uint8_t* w;
  const uint8_t* wscale; /* NVFP4: coded blob's table (device), else NULL */
  float scale;           /* NVFP4 global scale or FP8 per-tensor scale */
  float* y;
  int N;
} lq_stream_target;
/* 1..4 matrices sharing xh in one launch, each y = scale * xh . W^T * xinv, bit for bit what a separate call for that
 * matrix gives (each matrix's K is split over its own workgroups as it would be alone; matrices wanting different
 * tiles per wave, or mixing coded and raw NVFP4, take one launch per group). kernels.cuh:288-289 stream_gemm_multi */
int lq_stream_gemm_multi(int nvfp4, const uint16_t* xh, const float* xinv, int M, const lq_stream_target* t, int n,
                         int K, void* stream);

/* The sparse head: y[M][cap] = scale2 * xh . W[rows[i]]^T * xinv for i < *nrows (device count), -inf after; W the
 * tiled NVFP4 blob of the full matrix of N rows (raw: raw_scales null; coded: raw_scales = its raw scales, 128 B
 * per block). Each element's arithmetic is the full stream_gemm_nvfp4 launch's over the same blob, so a selected
 * row's logit is bit for bit the full head's. cap % 32 == 0. N is an addition to the reference's arguments: the
 * full launch's split of K depends on it here. kernels.cuh:294-295 stream_gemm_gather_nvfp4. */
int lq_stream_gemm_gather_nvfp4(const uint16_t* xh, const float* xinv, int M, const uint8_t* w,
                                const uint8_t* raw_scales, float scale2, const int* rows, const int* nrows, int cap,
                                float* y, int K, int N, void* stream);

/* Cache run-ahead: reads what a stream GEMM over (w, N, K) reads first, about `bytes` of it, and writes nothing, so
 * that launch's first loads hit the caches after a latency-bound stretch. fp4: NVFP4 blob (coded: the scale-coded
 * form), else FP8. w null or bytes 0: nothing happens. This library's split cuts K per workgroup, so the bytes
 * taken are each workgroup's first units (tile group x chunk) of its own range, by the workgroup of the same index,
 * not every tile's first chunks. src/core/kernels.cuh:405 l2_prefetch_weights (src/core/stream_gemm.cu:1864-1873) */
int lq_l2_prefetch_weights(const uint8_t* w, int fp4, int coded, int N, int K, size_t bytes, void* stream);

/* ---------------- rows path, BF16 formats (additive; per-channel FP8 scales, BF16 in and out) ---------------- */
/* y[M][N] = bf16(wscale_n[n] * x . W^T), W tiled FP8, x BF16 [M][K]. Replaces the engine's linear_fp8
 * (reference src/core/engine.cpp:1272-1281) for per-channel checkpoints. */
int lq_stream_fp8_pc(const uint16_t* x, int M, const uint8_t* w, const float* wscale_n, uint16_t* y, int N, int K,
                     void* stream);
/* The same computation with no allocation of any kind: no counterpart in the reference; for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Its split-K partial
 * sums and arrival counters live in a fixed 25 MiB + 256 KiB device array of the library (one per GPU, held until
 * the process ends) instead of the workspace: enough for any M <= 80 on devices of up to 320 CUs; launches needing
 * more (more than 320 workgroups' partials, or more than 65536 tile groups) fail with LQ_ERR_SHAPE before anything runs. Results equal lq_stream_fp8_pc's bit for
 * bit. All calls on one GPU share the array: calls that overlap on one GPU (two streams) race, so serialize them.
 * Call lq_init first when the first call may be graph-captured (it clears the array's counters eagerly). */
int lq_stream_fp8_pc_noalloc(const uint16_t* x, int M, const uint8_t* w, const float* wscale_n, uint16_t* y, int N,
                             int K, void* stream);
/* h[M][N] = bf16(silu(sg[n] * x . G^T) * (su[n] * x . U^T)): the MLP gate/up projections with the SiLU*mul
 * epilogue fused (reference engine.cpp:1699-1701 = stream_gemm_multi({gate, up}) + silu_mul). */
int lq_stream_fp8_pc_silu_mul(const uint16_t* x, int M, const uint8_t* w_gate, const float* s_gate,
                              const uint8_t* w_up, const float* s_up, uint16_t* h, int N, int K, void* stream);
/* y[M][N] = bf16(wscale_n[n] * x . W^T + resid[m][n]); y may be resid (in place). The down / out projection
 * with the residual add fused (reference engine.cpp:1227-1233 linear_fp8_residual = stream_gemm + add_inplace). */
int lq_stream_fp8_pc_residual(const uint16_t* x, int M, const uint8_t* w, const float* wscale_n,
                              const uint16_t* resid, uint16_t* y, int N, int K, void* stream);
/* The whole MLP step in one launch: h[M][I] = bf16(silu(sg . x G^T) * (su . x U^T)) (as stream_fp8_pc_silu_mul,
 * K = H), then y[M][H] = bf16(sd . h D^T + resid) (as stream_fp8_pc_residual, K = I); y may be resid. Bit for bit
 * the two calls' results. The launch keeps every workgroup resident (one per CU) and hands h from the first
 * phase to the second inside the kernel: only one such launch may run on a device at a time. Replaces the
 * reference's persistent FFN kernel (reference src/core/stream_gemm.cu:841-1072, ffn_step) for the FP8 rows path.
 * Experimental: it runs slower than the two calls on MI355X (about 2 us at M = 17); prefer them unless one launch
 * is required. */
int lq_stream_fp8_pc_ffn(const uint16_t* x, int M, const uint8_t* w_gate, const float* s_gate, const uint8_t* w_up,
                         const float* s_up, const uint8_t* w_down, const float* s_down, const uint16_t* resid,
                         uint16_t* h, uint16_t* y, int I, int H, void* stream);
/* Synchronous: *hit = 1 if, since the last call, a launch on the current device gave up an in-kernel wait at its
 * deadline: a stream_fp8_pc_ffn launch's wait for h (100 ms), or a skinny launch's finish workgroups' wait for the
 * streaming workgroups (1 s, reached only if the GPU stops the launch that long); the results of such a launch
 * are not valid. Else 0. The call clears the flags.
 * A caller of lq_stream_fp8_pc_ffn that cannot rule out a concurrent kernel holding CUs checks it after
 * synchronizing. No counterpart in the reference (its wait traps). */
int lq_stream_ffn_deadline_status(int* hit);
/* y[M][N] = bf16(scale2 * x . W^T), W tiled NVFP4 (raw, or coded with its device table), x BF16. The kernel
 * turns each 128-value chunk of a row of x into FP16 under a power-of-two scale from that chunk's largest
 * magnitude and multiplies the chunk's sums back in FP32. Replaces linear_fp4 (engine.cpp:1173-1177). */
int lq_stream_nvfp4_bf16(const uint16_t* x, int M, const uint8_t* w, const uint8_t* table, float scale2, uint16_t* y,
                         int N, int K, void* stream);

/* ---------------- prefill, NVFP4 (reference src/core/kernels.cuh:207-221) ---------------- */
/* y[M][0..N) (rows ldy apart, FP32) = alpha * xq . W^T, or += with accumulate; xq NVFP4 activations [M][K/2] with E4M3
 * block scales xs [M][K/16]; W the tiled NVFP4 blob (raw; or coded with wsf = its raw scales, 128 B per block).
 * Both operands are dequantized exactly (E2M1 x E4M3) and multiplied in FP32. N % 128 == 0, K % 128 == 0; M < 1
 * does nothing. kernels.cuh:210-211 prefill_gemm_nvfp4. */
int lq_prefill_gemm_nvfp4(const uint8_t* xq, const uint8_t* xs, int M, const uint8_t* w, float alpha, float* y, int ldy,
                          int N, int K, int accumulate, void* stream, const uint8_t* wsf);
/* The FFN's gate and up projections into the down projection's input: NVFP4 of BF16(silu(alpha_gate * xq . G^T) *
 * (alpha_up * xq . U^T)) with global scale 1 / out_input_scale, q_out [M][N/2], sf_out [M][N/16]; gate_sf / up_sf:
 * raw scales of coded blobs (both or neither). N % 128 == 0, K % 128 == 0. kernels.cuh:217-221 prefill_swiglu_nvfp4. */
int lq_prefill_swiglu_nvfp4(const uint8_t* xq, const uint8_t* xs, int M, const uint8_t* gate, float alpha_gate,
                            const uint8_t* up, float alpha_up, int N, int K, float out_input_scale, uint8_t* q_out,
                            uint8_t* sf_out, void* stream, const uint8_t* gate_sf, const uint8_t* up_sf);

/* ---------------- prefill activation producers (reference src/core/kernels.cuh:190-206) ---------------- */
/* x [M][K] FP32 -> NVFP4: q packed [M][K/2] (low nibble first), E4M3 block scales sf [M][K/16], global scale
 * 1 / input_scale; each value rounded to BF16 first. K % 16 == 0. kernels.cuh:193 quant_act_nvfp4. */
int lq_quant_act_nvfp4(const float* x, int M, int K, float input_scale, uint8_t* q, uint8_t* sf, void* stream);
/* The same for silu(g) * u (silu(v) = v / (1 + e^-v)). kernels.cuh:195-196 silu_mul_quant_nvfp4. */
int lq_silu_mul_quant_nvfp4(const float* g, const float* u, int M, int K, float input_scale, uint8_t* q, uint8_t* sf,
                            void* stream);
/* Gemma RMSNorm of each row, v = x * rstd * (1 + w) with rstd = 1 / sqrt(mean(x^2) + eps), into `out` (FP32,
 * may be null) and straight into the next GEMM's encoding: NVFP4 (q [M][H/2], sf [M][H/16]) when nvfp4, else FP8
 * E4M3(BF16(v) / input_scale) saturated (q [M][H]). H % 1024 == 0, H <= 65536; x, w, out, q 16-byte aligned.
 * kernels.cuh:203-204 rmsnorm_quant. */
int lq_rmsnorm_quant(const float* x, const uint16_t* w, float* out, int M, int H, float eps, int nvfp4,
                     float input_scale, uint8_t* q, uint8_t* sf, void* stream);

/* rmsnorm_quant with the FP32 copy replaced by a BF16 one (out BF16 [M][H], may be null): out = bf16(v), the same
 * rounding the quantizer applies. kernels.cuh:234-235 rmsnorm_quant_bf16 */
int lq_rmsnorm_quant_bf16(const float* x, const uint16_t* w, uint16_t* out, int M, int H, float eps, int nvfp4,
                          float input_scale, uint8_t* q, uint8_t* sf, void* stream);

/* ---------------- prefill, block-scaled FP8 (additive; reference src/core/kernels.cuh:190-221) ---------------- */
/* BF16 x [M][K] -> FP8 E4M3 q [M][K] with one FP32 scale per 1x128 group, scale [M][K/128] = amax / 448 (1 for an
 * all-zero group), q = E4M3_rne_sat(x * (1 / scale)) (reciprocal and product rounded to FP32, as quant_act_fp8
 * multiplies by 1 / input_scale); x 16-byte and q 8-byte aligned. The block-scaled counterpart of quant_act_fp8
 * (kernels.cuh:199). */
int lq_quant_act_fp8_g128(const uint16_t* x, int M, int K, uint8_t* q, float* scale, void* stream);
/* y[M][0..N) (rows ldy apart, BF16) = bf16(sum over 128-value K blocks kb of (xq . W^T over kb) * xs[m][kb] *
 * ws[n/128][kb]); xq FP8 [M][K], xs FP32 [M][K/128], W tiled FP8 (the stream GEMMs' blob), ws FP32 [N/128][K/128].
 * N % 128 == 0, K % 128 == 0; M < 1 does nothing. The block-scaled, BF16-out form of prefill_gemm_fp8
 * (kernels.cuh:213-214) and prefill_gemm_fp8_bf16out (kernels.cuh:239-240). */
int lq_prefill_fp8_block(const uint8_t* xq, const float* xs, int M, const uint8_t* w, const float* ws, uint16_t* y,
                         int ldy, int N, int K, void* stream);

/* ---------------- prefill, per-tensor FP8 (reference src/core/kernels.cuh:190-221,239-240) ---------------- */
/* FP32 x [M][K] -> FP8 E4M3 q = E4M3_satfinite(bf16(x) * (1 / input_scale)). K % 4 == 0.
 * kernels.cuh:199 quant_act_fp8 */
int lq_quant_act_fp8(const float* x, int M, int K, float input_scale, uint8_t* q, void* stream);
/* quant_act_fp8 over a BF16 copy x [M][K] (8-byte aligned): the bytes the FP32 values it was rounded from give.
 * kernels.cuh:237 quant_act_fp8_bf16in */
int lq_quant_act_fp8_bf16in(const uint16_t* x, int M, int K, float input_scale, uint8_t* q, void* stream);
/* The DeltaNet output norm into FP8 for the out-projection: per row of D = 128 (rows = tokens x heads),
 * v = bf16(x * rstd * w * silu(z)), rstd = 1 / sqrt(sum(x^2) / 128 + eps), q = E4M3_satfinite(v * (1 / input_scale)).
 * x, z FP32 [rows][128] (16-byte aligned), w BF16 [128], q [rows][128]. D != 128 is LQ_ERR_SHAPE.
 * kernels.cuh:205-206 gated_rmsnorm_fp8 */
int lq_gated_rmsnorm_fp8(const float* x, const float* z, const uint16_t* w, int rows, int D, float eps,
                         float input_scale, uint8_t* q, void* stream);
/* The same over BF16 x and z (8-byte aligned). kernels.cuh:244-246 gated_rmsnorm_fp8_bf16 */
int lq_gated_rmsnorm_fp8_bf16(const uint16_t* x, const uint16_t* z, const uint16_t* w, int rows, int D, float eps,
                              float input_scale, uint8_t* q, void* stream);
/* The gated attention output into FP8: q[i] = E4M3_satfinite(bf16(x[i] / (1 + e^-gate[i])) * (1 / input_scale)),
 * n values (n % 4 == 0; the reference drops a tail of n % 4, here it is LQ_ERR_SHAPE). kernels.cuh:207
 * sigmoid_mul_fp8 */
int lq_sigmoid_mul_fp8(const float* x, const float* gate, size_t n, float input_scale, uint8_t* q, void* stream);
/* y[M][0..N) (FP32, rows ldy apart) = alpha * xq . W^T, or += with accumulate; W tiled FP8. N % 128 == 0,
 * K % 128 == 0; M < 1 does nothing. kernels.cuh:213-214 prefill_gemm_fp8 */
int lq_prefill_gemm_fp8(const uint8_t* xq, int M, const uint8_t* w, float alpha, float* y, int ldy, int N, int K,
                        int accumulate, void* stream);
/* The same rounded to BF16 (never accumulated). kernels.cuh:239-240 prefill_gemm_fp8_bf16out */
int lq_prefill_gemm_fp8_bf16out(const uint8_t* xq, int M, const uint8_t* w, float alpha, uint16_t* y, int ldy, int N,
                                int K, void* stream);

/* ---------------- host weight quantizers (CPU threads; host pointers) ----------------
 * High-precision weights [N][K] (row-major) into the formats the GEMMs read, before lq_retile_* / the weight file.
 * E4M3 is OCP E4M3FN: round to nearest even, saturating to +-448. */
enum { LQ_DT_F32 = 0, LQ_DT_BF16 = 1, LQ_DT_F16 = 2 };
/* NVFP4 round-to-nearest of BF16 weights: *scale2 = g = amax / (448 * 6) (1 if all zero); scales [N][K/16] =
 * E4M3(max(amax16 / 6 / g, 2^-9)); values [N][K/2] (low nibble first) = the E2M1 code of the magnitude nearest to
 * w / (e4m3(scale) * g), ties to the smaller, sign only on non-zero codes. rel_sq_err (may be NULL) = sum of
 * squared errors / sum of squares. K % 16 == 0. Reference src/core/model.cu:188-249 quantize_nvfp4 (model.hpp:41). */
int lq_quantize_nvfp4(const uint16_t* w_bf16, int N, int K, uint8_t* values, uint8_t* scales, float* scale2,
                      double* rel_sq_err);
/* FP8 with one FP32 scale per output channel: scale [N] = max(amax_n / 448, 1e-12), q [N][K] = E4M3(w / scale).
 * Reference bench/quant/drafter_variants.py:77-81 fake_fp8 (the per-channel recipe of the benchmark configs). */
int lq_quantize_fp8_channel(const void* w, int dtype, int N, int K, uint8_t* q, float* scale);
/* FP8 in 128 x 128 blocks (the block-scaled prefill's weights): scale [ceil(N/128)][ceil(K/128)] = amax / 448
 * (1 for an all-zero block), q [N][K] = E4M3(w / scale). No reference counterpart (the reference's prefill is
 * per-tensor FP8, src/core/prefill_gemm.cu:4-7); the format of lq_prefill_fp8_block's ws. */
int lq_quantize_fp8_block128(const void* w, int dtype, int N, int K, uint8_t* q, float* scale);

/* ---------------- the on-disk kernel-order weight file (host only; no GPU is used) ----------------
 * The offline step the reference's README names ("ling-compile") and never built: its load path maps the
 * safetensors checkpoint (src/core/safetensors.hpp:14-52) and retiles every quantized linear on the GPU at each
 * load (src/core/model.cu:131-186 over kernels.cuh:168-188 retile_*). lq_wfile_compile does that once, on CPU
 * threads, writing each tiled blob byte-identical to lq_retile_fp8 / lq_retile_nvfp4 / lq_retile_nvfp4_coded
 * with its scale side tables; loading is then a copy of 4096-byte-aligned sections to device memory.
 *
 * Checkpoint tensors recognised per linear `P` (the reference's Model::fp4 / Model::fp8, model.cu:248-277):
 *   NVFP4: P.weight U8 [N][K/2], P.weight_scale F8_E4M3 [N][K/16], P.weight_scale_2 scalar, P.input_scale
 *          scalar (optional). Written coded (LQ_WENTRY_NVFP4_CODED) when the matrix has at most 64 distinct
 *          scale bytes and LQ_WFILE_NO_CODES is not set (the reference's LING_SCALE_CODES default), else raw.
 *   FP8:   P.weight F8_E4M3 [N][K] with P.weight_scale_inv [ceil(N/128)][ceil(K/128)] (block scales), or
 *          P.weight_scale as a scalar (per-tensor) or [N] / [N][1] (per-channel); P.input_scale optional.
 * Scales may be F32, BF16 or F16 in the checkpoint; the file holds FP32. With LQ_WFILE_PASSTHROUGH every
 * other tensor is copied as is (LQ_WENTRY_RAW). N % 16 == 0 and K % 128 == 0 for every quantized weight. */
#define LQ_WFILE_NO_CODES 1
#define LQ_WFILE_PASSTHROUGH 2
/* Quantize high-precision linears while compiling (at most one of these): every 2-D P.weight in BF16, F16 or F32
 * with no scale tensors, N % 16 == 0, K % 128 == 0 and a name containing neither "embed" nor "norm" becomes an FP8
 * per-channel (lq_quantize_fp8_channel), FP8 128x128-block (lq_quantize_fp8_block128) or NVFP4
 * (lq_quantize_nvfp4, F16 / F32 rounded to BF16 first) entry, marked LQ_WENTRY_QUANTIZED; the reference quantizes
 * such matrices at load (src/core/model.cu:188-249, src/core/drafter.cpp:93-100). */
#define LQ_WFILE_QUANT_FP8 4
#define LQ_WFILE_QUANT_FP8_BLOCK 8
#define LQ_WFILE_QUANT_NVFP4 16
enum { LQ_WENTRY_FP8 = 1, LQ_WENTRY_NVFP4 = 2, LQ_WENTRY_NVFP4_CODED = 3, LQ_WENTRY_RAW = 4 };
enum { LQ_WSCALE_NONE = 0, LQ_WSCALE_TENSOR = 1, LQ_WSCALE_CHANNEL = 2, LQ_WSCALE_BLOCK128 = 3 };
#define LQ_WENTRY_HAS_INPUT_SCALE 1
#define LQ_WENTRY_QUANTIZED 2 /* quantized by the compiler from the checkpoint dtype in `dtype` */

typedef struct lq_wfile lq_wfile;
typedef struct {
  const char* name;     /* the linear's prefix (P), or the tensor's name for LQ_WENTRY_RAW */
  int kind;             /* LQ_WENTRY_* */
  int scale_kind;       /* FP8: LQ_WSCALE_*; NVFP4: LQ_WSCALE_NONE (block scales live in the blob / aux) */
  int N, K;             /* logical matrix shape (0 for raw entries) */
  float weight_scale;   /* FP8 per-tensor weight_scale; NVFP4 weight_scale_2 */
  float input_scale;    /* when flags & LQ_WENTRY_HAS_INPUT_SCALE */
  int flags;
  char dtype[16];       /* checkpoint dtype of the weight ("U8", "F8_E4M3", "BF16", ...) */
  int ndim;
  int64_t shape[4];     /* checkpoint shape of the weight */
  const uint8_t* blob;  /* host-mapped: the tiled weight (raw entries: the tensor's bytes) */
  size_t blob_bytes;
  const uint8_t* aux;   /* coded NVFP4: raw scale copy (128 B per block); FP8: FP32 per-channel [N] or block
                           [ceil(N/128)][ceil(K/128)] scales; else NULL */
  size_t aux_bytes;
  const uint8_t* table; /* coded NVFP4: the 64-byte scale-code table; else NULL */
  size_t table_bytes;
} lq_wentry;

/* Compile the checkpoint directory (model.safetensors.index.json + shards, or model.safetensors) into
 * out_path (written to out_path.partial, then renamed). *entries_written may be NULL. No reference
 * counterpart (the never-built ling-compile). */
int lq_wfile_compile(const char* checkpoint_dir, const char* out_path, int flags, int* entries_written);
/* Map a compiled file and check its header, entry table hash and section bounds. */
int lq_wfile_open(const char* path, lq_wfile** out);
void lq_wfile_close(lq_wfile* f);
int lq_wfile_count(const lq_wfile* f);
/* Index of the entry named `name`, or -1. */
int lq_wfile_find(const lq_wfile* f, const char* name);
/* Entry i; its pointers stay valid until lq_wfile_close. */
int lq_wfile_entry(const lq_wfile* f, int i, lq_wentry* out);
/* Recompute entry i's section hashes (LQ_ERR_IO on a mismatch). */
int lq_wfile_verify(const lq_wfile* f, int i);
/* Host (CPU-thread) retiles, byte-identical to lq_retile_fp8 / lq_retile_nvfp4 / lq_retile_nvfp4_coded;
 * host pointers. kernels.cuh:168-169,183-184 */
int lq_host_retile_fp8(const uint8_t* w, uint8_t* out, int N, int K);
int lq_host_retile_nvfp4(const uint8_t* w, const uint8_t* wscale, uint8_t* out, int N, int K);
int lq_host_retile_nvfp4_coded(const uint8_t* w, const uint8_t* wscale, const uint8_t* code_of256, uint8_t* out,
                               uint8_t* raw_scales, int N, int K);

#ifdef __cplusplus
}
#endif
#endif
