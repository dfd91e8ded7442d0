// Block-scaled FP8 prefill GEMM on gfx950 MFMA, and the 1x128 FP8 activation quantizer that feeds it.
//
//   y[m][n] = bf16( sum_kb (sum_{k in kb} e4m3(xq[m][k]) * e4m3(wq[n][k])) * xs[m][kb] * ws[n/128][kb] )
//
// xq: FP8 E4M3 activations [M][K] (row-major) with one FP32 scale per 1x128 group, xs [M][K/128];
// wq: FP8 E4M3 weights in the tiled layout the skinny GEMMs stream (reference
// src/core/stream_gemm.cu:705-738), with one FP32 scale per 128x128 block, ws [N/128][K/128].
//
// Design:
//  * One v_mfma_f32_16x16x128_f8f6f4 per 16x16 output tile per 128-value K block: an MFMA covers exactly one
//    scale block, so its FP32 result is scaled once and added to the accumulator (one FMA per output per
//    block). Any permutation of K inside the block is harmless, since A and B use the same one.
//  * Weights are the A operand (rows n) and activations the B operand (columns m): a lane's four outputs
//    share one token and one 128-row weight block, so its block scale is one multiply per token tile.
//  * A workgroup (8 waves, 2 per SIMD: 2 along the weights x 4 along the tokens) computes 128 weight rows x
//    256 tokens; each wave 64 x 64 (4 x 4 MFMA tiles). Each K block's operands (16 KB of weights, 32 KB of
//    activations) are staged in LDS (double buffered) as [row][8 x 16-byte units] with the unit index
//    XOR-swizzled by row, so the fragment reads are bank-conflict free. Global loads run two K blocks ahead
//    through two register staging sets: a block's loads are issued two iterations before it is written to
//    LDS and computed.
//  * Tile order: each XCD works through a contiguous range of a grouped raster (8 weight tiles x every
//    token tile per group), so the workgroups running at once on an XCD share the K slices of both operands
//    in its L2 instead of re-streaming the whole activation matrix per weight tile.
#include "lq_common.hpp"

#include <algorithm>
#include <string>

namespace lq {
namespace {

constexpr int kBN = 128;  // weight rows per workgroup
constexpr int kBM = 256;  // tokens per workgroup
constexpr int kThreads = 512;
constexpr int kGroupN = 8;  // weight tiles per raster group
constexpr int kRowBytes = 128;                       // one K block of one row (FP8)
constexpr int kStage = (kBN + kBM) * kRowBytes;      // 48 KB: weights then activations

// Byte offset of 16-byte unit u of row `row` in an LDS operand tile.
__device__ __forceinline__ int lds_off(int row, int u) { return row * kRowBytes + ((u ^ ((row >> 1) & 7)) << 4); }

struct PrefillArgs {
  const uint8_t* xq;
  const float* xs;
  const uint8_t* w;
  const float* ws;
  uint16_t* y;
  int ldy, M, N, K, KB;
  int tiles_m, tiles_n;
};

__global__ void __launch_bounds__(kThreads) prefill_fp8_kernel(const PrefillArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, t = lane >> 4;
  const int wn = wave & 1, wm = wave >> 1;  // wave's 64-row weight half and 64-token quarter

  // Tile order. The hardware places block b on XCD b % 8; each XCD takes a contiguous range of the logical
  // tile order, in which tiles come in groups of kGroupN weight tiles x all token tiles, token tile slowest
  // within a group. The ~32 workgroups an XCD runs at once then cover kGroupN weight tiles x a few token
  // tiles, so the K slices of both operands they read at a time are shared in that XCD's L2.
  const int nb = gridDim.x, b = blockIdx.x;
  int tile = b;
  if ((nb & 7) == 0) tile = (b & 7) * (nb >> 3) + (b >> 3);
  const int grp = tile / (kGroupN * a.tiles_m), rem = tile % (kGroupN * a.tiles_m);
  const int gsize = min(kGroupN, a.tiles_n - grp * kGroupN);
  const int tn = grp * kGroupN + rem % gsize, tm = rem / gsize;
  const int n0 = tn * kBN, m0 = tm * kBM;

  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.w), 0, 0x7fffffff, 0x00020000);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.xq), 0, 0x7fffffff, 0x00020000);

  // Global -> LDS copy plan, 2 + 4 16-byte pieces per thread and K block.
  // Weights: piece j (0..1023) = tiled block (16-row tile tw = j / 128, piece p = j % 128) of the current chunk;
  // p = ((h*2 + q)*8 + g)*4 + tt holds row g + 8h, values [32 tt + 16 q, +16): LDS row 16 tw + g + 8h, unit 2 tt + q.
  constexpr int WP = kBN * kRowBytes / 16 / kThreads, XP = kBM * kRowBytes / 16 / kThreads;
  int wsrc[WP], wdst[WP], xsrc[XP], xdst[XP];
#pragma unroll
  for (int i = 0; i < WP; ++i) {
    const int j = i * kThreads + threadIdx.x;
    const int tw = j >> 7, p = j & 127;
    const int tt = p & 3, g = (p >> 2) & 7, q = (p >> 5) & 1, h = p >> 6;
    wsrc[i] = ((n0 >> 4) + tw) * a.KB * kTileBytesFp8 + p * 16;
    wdst[i] = lds_off(16 * tw + g + 8 * h, 2 * tt + q);
  }
#pragma unroll
  for (int i = 0; i < XP; ++i) {
    // activations: row j / 8 of the token tile, unit j % 8 (rows past M read as zeros, out of range)
    const int j = i * kThreads + threadIdx.x;
    const int row = j >> 3, u = j & 7, m = m0 + row;
    xsrc[i] = m < a.M ? m * a.K + u * 16 : static_cast<int>(0x80000000u);
    xdst[i] = kBN * kRowBytes + lds_off(row, u);
  }

  // per-lane block-scale inputs: this lane's four tokens (one per token tile); their activation scales travel
  // with the block's operands (loaded into the same staging set), so waiting for a scale never waits for a
  // later block's prefetch (loads retire in issue order)
  int xso[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) xso[j] = min(m0 + wm * 64 + 16 * j + r, a.M - 1) * a.KB * 4;
  const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.xs), 0, 0x7fffffff, 0x00020000);
  const float* wsrow = a.ws + static_cast<size_t>(tn) * a.KB;

  u32x4 stg[2][WP + XP];
  float xsc[2][4];
  auto load = [&](int sset, int kb) {
    const unsigned oob = kb < a.KB ? 0u : 0x80000000u;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      xsc[sset][j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sr, static_cast<int>(xso[j] | oob), kb * 4, 0));
#pragma unroll
    for (int i = 0; i < WP; ++i)
      stg[sset][i] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, static_cast<int>(wsrc[i] | oob), kb * kTileBytesFp8, 0));
#pragma unroll
    for (int i = 0; i < XP; ++i)
      stg[sset][WP + i] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, static_cast<int>(xsrc[i] | oob), kb * kRowBytes, 0));
  };
  auto store = [&](int sset, uint8_t* st) {
#pragma unroll
    for (int i = 0; i < WP; ++i) *reinterpret_cast<u32x4*>(st + wdst[i]) = stg[sset][i];
#pragma unroll
    for (int i = 0; i < XP; ++i) *reinterpret_cast<u32x4*>(st + xdst[i]) = stg[sset][WP + i];
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // K block kb: loaded into staging set kb % 2 two iterations ahead, written to LDS buffer kb % 2, computed.
  // LDS buffer kb % 2 was last read by block kb - 2, which every wave finished before the barrier of kb - 1.
  load(0, 0);
  load(1, 1);
  const int KBP = (a.KB + 1) & ~1;
  for (int kb0 = 0; kb0 < KBP; kb0 += 2) {
#pragma unroll
    for (int ph = 0; ph < 2; ++ph) {
      const int kb = kb0 + ph;
      uint8_t* st = smem + ph * kStage;
      store(ph, st);
      // the block's combined scales, taken before this staging set is refilled
      const float wsc = kb < a.KB ? wsrow[kb] : 0.f;
      float sc[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) sc[j] = xsc[ph][j] * wsc;
      __syncthreads();
      load(ph, kb + 2);  // out-of-range blocks load nothing
      if (kb < a.KB) {
        // fragments: weights rows wn*64 + 16i + r, activations rows wm*64 + 16j + r; 32 bytes at K 32t
        i32x8 af[4], bf[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = wn * 64 + 16 * i + r;
          const u32x4 lo = *reinterpret_cast<const u32x4*>(st + lds_off(row, 2 * t));
          const u32x4 hi = *reinterpret_cast<const u32x4*>(st + lds_off(row, 2 * t + 1));
          af[i] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int row = wm * 64 + 16 * j + r;
          const uint8_t* xb = st + kBN * kRowBytes;
          const u32x4 lo = *reinterpret_cast<const u32x4*>(xb + lds_off(row, 2 * t));
          const u32x4 hi = *reinterpret_cast<const u32x4*>(xb + lds_off(row, 2 * t + 1));
          bf[j] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            // E8M0 scale 127 = 1.0 on both operands: the plain FP8 x FP8 product of one 128-value block
            const f32x4 p = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af[i], bf[j], f32x4{0.f, 0.f, 0.f, 0.f},
                                                                            0, 0, 0, 127, 0, 127);
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[i][j][v] = __builtin_fmaf(p[v], sc[j], acc[i][j][v]);
          }
      }
    }
  }

  // epilogue: lane holds rows n = n0 + wn*64 + 16i + 4t + v, token m = m0 + wm*64 + 16j + r
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int m = m0 + wm * 64 + 16 * j + r;
    if (m >= a.M) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = n0 + wn * 64 + 16 * i + 4 * t;
      uint16_t* dst = a.y + static_cast<size_t>(m) * a.ldy + n;
      *reinterpret_cast<u32x2*>(dst) = u32x2{f32_to_bf16(acc[i][j][0]) | (uint32_t(f32_to_bf16(acc[i][j][1])) << 16),
                                             f32_to_bf16(acc[i][j][2]) | (uint32_t(f32_to_bf16(acc[i][j][3])) << 16)};
    }
  }
}

// 1x128 FP8 activation quantizer: one wave per (row, 128-value group); s = amax / 448 (1 for an all-zero
// group), q = E4M3(x / s) rounded to nearest even (|x / s| <= 448 by construction; clamped for safety, which
// is the saturating conversion). Two values per lane.
__global__ void __launch_bounds__(256) quant_fp8_g128_kernel(const uint16_t* __restrict__ x, int M, int K,
                                                             uint8_t* __restrict__ q, float* __restrict__ scale) {
  const int KB = K / 128;
  const long long grp = (static_cast<long long>(blockIdx.x) * 256 + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (grp >= static_cast<long long>(M) * KB) return;
  const int m = static_cast<int>(grp / KB), kb = static_cast<int>(grp % KB);
  const size_t base = static_cast<size_t>(m) * K + static_cast<size_t>(kb) * 128 + 2 * lane;
  const uint32_t pair = *reinterpret_cast<const uint32_t*>(x + base);
  const float v0 = bf16_to_f32(pair & 0xffff), v1 = bf16_to_f32(pair >> 16);
  float mx = fmaxf(fabsf(v0), fabsf(v1));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  const float s = mx > 0.f ? mx / 448.f : 1.f;
  const float a0 = fminf(fmaxf(v0 / s, -448.f), 448.f), a1 = fminf(fmaxf(v1 / s, -448.f), 448.f);
  const uint32_t packed = __builtin_amdgcn_cvt_pk_fp8_f32(a0, a1, 0, false);
  *reinterpret_cast<uint16_t*>(q + base) = static_cast<uint16_t>(packed & 0xffff);
  if (lane == 0) scale[static_cast<size_t>(m) * KB + kb] = s;
}

}  // namespace
}  // namespace lq

using namespace lq;

extern "C" {

int lq_quant_act_fp8_g128(const uint16_t* x, int M, int K, uint8_t* q, float* scale, void* stream) {
  if (M < 1 || K <= 0 || K % 128 != 0) return fail(LQ_ERR_SHAPE, "quant_act_fp8_g128: M >= 1 and K % 128 == 0");
  if (!x || !q || !scale) return fail(LQ_ERR_ARG, "quant_act_fp8_g128: null pointer");
  const long long groups = static_cast<long long>(M) * (K / 128);
  hipLaunchKernelGGL(quant_fp8_g128_kernel, dim3(static_cast<unsigned>((groups + 3) / 4)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, M, K, q, scale);
  return check_launch("quant_act_fp8_g128");
}

int lq_prefill_fp8_block(const uint8_t* xq, const float* xs, int M, const uint8_t* w, const float* ws, uint16_t* y,
                         int ldy, int N, int K, void* stream) {
  if (N <= 0 || K <= 0 || N % 128 != 0 || K % 128 != 0)
    return fail(LQ_ERR_SHAPE, "prefill_gemm: N % 128 and K % 128 must be 0");
  if (M < 1) return LQ_OK;  // nothing to do (the reference returns silently)
  if (ldy < N || ldy % 4 != 0) return fail(LQ_ERR_SHAPE, "prefill_gemm: ldy must be >= N and a multiple of 4");
  if (!xq || !xs || !w || !ws || !y) return fail(LQ_ERR_ARG, "prefill_gemm: null pointer");
  PrefillArgs a{};
  a.xq = xq;
  a.xs = xs;
  a.w = w;
  a.ws = ws;
  a.y = y;
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  a.KB = K / 128;
  a.tiles_m = cdiv(M, kBM);
  a.tiles_n = N / kBN;
  const long long blocks = static_cast<long long>(a.tiles_m) * a.tiles_n;
  // 96 KB of dynamic LDS is above the default per-launch limit; raise it (idempotent, per process).
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_fp8_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          2 * kStage);
  if (attr != hipSuccess) return fail(LQ_ERR_LAUNCH, std::string("prefill_gemm: ") + hipGetErrorString(attr));
  hipLaunchKernelGGL(prefill_fp8_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 2 * kStage,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("prefill_gemm");
}

}  // extern "C"
