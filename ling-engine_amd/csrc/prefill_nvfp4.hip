// NVFP4 prefill GEMMs on gfx950 (reference prefill_gemm_nvfp4 / prefill_swiglu_nvfp4, src/core/prefill_gemm.cu:
// 269-342, 593-704):
//
//   y[m][n] = alpha * sum_k (e2m1(xq[m][k]) * e4m3(xs[m][k/16])) * (e2m1(w[n][k]) * e4m3(ws[n][k/16]))   (+= y)
//
// and the FFN's gate|up form, whose output goes straight into the down projection's NVFP4 encoding:
//   v = BF16(silu(alpha_g * G) * (alpha_u * U)), then NVFP4 blocks of 16 output columns (as quant_act_nvfp4).
//
// CDNA4 has no MFMA that takes E4M3 scales per 16 values (its block-scaled MFMAs take E8M0 per 32), so both
// operands are dequantized in registers to FP16 - exact: an E2M1 value times an E4M3 scale has at most 6
// significant bits and lies in [2^-10, 2688] - and multiplied on v_mfma_f32_16x16x32_f16 with FP32
// accumulation across all of K; alpha is applied at the end.
//
//  * A workgroup (8 waves: 2 along the weights x 4 along the tokens) computes 256 weight rows x 256 tokens; each
//    wave 128 x 64 (8 x 4 MFMA tiles). Per 128-value chunk a lane holds the raw 16 bytes (32 E2M1 values) and
//    2 scale bytes of its row for each of its 8 weight tiles and 4 token tiles, and dequantizes one 8-value
//    step at a time: lane (r, t) supplies K 32t + 8s .. +8 at step s for both operands (a permutation of K
//    inside the chunk, harmless as both operands use it; the weights' tiled layout holds exactly these 16
//    bytes per (row, t), slot r * 4 + t).
//  * Operands go from global memory straight to LDS (buffer loads with the LDS flag): per chunk 16 KB of
//    weight values, 2 KB of weight scales, and the same for the activations, in three stages (108 KB), so the
//    loads of chunk c + 2 overlap the compute of chunk c. The 16-byte units of a 64-byte row are XOR-swizzled
//    by swz4(row) so the 16-byte fragment reads are conflict free whether the LDS serves 8 or 16 lanes of
//    them per cycle.
#include "lq_common.hpp"

#include <algorithm>
#include <string>

namespace lq {
namespace {

constexpr int kBN = 256, kBM = 256, kThreads = 512, kStages = 3, kGroupN = 4;
constexpr int kValBytes = 256 * 64;     // one operand's chunk of values in LDS
constexpr int kScBytes = 256 * 8;       // its E4M3 scales
constexpr int kStage = 2 * (kValBytes + kScBytes);
// stage layout: [A values][A scales][B values][B scales]
constexpr int kOffAs = kValBytes, kOffB = kValBytes + kScBytes, kOffBs = 2 * kValBytes + kScBytes;

// 16 lanes read one 16-byte unit each of rows r .. r + 15 (r % 16 == 0): banks (row % 4, unit) must be distinct
// over the 16 rows, and (row % 2, unit) over each aligned 8.
__device__ __forceinline__ int swz4(int row) { return ((row >> 1) & 3) ^ ((row >> 3) & 1); }
__device__ __forceinline__ int val_off(int row, int u) { return row * 64 + ((u ^ swz4(row)) << 4); }

struct Nvfp4Args {
  const uint8_t* xq;  // [M][K/2]
  const uint8_t* xs;  // [M][K/16]
  const uint8_t* w;   // tiled NVFP4 (raw 1152 B blocks, or coded 1024 B value blocks with wsf)
  const uint8_t* wsf; // coded blob's raw scales (128 B per block) or null
  const uint8_t* w2;  // SwiGLU: the up matrix (gate in w)
  const uint8_t* wsf2;
  float alpha, alpha2;
  float* y;
  int ldy, M, N, K, C;
  int accumulate;
  float gscale_out;  // SwiGLU: 1 / out_input_scale
  uint8_t* q_out;    // [M][N/2]
  uint8_t* sf_out;   // [M][N/16]
  int tiles_m, tiles_n, rows_per_tile;  // rows_per_tile: 256 (plain) or 128 output columns (SwiGLU)
};

typedef __attribute__((address_space(3))) void* lds_ptr;
// soff is uniform over the wave; saying so keeps it in an SGPR (held in a VGPR, the compiler wraps every load in a
// loop over the lanes' distinct values).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rs, uint8_t* lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(lds), 16, voff, __builtin_amdgcn_readfirstlane(soff), 0, 0);
}
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t rs, uint8_t* lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(lds), 4, voff, __builtin_amdgcn_readfirstlane(soff), 0, 0);
}

// Step s of a lane's raw chunk (word d = 8 E2M1 codes of its 16 bytes, two E4M3 scale bytes): 8 FP16 values
// e2m1 * scale (exact); steps 0, 1 use the first scale (K 32t .. +16), steps 2, 3 the second.
__device__ __forceinline__ u32x4 deq_word(uint32_t d, uint32_t sc, int s) {
  const uint32_t b = (s < 2) ? (sc & 0xffu) : ((sc >> 8) & 0xffu);
  const f16x2 scv = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(b | (b << 8), 1.0f, false);
  const f16x2 e0 = fp4x2_to_f16x2<0>(d) * scv, e1 = fp4x2_to_f16x2<1>(d) * scv;
  const f16x2 e2 = fp4x2_to_f16x2<2>(d) * scv, e3 = fp4x2_to_f16x2<3>(d) * scv;
  return u32x4{__builtin_bit_cast(uint32_t, e0), __builtin_bit_cast(uint32_t, e1), __builtin_bit_cast(uint32_t, e2),
               __builtin_bit_cast(uint32_t, e3)};
}

#define LQ_WAIT_VM(n) asm volatile("s_waitcnt vmcnt(" #n ")" ::: "memory")

template <bool SWIGLU>
__global__ void __launch_bounds__(kThreads) prefill_nvfp4_kernel(const Nvfp4Args a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, t = lane >> 4;
  const int wn = wave & 1, wm = wave >> 1;

  // grouped raster per XCD, as the FP8 prefill kernel
  const int nb = gridDim.x, b = blockIdx.x;
  int tile = b;
  if ((nb & 7) == 0) tile = (b & 7) * (nb >> 3) + (b >> 3);
  const int grp = tile / (kGroupN * a.tiles_m), rem = tile % (kGroupN * a.tiles_m);
  const int gsize = min(kGroupN, a.tiles_n - grp * kGroupN);
  const int tn = grp * kGroupN + rem % gsize, tm = rem / gsize;
  const int n0 = tn * a.rows_per_tile, m0 = tm * kBM;

  // weight LDS rows: plain, row = n - n0 (256 rows of w); SwiGLU, rows 0..127 = gate rows n0 .., 128..255 = up
  const int rows_w = SWIGLU ? a.N : a.N;
  const int blkb = a.wsf ? kValueBytesFp4 : kTileBytesFp4;
  const int nbytes = (rows_w / 16) * a.C * blkb;
  const __amdgpu_buffer_rsrc_t wr1 = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.w), 0, nbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t wr2 = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(SWIGLU ? a.w2 : a.w), 0,
                                                                        nbytes, 0x00020000);
  const int sbytes = a.wsf ? (rows_w / 16) * a.C * 128 : nbytes;
  const __amdgpu_buffer_rsrc_t sr1 = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(a.wsf ? a.wsf : a.w), 0, sbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t sr2 = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(SWIGLU ? (a.wsf2 ? a.wsf2 : a.w2) : (a.wsf ? a.wsf : a.w)), 0, sbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.xq), 0, a.M * (a.K / 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t xsr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.xs), 0, a.M * (a.K / 16), 0x00020000);

  // Load plan. Values: load i (0, 1) of wave w writes LDS units P = (i * 8 + w) * 64 + lane: row (i * 8 + w) * 16 +
  // lane / 4, physical unit lane % 4, source unit u = lane % 4 ^ swz4(row) (row % 16 = lane / 4: the same for
  // both loads). Scales: thread x writes 4 bytes at 4x: row x / 2, half x % 2.
  const int vrow = wave * 16 + (lane >> 2), vu = (lane & 3) ^ swz4(lane >> 2);
  auto wrow_src = [&](int row) {  // (matrix half, weight row) of LDS row `row`
    return SWIGLU ? (n0 + (row & 127)) : (n0 + row);
  };
  int wsrc[2], wssrc;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = i * 128 + vrow, n = wrow_src(row);
    const int slot = (n & 15) * 4 + vu;
    wsrc[i] = n < a.N ? ((n >> 4) * a.C) * blkb + slot * 16 : static_cast<int>(0x80000000u);
  }
  const int srow = static_cast<int>(threadIdx.x) >> 1, shalf = threadIdx.x & 1;
  {
    const int n = wrow_src(srow);
    const int so = a.wsf ? ((n >> 4) * a.C) * 128 + (n & 15) * 8 : ((n >> 4) * a.C) * blkb + 1024 + (n & 15) * 8;
    wssrc = n < a.N ? so + shalf * 4 : static_cast<int>(0x80000000u);
  }
  const int sstep = a.wsf ? 128 : blkb;  // scale bytes per chunk step of a block
  int xsrc[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int m = m0 + i * 128 + vrow;
    xsrc[i] = m < a.M ? m * (a.K / 2) + vu * 16 : static_cast<int>(0x80000000u);
  }
  const int xssrc = (m0 + srow) < a.M ? (m0 + srow) * (a.K / 16) + shalf * 4 : static_cast<int>(0x80000000u);

  auto issue = [&](int st, int c) {
    uint8_t* base = smem + st * kStage;
    dma16(wr1, base + (0 * 8 + wave) * 1024, wsrc[0], c * blkb);
    dma16(wr2, base + (1 * 8 + wave) * 1024, wsrc[1], c * blkb);
    if (SWIGLU ? wave < 4 : true) dma4(sr1, base + kOffAs + wave * 256, wssrc, c * sstep);
    else dma4(sr2, base + kOffAs + wave * 256, wssrc, c * sstep);
    dma16(xr, base + kOffB + (0 * 8 + wave) * 1024, xsrc[0], c * 64);
    dma16(xr, base + kOffB + (1 * 8 + wave) * 1024, xsrc[1], c * 64);
    dma4(xsr, base + kOffBs + wave * 256, xssrc, c * 8);
  };

  f32x4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  issue(0, 0);
  if (a.C > 1) issue(1, 1);
  else issue(1, 0);  // keeps the wait counts uniform; the stage is never read
  LQ_WAIT_VM(6);
  __builtin_amdgcn_s_barrier();
  for (int c = 0; c < a.C; ++c) {
    const int st = c % kStages;
    const uint8_t* sa = smem + st * kStage;
    // loads of chunk c + 2 (a repeat of the last chunk past the end, never read, keeps the waits uniform)
    issue((c + 2) % kStages, min(c + 2, a.C - 1));
    // the scale bytes are held for the chunk; each tile's word of step s is read when needed
    uint32_t as[8], bs[4];
#pragma unroll
    for (int i = 0; i < 8; ++i) as[i] = *reinterpret_cast<const uint16_t*>(sa + kOffAs + (wn * 128 + 16 * i + r) * 8 + t * 2);
#pragma unroll
    for (int j = 0; j < 4; ++j) bs[j] = *reinterpret_cast<const uint16_t*>(sa + kOffBs + (wm * 64 + 16 * j + r) * 8 + t * 2);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u32x4 bf[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bf[j] = deq_word(*reinterpret_cast<const uint32_t*>(sa + kOffB + val_off(wm * 64 + 16 * j + r, t) + 4 * s), bs[j], s);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        // (empty volatile statements keep each read in its place: hoisted, the reads run the wave out of registers)
        asm volatile("" ::: "memory");
        const uint32_t d = *reinterpret_cast<const uint32_t*>(sa + val_off(wn * 128 + 16 * i + r, t) + 4 * s);
        const u32x4 af = deq_word(d, as[i], s);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16x16x32(af, bf[j], acc[i][j], true);
      }
      asm volatile("" ::: "memory");
    }
    // this thread's loads of chunk c + 1 have landed (only chunk c + 2's six are newer); after the barrier every
    // wave's have, and every wave is done with stage c
    LQ_WAIT_VM(6);
    __builtin_amdgcn_s_barrier();
  }
  LQ_WAIT_VM(0);

  // lane holds weight rows wn*128 + 16i + 4t + v, token m0 + wm*64 + 16j + r
  if constexpr (!SWIGLU) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = m0 + wm * 64 + 16 * j + r;
      if (m >= a.M) continue;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int n = n0 + wn * 128 + 16 * i + 4 * t;
        if (n >= a.N) continue;
        f32x4 v = f32x4{acc[i][j][0] * a.alpha, acc[i][j][1] * a.alpha, acc[i][j][2] * a.alpha, acc[i][j][3] * a.alpha};
        f32x4* dst = reinterpret_cast<f32x4*>(a.y + static_cast<size_t>(m) * a.ldy + n);
        if (a.accumulate) {
          const f32x4 o = *dst;
          v = f32x4{o[0] + v[0], o[1] + v[1], o[2] + v[2], o[3] + v[3]};
        }
        *dst = v;
      }
    }
  } else {
    // The up waves (wn = 1) hand alpha_up * acc to the gate waves (wn = 0) through LDS, four weight tiles at a
    // time (64 KB): element (i, j, v) of lane L of token quarter wm at ((wm * 4 + ih) * 16 + j * 4 + v) * 64 + L.
    float* xch = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      __syncthreads();
      if (wn == 1) {
#pragma unroll
        for (int ih = 0; ih < 4; ++ih)
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v)
              xch[((wm * 4 + ih) * 16 + j * 4 + v) * 64 + lane] = acc[half * 4 + ih][j][v] * a.alpha2;
      }
      __syncthreads();
      if (wn == 0) {
#pragma unroll
        for (int ih = 0; ih < 4; ++ih) {
          const int i = half * 4 + ih;
          const int ncol = n0 + 16 * i;  // the block's first output column
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float v[4], amax = 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float gv = acc[i][j][e] * a.alpha;
              const float uv = xch[((wm * 4 + ih) * 16 + j * 4 + e) * 64 + lane];
              v[e] = bf16_to_f32(f32_to_bf16((gv / (1.f + __expf(-gv))) * uv));
              amax = fmaxf(amax, fabsf(v[e]));
            }
            // the block's 16 values are in lanes r, r + 16, r + 32, r + 48 (t = 0 .. 3)
            amax = fmaxf(amax, __shfl_xor(amax, 16));
            amax = fmaxf(amax, __shfl_xor(amax, 32));
            const float sraw = a.gscale_out * (amax * (1.f / 6.f));
            const uint32_t sc = __builtin_amdgcn_cvt_pk_fp8_f32(fminf(sraw, 448.f), 0.f, 0, false) & 0xffu;
            const float sv = e4m3_to_f32(sc);
            const float os = sv != 0.f ? 1.f / (sv * (1.f / a.gscale_out)) : 0.f;
            const int m = m0 + wm * 64 + 16 * j + r;
            if (m < a.M && ncol < a.N) {
              uint8_t* qr = a.q_out + static_cast<size_t>(m) * (a.N / 2) + ncol / 2 + 2 * t;
              const uint32_t b0 = e2m1x2_rne(v[0] * os, v[1] * os);
              const uint32_t b1 = e2m1x2_rne(v[2] * os, v[3] * os);
              *reinterpret_cast<uint16_t*>(qr) = static_cast<uint16_t>(b0 | (b1 << 8));
              if (t == 0) a.sf_out[static_cast<size_t>(m) * (a.N / 16) + ncol / 16] = static_cast<uint8_t>(sc);
            }
          }
        }
      }
    }
  }
}

template <bool SWIGLU>
int nvfp4_launch(Nvfp4Args a, const char* name, hipStream_t s) {
  const std::string nm(name);
  if (a.N <= 0 || a.K <= 0 || a.N % 128 != 0 || a.K % 128 != 0)
    return fail(LQ_ERR_SHAPE, nm + ": N % 128 and K % 128 must be 0");
  if (a.M < 1) return LQ_OK;
  if (!SWIGLU && (a.ldy < a.N || a.ldy % 4 != 0)) return fail(LQ_ERR_SHAPE, nm + ": ldy must be >= N and a multiple of 4");
  const long long wb = static_cast<long long>(a.N / 16) * (a.K / 128) * kTileBytesFp4;
  if (wb >= (1LL << 31) || static_cast<long long>(a.M) * (a.K / 2) >= (1LL << 31))
    return fail(LQ_ERR_SHAPE, nm + ": operands must be below 2^31 bytes");
  if (!a.xq || !a.xs || !a.w || (SWIGLU ? (!a.w2 || !a.q_out || !a.sf_out) : !a.y))
    return fail(LQ_ERR_ARG, nm + ": null pointer");
  if (!SWIGLU && reinterpret_cast<uintptr_t>(a.y) % 16 != 0) return fail(LQ_ERR_ARG, nm + ": y must be 16-byte aligned");
  a.C = a.K / 128;
  a.rows_per_tile = SWIGLU ? 128 : kBN;
  a.tiles_m = cdiv(a.M, kBM);
  a.tiles_n = cdiv(a.N, a.rows_per_tile);
  const long long blocks = static_cast<long long>(a.tiles_m) * a.tiles_n;
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_nvfp4_kernel<SWIGLU>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, kStages * kStage);
  if (attr != hipSuccess) return fail(LQ_ERR_LAUNCH, nm + ": " + hipGetErrorString(attr));
  hipLaunchKernelGGL((prefill_nvfp4_kernel<SWIGLU>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads),
                     kStages * kStage, s, a);
  return check_launch(name);
}

}  // namespace
}  // namespace lq

using namespace lq;

extern "C" {

int lq_prefill_gemm_nvfp4(const uint8_t* xq, const uint8_t* xs, int M, const uint8_t* w, float alpha, float* y, int ldy,
                          int N, int K, int accumulate, void* stream, const uint8_t* wsf) {
  Nvfp4Args a{};
  a.xq = xq;
  a.xs = xs;
  a.w = w;
  a.wsf = wsf;
  a.alpha = alpha;
  a.y = y;
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  a.accumulate = accumulate;
  return nvfp4_launch<false>(a, "prefill_gemm_nvfp4", static_cast<hipStream_t>(stream));
}

int lq_prefill_swiglu_nvfp4(const uint8_t* xq, const uint8_t* xs, int M, const uint8_t* gate, float alpha_gate,
                            const uint8_t* up, float alpha_up, int N, int K, float out_input_scale, uint8_t* q_out,
                            uint8_t* sf_out, void* stream, const uint8_t* gate_sf, const uint8_t* up_sf) {
  if ((gate_sf == nullptr) != (up_sf == nullptr))
    return fail(LQ_ERR_ARG, "prefill_swiglu_nvfp4: gate and up must both be raw or both coded");
  Nvfp4Args a{};
  a.xq = xq;
  a.xs = xs;
  a.w = gate;
  a.wsf = gate_sf;
  a.w2 = up;
  a.wsf2 = up_sf;
  a.alpha = alpha_gate;
  a.alpha2 = alpha_up;
  a.M = M;
  a.N = N;
  a.K = K;
  a.gscale_out = 1.f / out_input_scale;
  a.q_out = q_out;
  a.sf_out = sf_out;
  return nvfp4_launch<true>(a, "prefill_swiglu_nvfp4", static_cast<hipStream_t>(stream));
}

}  // extern "C"
