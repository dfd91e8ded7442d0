// Weight-streaming ("skinny") GEMMs for 1..80 rows on gfx950: decode, speculative verify, drafter.
//
//   y[m][n] = epilogue( sum_k x[m][k] * Wq[n][k] ),  Wq = FP8 E4M3 or NVFP4 (E2M1 x E4M3 block scale) codes
//
// The weights are read once from HBM in the reference's tiled layout (a 16-row x 128-value block is
// contiguous); everything else (activations, partial sums) stays in the caches. Design points:
//
//  * MFMA v_mfma_f32_16x16x32_{bf16,f16}: A = 16 weight rows x 32 K, B = 32 K x 16 activation rows.
//    Lane l (r = l % 16, t = l / 16) owns weight row r of a tile and K range [32t, 32t + 32) of each
//    128-value chunk. An FP8 block's 16-byte pieces for that row/range sit at ((h*2+q)*8+g)*4+t
//    (g = r % 8, h = r / 8, q = 0, 1) and an NVFP4 block's at slot r*4+t, so each load instruction of the
//    wave covers whole 512-byte (FP8) or 1024-byte (NVFP4) runs of the block. The MFMA's logical k of
//    step s maps to physical K 32t + 8s + j for the weights and the activations alike, so the dot
//    product is unchanged.
//  * Dequantization in registers, exact: FP8 -> BF16/FP16 with v_cvt_scalef32_pk_*_fp8 (scale 1.0);
//    NVFP4 -> FP16 with v_cvt_scalef32_pk_f16_fp4 (scale 1.0) then one v_pk_mul_f16 by the E4M3 block
//    scale (e2m1 * e4m3 has at most 5 significant bits: exact in FP16). The per-channel / global scale
//    is applied in FP32 in the epilogue.
//  * Work split: units = (tile group of kTiles tiles, K chunk); P workgroups each take a contiguous,
//    equal range of units (a stream-K split), so every CU streams the same number of bytes whatever
//    N and K are. Within a workgroup, wave w takes chunks c0 + w, c0 + w + kWaves, ... and the waves'
//    sums are added in LDS in wave order. A tile group split across workgroups is finished by the last
//    workgroup to arrive (an arrival counter per group), which adds the partial sums in workgroup order.
//  * Determinism and row invariance: P, the tile grouping and the chunk order depend only on N, K and
//    the device's CU count, never on M, and an MFMA's column j depends only on activation row j; so a
//    row's result is bit for bit the same at any M, as the reference guarantees
//    (reference src/core/stream_gemm.cu:10-13).
//  * XCD-aware placement: workgroup ids are permuted so that consecutive ranges of units (and the
//    partials exchanged between them) stay on one XCD's L2.
#include "lq_common.hpp"
#include "lq_workspace.hpp"

#include <algorithm>
#include <cstring>
#include <string>

namespace lq {
namespace {

constexpr int kTiles = 4;  // 16-row tiles per tile group (64 weight rows)
constexpr int kWaves = 4;  // waves per workgroup
constexpr int kThreads = kWaves * kWave;
constexpr int kMaxMats = 4;

enum WFmt { kFp8 = 0, kFp4 = 1, kFp4Coded = 2 };

struct StreamArgs {
  const void* x;      // [M][K] BF16 or FP16
  const float* xinv;  // [M] row scales of an FP16 copy, or null
  int M, K, C;        // C = K / 128
  int P;              // logical workgroups
  long long U;        // units = TG * C
  int TG;             // tile groups
  int count;          // matrices
  const uint8_t* w[kMaxMats];
  const uint8_t* table[kMaxMats];  // coded NVFP4: device scale-code table [64]
  const float* svec[kMaxMats];     // per-channel scales [N] or null
  float sc[kMaxMats];              // scalar scale (used when svec is null)
  void* y[kMaxMats];               // BF16 or FP32 [M][ldy]
  const uint16_t* resid[kMaxMats]; // BF16 residual [M][ldy] or null
  int N[kMaxMats];
  int tg0[kMaxMats + 1];  // first tile group of each matrix; tg0[count] = TG
  int ldy[kMaxMats];
  float* partials;  // [2 * P][kTiles * 16][G * 16]
  int* counters;    // [TG]
};

// One chunk of weights for the lane: FP8 32 bytes (two pieces) per tile; NVFP4 16 bytes + 2 scales.
template <int WF>
struct WRegs {
  u32x4 v[kTiles][WF == kFp8 ? 2 : 1];
  uint32_t sc[kTiles];  // NVFP4: the two E4M3 block scales (raw) or the 12-bit code (coded)
};

template <int G>
struct XRegs {
  u32x4 v[G][4];  // 4 x 8 activations = K [32t, 32t + 32) of row 16g + r
};

template <int WF>
__device__ __forceinline__ void load_w(WRegs<WF>& R, const uint8_t* const (&tb)[kTiles], const uint8_t* const (&cb)[kTiles],
                                       int c, int lane) {
  const int r = lane & 15, t = lane >> 4;
#pragma unroll
  for (int i = 0; i < kTiles; ++i) {
    if constexpr (WF == kFp8) {
      const int p0 = ((r >> 3) * 16 + (r & 7)) * 4 + t;  // piece of q = 0; q = 1 is 32 pieces on
      const uint8_t* b = tb[i] + static_cast<size_t>(c) * kTileBytesFp8 + p0 * 16;
      R.v[i][0] = load_nt(b);
      R.v[i][1] = load_nt(b + 512);
    } else if constexpr (WF == kFp4) {
      const int s = r * 4 + t;
      const uint8_t* b = tb[i] + static_cast<size_t>(c) * kTileBytesFp4;
      R.v[i][0] = load_nt(b + s * 16);
      R.sc[i] = *reinterpret_cast<const uint16_t*>(b + 1024 + s * 2);
    } else {
      const int s = r * 4 + t;
      const uint8_t* b = tb[i] + static_cast<size_t>(c) * kValueBytesFp4;
      R.v[i][0] = load_nt(b + s * 16);
      // slot s < 32: low byte at 2s, high nibble in the low half of byte 64 + s; slot 32 + L: byte 2L + 1
      // and the high half of byte 64 + L (reference src/core/stream_gemm.cu:740-780).
      const uint8_t* cd = cb[i] + static_cast<size_t>(c) * kCodeBytesFp4;
      const int L = s & 31, hi = s >> 5;
      const uint32_t lo = cd[2 * L + hi], nib = (cd[64 + L] >> (4 * hi)) & 15u;
      R.sc[i] = lo | (nib << 8);
    }
  }
}

template <int G>
__device__ __forceinline__ void load_x(XRegs<G>& X, const uint8_t* const (&xrow)[G], int c) {
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const uint8_t* p = xrow[g] + static_cast<size_t>(c) * (kChunk * 2);
#pragma unroll
    for (int s = 0; s < 4; ++s) X.v[g][s] = load16(p + 16 * s);
  }
}

// The A operand of MFMA step s (8 weights, K 32t + 8s .. +8) for tile i.
template <int WF, bool F16>
__device__ __forceinline__ u32x4 a_operand(const WRegs<WF>& R, int i, int s, const uint8_t* tab) {
  if constexpr (WF == kFp8) {
    const u32x4& v = R.v[i][s >> 1];
    const uint32_t d0 = (s & 1) ? v.z : v.x, d1 = (s & 1) ? v.w : v.y;
    const u32x2 a = F16 ? fp8x4_to_f16x4(d0) : fp8x4_to_bf16x4(d0);
    const u32x2 b = F16 ? fp8x4_to_f16x4(d1) : fp8x4_to_bf16x4(d1);
    return u32x4{a.x, a.y, b.x, b.y};
  } else {
    // the two block scales (K [32t, +16) and [32t + 16, +32)); s < 2 uses the first
    uint32_t scb;
    if constexpr (WF == kFp4) scb = (s < 2) ? (R.sc[i] & 0xffu) : (R.sc[i] >> 8);
    else scb = tab[(s < 2) ? (R.sc[i] & 63u) : (R.sc[i] >> 6)];
    const f16x2 scv = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(scb | (scb << 8), 1.0f, false);
    const uint32_t d = s == 0 ? R.v[i][0].x : s == 1 ? R.v[i][0].y : s == 2 ? R.v[i][0].z : R.v[i][0].w;
    const f16x2 e0 = fp4x2_to_f16x2<0>(d) * scv, e1 = fp4x2_to_f16x2<1>(d) * scv;
    const f16x2 e2 = fp4x2_to_f16x2<2>(d) * scv, e3 = fp4x2_to_f16x2<3>(d) * scv;
    return u32x4{__builtin_bit_cast(uint32_t, e0), __builtin_bit_cast(uint32_t, e1), __builtin_bit_cast(uint32_t, e2),
                 __builtin_bit_cast(uint32_t, e3)};
  }
}

template <int WF, bool F16, int G>
__device__ __forceinline__ void compute(const WRegs<WF>& R, const XRegs<G>& X, f32x4 (&acc)[kTiles][G],
                                        const uint8_t* const (&tab)[kTiles]) {
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int i = 0; i < kTiles; ++i) {
      const u32x4 a = a_operand<WF, F16>(R, i, s, tab[i]);
#pragma unroll
      for (int g = 0; g < G; ++g) acc[i][g] = mfma16x16x32(a, X.v[g][s], acc[i][g], F16);
    }
}

__device__ __forceinline__ float silu(float v) { return v / (1.0f + __expf(-v)); }

// Applies the epilogue to one reduced sum and stores it. `row` is the tile group's row (0 .. 63).
template <bool PAIR, bool OUTF32, int G>
__device__ __forceinline__ void epilogue_store(const StreamArgs& a, int mi, int tile0, float (*red)[G * 16 + 1],
                                               int row, int tok) {
  if constexpr (PAIR) {
    const int n = tile0 * 16 + row;  // gate / up column
    if (n >= a.N[0]) return;
    const float g = red[row][tok], u = red[row + kTiles * 8][tok];
    const float gs = g * (a.svec[0] ? a.svec[0][n] : a.sc[0]);
    const float us = u * (a.svec[1] ? a.svec[1][n] : a.sc[1]);
    reinterpret_cast<uint16_t*>(a.y[0])[static_cast<size_t>(tok) * a.ldy[0] + n] = f32_to_bf16(silu(gs) * us);
  } else {
    const int n = tile0 * 16 + row;
    if (n >= a.N[mi]) return;
    float v = red[row][tok] * (a.svec[mi] ? a.svec[mi][n] : a.sc[mi]);
    if (a.xinv) v = v * a.xinv[tok];
    const size_t o = static_cast<size_t>(tok) * a.ldy[mi] + n;
    if constexpr (OUTF32) {
      reinterpret_cast<float*>(a.y[mi])[o] = v;
    } else {
      if (a.resid[mi]) v = v + bf16_to_f32(a.resid[mi][o]);
      reinterpret_cast<uint16_t*>(a.y[mi])[o] = f32_to_bf16(v);
    }
  }
}

__device__ __forceinline__ int wg_of_unit(long long u, int P, long long U) {
  return static_cast<int>(((u + 1) * P - 1) / U);
}
__device__ __forceinline__ long long unit_start(int p, int P, long long U) { return static_cast<long long>(p) * U / P; }

template <int G, int WF, bool F16, bool PAIR, bool OUTF32>
__global__ void __launch_bounds__(kThreads) stream_kernel(const StreamArgs a) {
  constexpr int ROWS = kTiles * 16, COLS = G * 16;
  __shared__ float red[ROWS][COLS + 1];
  __shared__ uint8_t tabs[kMaxMats][64];
  __shared__ int last_flag;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, t = lane >> 4;

  if constexpr (WF == kFp4Coded) {
    for (int i = threadIdx.x; i < a.count * 64; i += kThreads) tabs[i >> 6][i & 63] = a.table[i >> 6][i & 63];
    __syncthreads();
  }

  // Logical workgroup id: blockIdx.x % 8 is the XCD the hardware places it on; consecutive logical ids
  // share an XCD, so a tile group's partials are exchanged within one L2.
  int p = blockIdx.x;
  if ((a.P & 7) == 0) p = (blockIdx.x & 7) * (a.P >> 3) + (blockIdx.x >> 3);
  const long long u0 = unit_start(p, a.P, a.U), u1 = unit_start(p + 1, a.P, a.U);
  const int tg_first = static_cast<int>(u0 / a.C);

  // Activation row pointers of this lane (rows past M read row M - 1; their columns are never stored).
  const uint8_t* xrow[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int m = min(16 * g + r, a.M - 1);
    xrow[g] = reinterpret_cast<const uint8_t*>(a.x) + (static_cast<size_t>(m) * a.K + 32 * t) * 2;
  }

  for (long long u = u0; u < u1;) {
    const int tg = static_cast<int>(u / a.C), c0 = static_cast<int>(u % a.C);
    const int c1 = static_cast<int>(min(static_cast<long long>(a.C), c0 + (u1 - u)));
    u += c1 - c0;

    // The tile group's tiles: PAIR = kTiles/2 gate tiles then the same up tiles; else kTiles tiles of one matrix.
    int mi = 0;
    if constexpr (!PAIR) {
      while (mi + 1 < a.count && tg >= a.tg0[mi + 1]) ++mi;
    }
    const int tile0 = PAIR ? tg * (kTiles / 2) : (tg - a.tg0[mi]) * kTiles;
    const uint8_t* tb[kTiles];
    const uint8_t* cb[kTiles];
    const uint8_t* tab[kTiles];
#pragma unroll
    for (int i = 0; i < kTiles; ++i) {
      const int m = PAIR ? (i < kTiles / 2 ? 0 : 1) : mi;
      const int tile = min((PAIR ? tile0 + (i % (kTiles / 2)) : tile0 + i), a.N[m] / 16 - 1);
      const size_t blk = WF == kFp8 ? kTileBytesFp8 : WF == kFp4 ? kTileBytesFp4 : kValueBytesFp4;
      tb[i] = a.w[m] + static_cast<size_t>(tile) * a.C * blk;
      cb[i] = a.w[m] + static_cast<size_t>(a.N[m] / 16) * a.C * kValueBytesFp4 +
              static_cast<size_t>(tile) * a.C * kCodeBytesFp4;
      tab[i] = tabs[m];
    }

    f32x4 acc[kTiles][G];
#pragma unroll
    for (int i = 0; i < kTiles; ++i)
#pragma unroll
      for (int g = 0; g < G; ++g) acc[i][g] = f32x4{0.f, 0.f, 0.f, 0.f};

    int c = c0 + wave;
    if (c < c1) {
      WRegs<WF> cur;
      load_w<WF>(cur, tb, cb, c, lane);
      for (; c < c1; c += kWaves) {
        WRegs<WF> nxt;
        const bool more = c + kWaves < c1;
        if (more) load_w<WF>(nxt, tb, cb, c + kWaves, lane);
        XRegs<G> X;
        load_x<G>(X, xrow, c);
        compute<WF, F16, G>(cur, X, acc, tab);
        if (more) cur = nxt;
      }
    }

    // Waves' sums into LDS in wave order: red[16i + 4t + v][16g + r].
#pragma unroll 1
    for (int w = 0; w < kWaves; ++w) {
      if (wave == w) {
#pragma unroll
        for (int i = 0; i < kTiles; ++i)
#pragma unroll
          for (int g = 0; g < G; ++g)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              float& d = red[16 * i + 4 * t + v][16 * g + r];
              d = (w == 0) ? acc[i][g][v] : d + acc[i][g][v];
            }
      }
      __syncthreads();
    }

    const int out_rows = PAIR ? ROWS / 2 : ROWS;
    if (c0 == 0 && c1 == a.C) {
      for (int e = threadIdx.x; e < out_rows * a.M; e += kThreads)
        epilogue_store<PAIR, OUTF32, G>(a, mi, tile0, red, e % out_rows, e / out_rows);
      __syncthreads();
      continue;
    }

    // Split tile group: publish this workgroup's partial, count arrivals; the last one adds all partials
    // in workgroup order and applies the epilogue.
    const int pf = wg_of_unit(static_cast<long long>(tg) * a.C, a.P, a.U);
    const int pl = wg_of_unit(static_cast<long long>(tg) * a.C + a.C - 1, a.P, a.U);
    constexpr int SLOT = ROWS * COLS;
    float* slot = a.partials + static_cast<size_t>(2 * p + (tg == tg_first ? 0 : 1)) * SLOT;
    for (int e = threadIdx.x; e < SLOT; e += kThreads) slot[e] = red[e / COLS][e % COLS];
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
      const int old = atomicAdd(a.counters + tg, 1);
      last_flag = old == pl - pf;
      if (last_flag) atomicExch(a.counters + tg, 0);
    }
    __syncthreads();
    if (last_flag) {
      __threadfence();
      for (int e = threadIdx.x; e < SLOT; e += kThreads) {
        float s = 0.f;
        for (int q = pf; q <= pl; ++q) {
          const int qf = static_cast<int>(unit_start(q, a.P, a.U) / a.C);
          const float* sq = a.partials + static_cast<size_t>(2 * q + (tg == qf ? 0 : 1)) * SLOT;
          const float v = __builtin_nontemporal_load(sq + e);
          s = (q == pf) ? v : s + v;
        }
        red[e / COLS][e % COLS] = s;
      }
      __syncthreads();
      for (int e = threadIdx.x; e < out_rows * a.M; e += kThreads)
        epilogue_store<PAIR, OUTF32, G>(a, mi, tile0, red, e % out_rows, e / out_rows);
    }
    __syncthreads();
  }
}

// ---------------- activation copies (reference src/core/stream_gemm.cu:480-566) ----------------
// Grid (M, S): every block finds the row's largest magnitude (a maximum is exact in any order, so all
// blocks agree) and converts its slice of K: xh = f16_rn(x * 2^(15 - e)), xinv = 2^(e - 15).
template <bool BF16IN>
__global__ void __launch_bounds__(256) half_rows_kernel(const void* __restrict__ x, int K, int slice,
                                                        _Float16* __restrict__ out, float* __restrict__ xinv) {
  __shared__ float red[4];
  const size_t m = blockIdx.x;
  auto val = [&](int k) -> float {
    if constexpr (BF16IN) return bf16_to_f32(reinterpret_cast<const uint16_t*>(x)[m * K + k]);
    else return reinterpret_cast<const float*>(x)[m * K + k];
  };
  float mx = 0.f;
  for (int k = threadIdx.x; k < K; k += 256) mx = fmaxf(mx, fabsf(val(k)));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int e = 0;
  if (mx > 0.f && isfinite(mx)) frexpf(mx, &e);
  const float s = ldexpf(1.f, 15 - e);
  const int k0 = blockIdx.y * slice, k1 = min(K, k0 + slice);
  for (int k = k0 + threadIdx.x; k < k1; k += 256) out[m * K + k] = static_cast<_Float16>(val(k) * s);
  if (blockIdx.y == 0 && threadIdx.x == 0) xinv[m] = ldexpf(1.f, e - 15);
}

// ---------------- host side ----------------

struct Mat {
  const uint8_t* w;
  const uint8_t* table;
  const float* svec;
  float sc;
  void* y;
  const uint16_t* resid;
  int N;
  int ldy;
};

// Workgroups per launch: about two per CU, a multiple of 8 (one share per XCD), never more than the units.
// Depends only on the unit count and the device, never on M (row invariance).
int choose_wgs(long long U) {
  int dev = 0;
  (void)hipGetDevice(&dev);
  long long P = static_cast<long long>(device_cus(dev)) * 2;
  if (P > U) P = U;
  if (P >= 8) P -= P % 8;
  return static_cast<int>(std::max<long long>(P, 1));
}

template <int G, int WF, bool F16, bool PAIR, bool OUTF32>
int launch_g(const StreamArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((stream_kernel<G, WF, F16, PAIR, OUTF32>), dim3(a.P), dim3(kThreads), 0, s, a);
  return check_launch("stream_gemm");
}

template <int WF, bool F16, bool PAIR, bool OUTF32>
int launch_m(const StreamArgs& a, hipStream_t s) {
  switch (cdiv(a.M, 16)) {
    case 1: return launch_g<1, WF, F16, PAIR, OUTF32>(a, s);
    case 2: return launch_g<2, WF, F16, PAIR, OUTF32>(a, s);
    case 3: return launch_g<3, WF, F16, PAIR, OUTF32>(a, s);
    case 4: return launch_g<4, WF, F16, PAIR, OUTF32>(a, s);
    default: return launch_g<5, WF, F16, PAIR, OUTF32>(a, s);
  }
}

// Validates, fills the launch arguments and launches. `fmt`: weight format; `f16`: activations are an
// FP16 row copy (with xinv) rather than BF16; `pair`: mats = {gate, up} with the SiLU*mul epilogue.
int stream_launch(const char* name, int fmt, bool f16, bool pair, bool outf32, const void* x, const float* xinv, int M,
                  const Mat* mats, int n, int K, hipStream_t s) {
  const std::string nm(name);
  if (K <= 0 || K % kChunk != 0) return fail(LQ_ERR_SHAPE, nm + ": K must be a multiple of 128");
  if (M < 1 || M > LQ_MAX_STREAM_ROWS) return fail(LQ_ERR_SHAPE, nm + ": M must be in [1, 80]");
  if (n < 1 || n > kMaxMats) return fail(LQ_ERR_SHAPE, nm + ": 1 to 4 matrices per launch");
  if (!x) return fail(LQ_ERR_ARG, nm + ": null activations");
  if (f16 && !xinv) return fail(LQ_ERR_ARG, nm + ": null xinv");
  StreamArgs a{};
  a.x = x;
  a.xinv = xinv;
  a.M = M;
  a.K = K;
  a.C = K / kChunk;
  a.count = n;
  int tg = 0;
  for (int i = 0; i < n; ++i) {
    const Mat& m = mats[i];
    if (m.N <= 0 || m.N % 16 != 0) return fail(LQ_ERR_SHAPE, nm + ": N % 16 and K % 128 must be 0");
    if (!m.w || !m.y) return fail(LQ_ERR_ARG, nm + ": null weight or output");
    if (fmt == kFp4Coded && !m.table) return fail(LQ_ERR_ARG, nm + ": null scale-code table");
    a.w[i] = m.w;
    a.table[i] = m.table;
    a.svec[i] = m.svec;
    a.sc[i] = m.sc;
    a.y[i] = m.y;
    a.resid[i] = m.resid;
    a.N[i] = m.N;
    a.ldy[i] = m.ldy;
    a.tg0[i] = tg;
    if (!pair) tg += cdiv(m.N / 16, kTiles);
  }
  if (pair) {
    if (n != 2 || mats[0].N != mats[1].N) return fail(LQ_ERR_SHAPE, nm + ": gate and up must have the same N");
    tg = cdiv(mats[0].N / 16, kTiles / 2);
  }
  a.tg0[n] = tg;
  a.TG = tg;
  a.U = static_cast<long long>(tg) * a.C;
  a.P = choose_wgs(a.U);
  Workspace* ws = workspace_for_current_device();
  if (!ws) return LQ_ERR_DEVICE;
  const size_t slot_floats = static_cast<size_t>(kTiles * 16) * (cdiv(M, 16) * 16);
  int rc = ws->reserve_stream(static_cast<size_t>(2) * a.P * slot_floats * sizeof(float), static_cast<size_t>(tg));
  if (rc) return rc;
  a.partials = ws->partials;
  a.counters = ws->counters;
  if (pair) return f16 ? launch_m<kFp8, true, true, false>(a, s) : launch_m<kFp8, false, true, false>(a, s);
  if (fmt == kFp8) {
    if (f16) return outf32 ? launch_m<kFp8, true, false, true>(a, s) : launch_m<kFp8, true, false, false>(a, s);
    return outf32 ? launch_m<kFp8, false, false, true>(a, s) : launch_m<kFp8, false, false, false>(a, s);
  }
  if (!f16) return fail(LQ_ERR_ARG, nm + ": NVFP4 streams FP16 activations");
  if (fmt == kFp4) return outf32 ? launch_m<kFp4, true, false, true>(a, s) : launch_m<kFp4, true, false, false>(a, s);
  return outf32 ? launch_m<kFp4Coded, true, false, true>(a, s) : launch_m<kFp4Coded, true, false, false>(a, s);
}

// Shape checks first (the reference throws these before looking at pointers).
int check_rows(const char* name, int M, int N, int K) {
  const std::string nm(name);
  if (K <= 0 || K % kChunk != 0) return fail(LQ_ERR_SHAPE, nm + ": K must be a multiple of 128");
  if (M < 1 || M > LQ_MAX_STREAM_ROWS) return fail(LQ_ERR_SHAPE, nm + ": M must be in [1, 80]");
  if (N <= 0 || N % 16 != 0) return fail(LQ_ERR_SHAPE, nm + ": N % 16 and K % 128 must be 0");
  return LQ_OK;
}

int half_rows(bool bf16in, const void* x, int M, int K, uint16_t* xh, float* xinv, hipStream_t s) {
  const char* nm = bf16in ? "bf16_to_half_rows" : "to_half_rows";
  if (M < 1 || K < 1) return fail(LQ_ERR_SHAPE, std::string(nm) + ": M and K must be positive");
  if (!x || !xh || !xinv) return fail(LQ_ERR_ARG, std::string(nm) + ": null pointer");
  const int split = std::max(1, std::min(K / 1024, cdiv(192, M)));
  const int slice = cdiv(K, split);
  const dim3 grid(M, cdiv(K, slice));
  if (bf16in)
    hipLaunchKernelGGL(half_rows_kernel<true>, grid, dim3(256), 0, s, x, K, slice, reinterpret_cast<_Float16*>(xh), xinv);
  else
    hipLaunchKernelGGL(half_rows_kernel<false>, grid, dim3(256), 0, s, x, K, slice, reinterpret_cast<_Float16*>(xh), xinv);
  return check_launch(nm);
}

}  // namespace
}  // namespace lq

using namespace lq;

extern "C" {

int lq_to_half_rows(const float* x, int M, int K, uint16_t* xh, float* xinv, void* stream) {
  return half_rows(false, x, M, K, xh, xinv, static_cast<hipStream_t>(stream));
}

int lq_bf16_to_half_rows(const uint16_t* x, int M, int K, uint16_t* xh, float* xinv, void* stream) {
  return half_rows(true, x, M, K, xh, xinv, static_cast<hipStream_t>(stream));
}

int lq_stream_gemm_fp8(const uint16_t* xh, const float* xinv, int M, const uint8_t* w, float wscale, float* y, int N,
                       int K, void* stream) {
  const Mat m{w, nullptr, nullptr, wscale, y, nullptr, N, N};
  return stream_launch("stream_gemm", kFp8, true, false, true, xh, xinv, M, &m, 1, K, static_cast<hipStream_t>(stream));
}

int lq_stream_gemm_nvfp4(const uint16_t* xh, const float* xinv, int M, const uint8_t* w, const uint8_t* table,
                         float scale2, float* y, int N, int K, void* stream) {
  const Mat m{w, table, nullptr, scale2, y, nullptr, N, N};
  return stream_launch("stream_gemm", table ? kFp4Coded : kFp4, true, false, true, xh, xinv, M, &m, 1, K,
                       static_cast<hipStream_t>(stream));
}

int lq_stream_gemm_multi(int nvfp4, const uint16_t* xh, const float* xinv, int M, const lq_stream_target* t, int n,
                         int K, void* stream) {
  if (n < 1 || n > kMaxMats) return fail(LQ_ERR_SHAPE, "stream_gemm: 1 to 4 matrices per launch");
  if (!t) return fail(LQ_ERR_ARG, "stream_gemm: null targets");
  Mat coded[kMaxMats], plain[kMaxMats];
  int nc = 0, np = 0;
  for (int i = 0; i < n; ++i) {
    const Mat m{t[i].w, nvfp4 ? t[i].wscale : nullptr, nullptr, t[i].scale, t[i].y, nullptr, t[i].N, t[i].N};
    (m.table ? coded[nc++] : plain[np++]) = m;
  }
  const hipStream_t s = static_cast<hipStream_t>(stream);
  // A launch streams one weight format; coded and raw NVFP4 blobs in one call go as two launches (a matrix's
  // result does not depend on its launch companions).
  if (nc) {
    const int rc = stream_launch("stream_gemm", kFp4Coded, true, false, true, xh, xinv, M, coded, nc, K, s);
    if (rc) return rc;
  }
  if (np) return stream_launch("stream_gemm", nvfp4 ? kFp4 : kFp8, true, false, true, xh, xinv, M, plain, np, K, s);
  return LQ_OK;
}

int lq_stream_fp8_pc(const uint16_t* x, int M, const uint8_t* w, const float* wscale_n, uint16_t* y, int N, int K,
                     void* stream) {
  if (int rc = check_rows("stream_fp8_pc", M, N, K)) return rc;
  if (!wscale_n) return fail(LQ_ERR_ARG, "stream_fp8_pc: null scales");
  const Mat m{w, nullptr, wscale_n, 0.f, y, nullptr, N, N};
  return stream_launch("stream_fp8_pc", kFp8, false, false, false, x, nullptr, M, &m, 1, K,
                       static_cast<hipStream_t>(stream));
}

int lq_stream_fp8_pc_silu_mul(const uint16_t* x, int M, const uint8_t* w_gate, const float* s_gate,
                              const uint8_t* w_up, const float* s_up, uint16_t* h, int N, int K, void* stream) {
  if (int rc = check_rows("stream_fp8_pc_silu_mul", M, N, K)) return rc;
  if (!s_gate || !s_up) return fail(LQ_ERR_ARG, "stream_fp8_pc_silu_mul: null scales");
  const Mat m[2] = {{w_gate, nullptr, s_gate, 0.f, h, nullptr, N, N}, {w_up, nullptr, s_up, 0.f, h, nullptr, N, N}};
  return stream_launch("stream_fp8_pc_silu_mul", kFp8, false, true, false, x, nullptr, M, m, 2, K,
                       static_cast<hipStream_t>(stream));
}

int lq_stream_fp8_pc_residual(const uint16_t* x, int M, const uint8_t* w, const float* wscale_n,
                              const uint16_t* resid, uint16_t* y, int N, int K, void* stream) {
  if (int rc = check_rows("stream_fp8_pc_residual", M, N, K)) return rc;
  if (!wscale_n || !resid) return fail(LQ_ERR_ARG, "stream_fp8_pc_residual: null scales or residual");
  const Mat m{w, nullptr, wscale_n, 0.f, y, resid, N, N};
  return stream_launch("stream_fp8_pc_residual", kFp8, false, false, false, x, nullptr, M, &m, 1, K,
                       static_cast<hipStream_t>(stream));
}

int lq_stream_nvfp4_bf16(const uint16_t* x, int M, const uint8_t* w, const uint8_t* table, float scale2, uint16_t* y,
                         int N, int K, void* stream) {
  if (int rc = check_rows("stream_nvfp4_bf16", M, N, K)) return rc;
  Workspace* ws = workspace_for_current_device();
  if (!ws) return LQ_ERR_DEVICE;
  int rc = ws->reserve_half(static_cast<size_t>(M) * K);
  if (rc) return rc;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  rc = half_rows(true, x, M, K, ws->xh, ws->xinv, s);
  if (rc) return rc;
  const Mat m{w, table, nullptr, scale2, y, nullptr, N, N};
  return stream_launch("stream_nvfp4_bf16", table ? kFp4Coded : kFp4, true, false, false, ws->xh, ws->xinv, M, &m, 1, K,
                       s);
}

}  // extern "C"
