// Block-scaled FP8 prefill GEMM on gfx950 MFMA, and the 1x128 FP8 activation quantizer that feeds it.
//
//   y[m][n] = bf16( sum_kb (sum_{k in kb} e4m3(xq[m][k]) * e4m3(wq[n][k])) * xs[m][kb] * ws[n/128][kb] )
//
// xq: FP8 E4M3 activations [M][K] (row-major) with one FP32 scale per 1x128 group, xs [M][K/128];
// wq: FP8 E4M3 weights in the tiled layout the skinny GEMMs stream (reference
// src/core/stream_gemm.cu:705-738), with one FP32 scale per 128x128 block, ws [N/128][K/128].
//
// Design:
//  * One v_mfma_scale_f32_16x16x128_f8f6f4 per 16x16 output tile per 128-value K block: an MFMA covers exactly one
//    scale block, so its FP32 result is scaled once and added to the accumulator (one FMA per output per
//    block). Any permutation of K inside the block is harmless, since A and B use the same one.
//  * Weights are the A operand (rows n) and activations the B operand (columns m). A workgroup (8 waves, 2 per
//    SIMD: 2 along the weights x 4 along the tokens) computes 256 weight rows x 256 tokens; each wave 128 x 64
//    (8 x 4 MFMA tiles, 128 accumulator registers). A wave's 128 weight rows are one weight scale block, so
//    the block scale is a scalar and each lane's scale is that scalar times its token's activation scale.
//  * Operands reach LDS without passing through registers: buffer loads with the LDS flag write each lane's
//    16 bytes at the next 16 bytes of a 1 KB run, and the lane-to-source map implements the layout: a K
//    block of a 256-row operand is [row][8 x 16-byte units] with the unit index XOR-swizzled by the row, so
//    the fragment reads are bank-conflict free. The block's activation scales come along the same way.
//  * Two LDS stages (65 KB each): while a K block is computed from one, the next block's loads fill the
//    other. The waits are explicit: the compiler cannot see which LDS bytes a load-to-LDS writes.
//  * Tile order: each XCD works through a contiguous range of a grouped raster (kGroupN weight tiles x every
//    token tile per group), so the workgroups running at once on an XCD share the K slices of both operands
//    in its L2 instead of re-streaming the whole activation matrix per weight tile.
#include "lq_common.hpp"
#include "lq_workspace.hpp"

#include <algorithm>
#include <string>

namespace lq {
namespace {

constexpr int kBN = 256;  // weight rows per workgroup
constexpr int kBM = 256;  // tokens per workgroup
constexpr int kThreads = 512;
constexpr int kGroupN = 8;                       // weight tiles per raster group (config 4: 2-6 % faster than 2, 4 or 16)
constexpr int kMaxSplit = 4;                     // K parts of a tail tile
constexpr int kRowBytes = 128;                   // one K block of one row (FP8)
constexpr int kOpBytes = 256 * kRowBytes;        // one operand's K block in LDS: 32 KB
constexpr int kStage = 2 * kOpBytes + kBM * 4;   // weights, activations, activation scales: 65 KB

// Byte offset of 16-byte unit u of row `row` in an LDS operand tile: the unit index is XOR-swizzled by
// swz(row). A fragment read has 16 lanes reading one unit each of rows r .. r + 15 (r % 16 == 0). swz makes
// every aligned group of 8 rows hit 8 distinct units (8 lanes x 16 bytes cover the 32 banks once) and every
// group of 16 rows hit distinct (row parity, unit) pairs (16 lanes cover 64 banks once), so the reads are
// conflict free whether the LDS serves 8 or 16 lanes of a 16-byte read per cycle (measured: no bank
// conflicts; the former swizzle by row / 2 had them on half of all LDS cycles).
__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }
__device__ __forceinline__ int lds_off(int row, int u) { return row * kRowBytes + ((u ^ swz(row)) << 4); }

struct PrefillArgs {
  const uint8_t* xq;
  const float* xs;  // block-scaled: activation group scales [M][K/128]
  const uint8_t* w;
  const float* ws;  // block-scaled: weight block scales [N/128][K/128]
  float alpha;      // per-tensor: the one scale (input scale x weight scale)
  void* y;          // BF16 or FP32 [M][ldy]
  int ldy, M, N, K, KB;
  int tiles_m, tiles_n;
  // Tail split: tiles [full, full + rem) of the logical order are each computed by S workgroups over
  // consecutive K ranges; their FP32 partials meet in part[(rt * S + p) * kBN * kBM] and the last part to
  // arrive (counter cnt[rt]) adds them in part order and writes the tile.
  int full, rem, S;
  float* part;
  int* cnt;
};

// Output of a prefill GEMM: BF16, FP32, or FP32 added to what y holds.
enum PrefillOut { kOutBf16 = 0, kOutF32 = 1, kOutF32Acc = 2 };

typedef __attribute__((address_space(3))) void* lds_ptr;

// soff is uniform over the wave; saying so keeps it in an SGPR (held in a VGPR, the compiler wraps every load in a
// loop over the lanes' distinct values).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rs, uint8_t* lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(lds), 16, voff, __builtin_amdgcn_readfirstlane(soff), 0, 0);
}
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t rs, uint8_t* lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(lds), 4, voff, __builtin_amdgcn_readfirstlane(soff), 0, 0);
}
// s_waitcnt with only vmcnt / lgkmcnt constrained (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8])
#define LQ_WAIT_VM0() __builtin_amdgcn_s_waitcnt(0x0f70)
#define LQ_WAIT_LGKM0() __builtin_amdgcn_s_waitcnt(0xc07f)

// BLOCK: the block-scaled form (each 128-value block's product scaled by its activation and weight scales and
// folded into the accumulators); else one scale for the whole product, applied at the end, and the MFMAs
// accumulate across K themselves.
template <bool BLOCK, int OUT>
__global__ void __launch_bounds__(kThreads) prefill_fp8_kernel(const PrefillArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, t = lane >> 4;
  const int wn = wave & 1, wm = wave >> 1;  // the wave's 128-row weight half and 64-token quarter

  // Tile order. The hardware places block b on XCD b % 8; each XCD takes a contiguous range of the logical
  // tile order, in which tiles come in groups of kGroupN weight tiles x all token tiles, token tile slowest
  // within a group.
  // Split workgroups come after the whole tiles (the hardware dispatches in order, so they fill the last,
  // partial round); the S parts of a tile are on one XCD (same blockIdx % 8), sharing its L2.
  const int b = blockIdx.x;
  int tile = b, kb0 = 0, kb1 = a.KB, part = -1, rt = 0;
  if (b < a.full) {
    if ((a.full & 7) == 0) tile = (b & 7) * (a.full >> 3) + (b >> 3);
  } else {
    const int sidx = b - a.full, q = sidx >> 3;
    rt = (q / a.S) * 8 + (sidx & 7);
    part = q % a.S;
    if (rt >= a.rem) return;
    tile = a.full + rt;
    kb0 = part * a.KB / a.S;
    kb1 = (part + 1) * a.KB / a.S;
  }
  const int grp = tile / (kGroupN * a.tiles_m), rem = tile % (kGroupN * a.tiles_m);
  const int gsize = min(kGroupN, a.tiles_n - grp * kGroupN);
  const int tn = grp * kGroupN + rem % gsize, tm = rem / gsize;
  const int n0 = tn * kBN, m0 = tm * kBM;

  // Buffer resources sized to the operands: loads past the end (rows past N or M) return nothing.
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.w), 0, a.N * a.K, 0x00020000);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.xq), 0, a.M * a.K, 0x00020000);
  const __amdgpu_buffer_rsrc_t sr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.xs), 0, a.M * a.KB * 4, 0x00020000);

  // Load-to-LDS plan: load i (0..3) of wave w writes LDS bytes [((i * 8 + w) * 64 + lane) * 16, +16) of an
  // operand tile: row = (i * 8 + w) * 8 + lane / 8, swizzled unit lane % 8, i.e. source unit u = lane % 8 ^ swz(row)
  // (the same for every i, as i moves the row by 64). Weights: the row's 16-row tile tw and row rr in it; unit
  // u = 2 tt + q sits at tiled piece ((h*2 + q)*8 + g)*4 + tt (g = rr % 8, h = rr / 8); load i is 4 tiles on.
  // Activations: row-major, load i is 64 rows on (a multiple of 16 rows: swz is the same). The per-i and per-block steps go in the scalar offset.
  const int row0 = wave * 8 + (lane >> 3), u0 = (lane & 7) ^ swz(row0);
  const int wsrc = (((n0 >> 4) + (row0 >> 4)) * a.KB) * kTileBytesFp8 +
                   (((((row0 & 15) >> 3) * 2 + (u0 & 1)) * 8 + (row0 & 7)) * 4 + (u0 >> 1)) * 16;
  const int xsrc = (m0 + row0) * a.K + u0 * 16;
  const int wstep = 4 * a.KB * kTileBytesFp8, xstep = 64 * a.K;
  // activation scales: waves 0-3 load one token's scale per lane
  const int srow = wave * 64 + lane;
  const int ssrc = (wave < 4 && m0 + srow < a.M) ? (m0 + srow) * a.KB * 4 : static_cast<int>(0x80000000u);

  // A block's loads come in 5 parts (weights 0-1, 2-3, activations 0-1, 2-3, scales), issued one per tile
  // rather than in one burst, which would stall the waves on a full memory queue.
  auto issue_part = [&](int st, int kb, int part) {
    uint8_t* base = smem + st * kStage;
    if (part < 2) {
#pragma unroll
      for (int i = 2 * part; i < 2 * part + 2; ++i)
        dma16(wr, base + (i * 8 + wave) * 1024, wsrc, kb * kTileBytesFp8 + i * wstep);
    } else if (part < 4) {
#pragma unroll
      for (int i = 2 * (part - 2); i < 2 * (part - 2) + 2; ++i)
        dma16(xr, base + kOpBytes + (i * 8 + wave) * 1024, xsrc, kb * kRowBytes + i * xstep);
    } else if (BLOCK && wave < 4) {
      dma4(sr, base + 2 * kOpBytes + wave * 256, ssrc, kb * 4);
    }
  };
  auto issue = [&](int st, int kb) {
#pragma unroll
    for (int part = 0; part < 5; ++part) issue_part(st, kb, part);
  };

  f32x4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const float* wsrow = BLOCK ? a.ws + static_cast<size_t>((n0 >> 7) + wn) * a.KB : nullptr;
  const bool wrows = n0 + wn * 128 < a.N;  // this wave's weight half exists

  // Fragment reads from an LDS stage: weight tile i (rows wn*128 + 16i + r) and token tile j (rows wm*64 + 16j
  // + r), 32 bytes at K 32t each.
  auto frag = [&](const uint8_t* op, int row) {
    const u32x4 lo = *reinterpret_cast<const u32x4*>(op + lds_off(row, 2 * t));
    const u32x4 hi = *reinterpret_cast<const u32x4*>(op + lds_off(row, 2 * t + 1));
    return i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
  };
  i32x8 bf[4], af;
  float sc[4];
  f32x4 pr[4];
  // B fragments, the lane's four block scales and the first A fragment of K block kb (stage st)
  auto block_start = [&](int st, int kb) {
    const uint8_t* sa = smem + st * kStage;
    const float* sxs = reinterpret_cast<const float*>(sa + 2 * kOpBytes);
    const float wsc = (BLOCK && wrows) ? wsrow[kb] : 0.f;
    af = frag(sa, wn * 128 + r);
#pragma unroll
    for (int j = 0; j < 4; ++j) bf[j] = frag(sa + kOpBytes, wm * 64 + 16 * j + r);
    if constexpr (BLOCK) {
#pragma unroll
      for (int j = 0; j < 4; ++j) sc[j] = sxs[wm * 64 + 16 * j + r] * wsc;
    }
  };
  auto fold = [&](f32x4 (&dst)[4], const f32x4 (&p)[4], const float (&s)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) dst[j][v] = __builtin_fmaf(p[j][v], s[j], dst[j][v]);
  };

  issue(0, kb0);
  LQ_WAIT_VM0();
  __builtin_amdgcn_s_barrier();
  block_start(0, kb0);
  // Per K block and weight tile: the tile's four MFMAs, then the next tile's fragment read, then the fold of
  // the four results into the accumulators (the other wave on the SIMD issues its MFMAs meanwhile). The one
  // barrier per block sits after tile 7's MFMAs are issued: it publishes the next block's loads and frees this
  // block's stage for its refill. Empty volatile statements pin this order (the compiler would otherwise sink
  // the MFMAs to their use, hoist the reads and defer the folds, and run out of registers).
  for (int kb = kb0; kb < kb1; ++kb) {
    const int st = (kb - kb0) & 1;
    const uint8_t* sa = smem + st * kStage;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i < 5 && kb + 1 < kb1) issue_part(st ^ 1, kb + 1, i);
      // the tile's MFMAs at raised issue priority: the SIMD's other wave gets the slots between them for its
      // folds and fragment reads (measured 1-2 % faster than equal priority)
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // E8M0 scale 127 = 1.0 on both operands: the plain FP8 x FP8 product of one 128-value block
        if constexpr (BLOCK)
          pr[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af, bf[j], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 127,
                                                                  0, 127);
        else
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af, bf[j], acc[i][j], 0, 0, 0, 127, 0, 127);
      }
      if constexpr (BLOCK)
        asm volatile("" ::"v"(pr[0]), "v"(pr[1]), "v"(pr[2]), "v"(pr[3]) : "memory");
      else
        asm volatile("" ::"v"(acc[i][0]), "v"(acc[i][1]), "v"(acc[i][2]), "v"(acc[i][3]) : "memory");
      __builtin_amdgcn_s_setprio(0);
      if (i < 7) {
        af = frag(sa, wn * 128 + 16 * (i + 1) + r);
      } else {
        // every wave's reads of this stage have returned and its loads of the next block have landed
        LQ_WAIT_LGKM0();
        LQ_WAIT_VM0();
        __builtin_amdgcn_s_barrier();
      }
      if constexpr (BLOCK) {
        asm volatile("" ::: "memory");
        fold(acc[i], pr, sc);
        asm volatile("" ::"v"(acc[i][0]), "v"(acc[i][1]), "v"(acc[i][2]), "v"(acc[i][3]));
      }
    }
    if (kb + 1 < kb1) block_start(st ^ 1, kb + 1);
  }

  if (part >= 0) {
    // A split tile: publish this part (agent-coherent stores: vector v = i * 4 + j of thread tid at
    // (v * kThreads + tid) * 16 bytes), count the arrival; the last part adds all parts in order.
    __shared__ int last_part;
    constexpr int kTileBytes = kBN * kBM * 4;
    const __amdgpu_buffer_rsrc_t pr_rs =
        __builtin_amdgcn_make_buffer_rsrc(a.part + static_cast<size_t>(rt) * a.S * (kBN * kBM), 0, a.S * kTileBytes,
                                          0x00020000);
    const int own = part * kTileBytes + static_cast<int>(threadIdx.x) * 16;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        __builtin_amdgcn_raw_buffer_store_b128(acc[i][j], pr_rs, own + (i * 4 + j) * kThreads * 16, 0, 16 /* sc1 */);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
      const int old = __hip_atomic_fetch_add(a.cnt + rt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last_part = old == a.S - 1;
      if (last_part) __hip_atomic_store(a.cnt + rt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last_part) return;
    // sum over parts 0 .. S-1 in order, one weight tile (4 vectors x S parts) per batch of loads; this
    // workgroup's own part is in its registers
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      f32x4 pv[kMaxSplit][4];
#pragma unroll
      for (int p = 0; p < kMaxSplit; ++p)
        if (p < a.S && p != part)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            pv[p][j] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           pr_rs, p * kTileBytes + static_cast<int>(threadIdx.x) * 16 + (i * 4 + j) * kThreads * 16,
                           0, 16 /* sc1 */));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f32x4 sum = part == 0 ? acc[i][j] : pv[0][j];
#pragma unroll
        for (int p = 1; p < kMaxSplit; ++p)
          if (p < a.S) sum = sum + (p == part ? acc[i][j] : pv[p][j]);
        acc[i][j] = sum;
      }
    }
  }

  // epilogue: lane holds rows n = n0 + wn*128 + 16i + 4t + v, token m = m0 + wm*64 + 16j + r
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int m = m0 + wm * 64 + 16 * j + r;
    if (m >= a.M) continue;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int n = n0 + wn * 128 + 16 * i + 4 * t;
      if (n >= a.N) continue;
      f32x4 v = acc[i][j];
      if constexpr (!BLOCK) v = f32x4{v[0] * a.alpha, v[1] * a.alpha, v[2] * a.alpha, v[3] * a.alpha};
      const size_t o = static_cast<size_t>(m) * a.ldy + n;
      if constexpr (OUT == kOutBf16) {
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.y) + o) =
            u32x2{f32_to_bf16(v[0]) | (uint32_t(f32_to_bf16(v[1])) << 16),
                  f32_to_bf16(v[2]) | (uint32_t(f32_to_bf16(v[3])) << 16)};
      } else {
        f32x4* dst = reinterpret_cast<f32x4*>(static_cast<float*>(a.y) + o);
        if constexpr (OUT == kOutF32Acc) {
          const f32x4 old = *dst;
          v = f32x4{old[0] + v[0], old[1] + v[1], old[2] + v[2], old[3] + v[3]};
        }
        *dst = v;
      }
    }
  }
}

// 1x128 FP8 activation quantizer: 16 lanes per (row, 128-value group), eight values (16 bytes) per lane, so a
// wave covers four groups with 16-byte loads and 8-byte stores; s = amax / 448 (1 for an all-zero group),
// q = E4M3(x * (1 / s)) rounded to nearest even, the product and the reciprocal each rounded to FP32 (the
// reference's activation quantizer multiplies by the reciprocal of its scale too, src/core/prefill_gemm.cu:496-511;
// eight divisions per lane made this kernel VALU-bound: 19.4 against 15.5 us at 4096 x 5120). |x / s| <= 448 up
// to that rounding; clamped, which is the saturating conversion.
__global__ void __launch_bounds__(256) quant_fp8_g128_kernel(const uint16_t* __restrict__ x, int M, int K,
                                                             uint8_t* __restrict__ q, float* __restrict__ scale) {
  // blockIdx.x: 16 groups of a row; blockIdx.y + k gridDim.y: the rows (no integer division per thread)
  const int KB = K / 128;
  const int kb = blockIdx.x * 16 + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  const bool ok = kb < KB;  // the 16 lanes of a group agree
  for (int m = blockIdx.y; m < M; m += gridDim.y) {
    const size_t base = static_cast<size_t>(m) * K + static_cast<size_t>(kb) * 128 + 8 * sub;
    u32x4 raw = u32x4{0u, 0u, 0u, 0u};
    if (ok) raw = *reinterpret_cast<const u32x4*>(x + base);
    float v[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = bf16_to_f32(raw[i] & 0xffff);
      v[2 * i + 1] = bf16_to_f32(raw[i] >> 16);
    }
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(v[i]));
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    const float s = mx > 0.f ? mx / 448.f : 1.f;
    const float rs = 1.f / s;
    uint32_t w[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float a[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = fminf(fmaxf(v[4 * h + i] * rs, -448.f), 448.f);
      const uint32_t lo = __builtin_amdgcn_cvt_pk_fp8_f32(a[0], a[1], 0, false);
      w[h] = __builtin_amdgcn_cvt_pk_fp8_f32(a[2], a[3], lo, true);
    }
    if (ok) {
      *reinterpret_cast<u32x2*>(q + base) = u32x2{w[0], w[1]};
      if (sub == 0) scale[static_cast<size_t>(m) * KB + kb] = s;
    }
  }
}

// Per-tensor FP8 activation quantizer (reference src/core/prefill_gemm.cu:496-511): each value rounded to BF16
// first (production's activations are BF16), times 1 / input_scale, then E4M3 with saturation to +-448 (NaN
// stays NaN). Four values per thread.
// BF16IN: x holds BF16 values (reference quant_act_fp8_bf16in, prefill_gemm.cu:626-630): the same bytes as from the
// FP32 values they were rounded from.
template <bool BF16IN>
__global__ void __launch_bounds__(256) quant_fp8_pt_kernel(const void* __restrict__ x, size_t quads, float inv_scale,
                                                           uint8_t* __restrict__ q) {
  for (size_t i = blockIdx.x * static_cast<size_t>(256) + threadIdx.x; i < quads; i += static_cast<size_t>(gridDim.x) * 256) {
    float f[4];
    if constexpr (BF16IN) {
      const u32x2 h = reinterpret_cast<const u32x2*>(x)[i];
      f[0] = __uint_as_float(h.x << 16);
      f[1] = __uint_as_float(h.x & 0xffff0000u);
      f[2] = __uint_as_float(h.y << 16);
      f[3] = __uint_as_float(h.y & 0xffff0000u);
    } else {
      const f32x4 v4 = reinterpret_cast<const f32x4*>(x)[i];
#pragma unroll
      for (int k = 0; k < 4; ++k) f[k] = bf16_to_f32(f32_to_bf16(v4[k]));
    }
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float b = f[k] * inv_scale;
      v[k] = isnan(b) ? b : fminf(fmaxf(b, -448.f), 448.f);
    }
    const uint32_t lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], 0, false);
    const uint32_t w = __builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], lo, true);
    reinterpret_cast<uint32_t*>(q)[i] = w;
  }
}

template <bool BLOCK, int OUT>
int prefill_launch(PrefillArgs a, const char* name, hipStream_t s) {
  const std::string nm(name);
  if (a.N <= 0 || a.K <= 0 || a.N % 128 != 0 || a.K % 128 != 0)
    return fail(LQ_ERR_SHAPE, "prefill_gemm: N % 128 and K % 128 must be 0");
  if (a.M < 1) return LQ_OK;  // nothing to do (the reference returns silently)
  if (a.ldy < a.N || a.ldy % 4 != 0) return fail(LQ_ERR_SHAPE, nm + ": ldy must be >= N and a multiple of 4");
  // operand byte offsets are 32-bit
  if (static_cast<long long>(a.N) * a.K >= (1LL << 31) || static_cast<long long>(a.M) * a.K >= (1LL << 31))
    return fail(LQ_ERR_SHAPE, nm + ": N * K and M * K must be below 2^31");
  if (!a.xq || !a.w || !a.y || (BLOCK && (!a.xs || !a.ws))) return fail(LQ_ERR_ARG, nm + ": null pointer");
  if (reinterpret_cast<uintptr_t>(a.y) % (OUT == kOutBf16 ? 8 : 16) != 0)
    return fail(LQ_ERR_ARG, nm + ": y must be 8-byte (BF16) or 16-byte (FP32) aligned");
  a.KB = a.K / 128;
  a.tiles_m = cdiv(a.M, kBM);
  a.tiles_n = cdiv(a.N, kBN);
  const long long tiles = static_cast<long long>(a.tiles_m) * a.tiles_n;
  // Tail split: when the tiles leave the last round of one-tile-per-CU workgroups at most a third full, the
  // tiles of that round are each split along K into S parts (S <= #CUs / rem, each part >= 8 K blocks, S <= 4).
  // Measured on config 4: down (64 of 256 CUs busy in the last round, S = 4) gains 8%; a half-full last round
  // (gate|up, S would be 2) loses 4% to the partial traffic, as the clock rises when CUs idle.
  int dev = 0;
  (void)hipGetDevice(&dev);
  const long long P = device_cus(dev);
  a.rem = static_cast<int>(tiles % P);
  a.S = a.rem ? static_cast<int>(std::min<long long>({P / a.rem, a.KB / 8, kMaxSplit})) : 1;
  if (a.S < 3) {
    a.S = 1;
    a.rem = 0;
  }
  a.full = static_cast<int>(tiles - a.rem);
  const long long blocks = a.full + (a.rem ? 8LL * cdiv(a.rem, 8) * a.S : 0);
  if (a.rem) {
    // rem * S <= P partial tiles: the bound is reserved once per device (lq_init, or here on first use) and never
    // reallocated, so a graph captured with these pointers stays valid whatever shapes run later
    Workspace* ws = workspace_for_current_device();
    if (!ws) return LQ_ERR_DEVICE;
    const int rc = reserve_prefill_scratch(ws);
    if (rc) return rc;
    a.part = ws->pf_partials;
    a.cnt = ws->pf_counters;
  }
  // 130 KB of dynamic LDS is above the default per-launch limit; raise it (once per instantiation).
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_fp8_kernel<BLOCK, OUT>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, 2 * kStage);
  if (attr != hipSuccess) return fail(LQ_ERR_LAUNCH, nm + ": " + hipGetErrorString(attr));
  hipLaunchKernelGGL((prefill_fp8_kernel<BLOCK, OUT>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 2 * kStage,
                     s, a);
  return check_launch(name);
}

}  // namespace

int reserve_prefill_scratch(Workspace* ws) {
  int dev = 0;
  (void)hipGetDevice(&dev);
  const size_t P = static_cast<size_t>(device_cus(dev));
  return ws->reserve_prefill(P * kBN * kBM * sizeof(float), P);
}

}  // namespace lq

using namespace lq;

extern "C" {

int lq_quant_act_fp8_g128(const uint16_t* x, int M, int K, uint8_t* q, float* scale, void* stream) {
  if (M < 1 || K <= 0 || K % 128 != 0) return fail(LQ_ERR_SHAPE, "quant_act_fp8_g128: M >= 1 and K % 128 == 0");
  if (!x || !q || !scale) return fail(LQ_ERR_ARG, "quant_act_fp8_g128: null pointer");
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(q) % 8 != 0)
    return fail(LQ_ERR_ARG, "quant_act_fp8_g128: x must be 16-byte and q 8-byte aligned");
  const unsigned rows = static_cast<unsigned>(std::min(M, 65535));
  hipLaunchKernelGGL(quant_fp8_g128_kernel, dim3(static_cast<unsigned>((K / 128 + 15) / 16), rows), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, M, K, q, scale);
  return check_launch("quant_act_fp8_g128");
}

int lq_prefill_fp8_block(const uint8_t* xq, const float* xs, int M, const uint8_t* w, const float* ws, uint16_t* y,
                         int ldy, int N, int K, void* stream) {
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
  return prefill_launch<true, kOutBf16>(a, "prefill_gemm", static_cast<hipStream_t>(stream));
}

int lq_quant_act_fp8(const float* x, int M, int K, float input_scale, uint8_t* q, void* stream) {
  if (M < 1 || K <= 0 || K % 4 != 0) return fail(LQ_ERR_SHAPE, "quant_act_fp8: M >= 1 and K % 4 == 0");
  if (!x || !q) return fail(LQ_ERR_ARG, "quant_act_fp8: null pointer");
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(q) % 4 != 0)
    return fail(LQ_ERR_ARG, "quant_act_fp8: x must be 16-byte and q 4-byte aligned");
  const size_t quads = static_cast<size_t>(M) * K / 4;
  const unsigned grid = static_cast<unsigned>(std::min<size_t>((quads + 255) / 256, 256 * 64));
  hipLaunchKernelGGL(quant_fp8_pt_kernel<false>, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream), x, quads,
                     1.f / input_scale, q);
  return check_launch("quant_act_fp8");
}

int lq_quant_act_fp8_bf16in(const uint16_t* x, int M, int K, float input_scale, uint8_t* q, void* stream) {
  if (M < 1 || K <= 0 || K % 4 != 0) return fail(LQ_ERR_SHAPE, "quant_act_fp8_bf16in: M >= 1 and K % 4 == 0");
  if (!x || !q) return fail(LQ_ERR_ARG, "quant_act_fp8_bf16in: null pointer");
  if (reinterpret_cast<uintptr_t>(x) % 8 != 0 || reinterpret_cast<uintptr_t>(q) % 4 != 0)
    return fail(LQ_ERR_ARG, "quant_act_fp8_bf16in: x must be 8-byte and q 4-byte aligned");
  const size_t quads = static_cast<size_t>(M) * K / 4;
  const unsigned grid = static_cast<unsigned>(std::min<size_t>((quads + 255) / 256, 256 * 64));
  hipLaunchKernelGGL(quant_fp8_pt_kernel<true>, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream), x, quads,
                     1.f / input_scale, q);
  return check_launch("quant_act_fp8_bf16in");
}

int lq_prefill_gemm_fp8(const uint8_t* xq, int M, const uint8_t* w, float alpha, float* y, int ldy, int N, int K,
                        int accumulate, void* stream) {
  PrefillArgs a{};
  a.xq = xq;
  a.w = w;
  a.alpha = alpha;
  a.y = y;
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  return accumulate ? prefill_launch<false, kOutF32Acc>(a, "prefill_gemm_fp8", s)
                    : prefill_launch<false, kOutF32>(a, "prefill_gemm_fp8", s);
}

int lq_prefill_gemm_fp8_bf16out(const uint8_t* xq, int M, const uint8_t* w, float alpha, uint16_t* y, int ldy, int N,
                                int K, void* stream) {
  PrefillArgs a{};
  a.xq = xq;
  a.w = w;
  a.alpha = alpha;
  a.y = y;
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  return prefill_launch<false, kOutBf16>(a, "prefill_gemm_fp8_bf16out", static_cast<hipStream_t>(stream));
}

}  // extern "C"
