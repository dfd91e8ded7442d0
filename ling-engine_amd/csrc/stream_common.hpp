// Device helpers shared by the skinny (stream) GEMM kernels: launch arguments, weight loads from the tiled
// layout into registers, exact dequantization into MFMA operands, the epilogues, the stream-K unit arithmetic and
// the split-K partial exchange.
#pragma once

#include "lq_common.hpp"
#include "lq_div.hpp"
#include "lq_workspace.hpp"

#include <cstddef>
#include <type_traits>
#include <utility>

namespace lq {

constexpr int kWaves = 4;  // waves per workgroup, one per tile slot of the tile group
constexpr int kThreads = kWaves * kWave;
constexpr int kMaxMats = 4;

enum WFmt { kFp8 = 0, kFp4 = 1, kFp4Coded = 2 };

// 16-row tiles per wave (T): one gate and one up tile with the SiLU*mul epilogue; two FP8 tiles; four NVFP4 tiles
// (half the bytes per tile and chunk). Enough weight bytes per load stage keep the HBM stream deep, and every
// activation operand read from LDS feeds T MFMAs. One FP8 tile per wave instead where each workgroup's range is
// short (choose_tiles): there the split-K finish, whose fan-in halves with T, outweighs the stream's depth.
// Chosen by N, K and the CU count only, never by M (row invariance).
__host__ __device__ constexpr int tiles_per_wave(int wf, bool pair) { return pair ? 2 : wf == kFp8 ? 2 : 4; }
// Output rows (columns of y) per tile group: the workgroup's 4 waves' tiles (gate rows only for a pair).
__host__ __device__ constexpr int group_rows(int T, bool pair) { return 16 * 4 * (pair ? T / 2 : T); }

// Weight chunks in flight per wave (the computed one included). Shallow on purpose: with every CU streaming, more
// stages add no bandwidth but lengthen the prologue (all of them are issued before the first chunk is computed) and
// the registers they hold. Measured against the earlier register-budget depths (12/10/8/6 at one tile, 8/6/4 at two,
// 6/4/3/2 at four): verify step at M = 17 56.2 -> 53.7 us, the NVFP4 fc 8-12 % faster, FP8 launches under 10 us
// 15-20 % faster, no shape slower; two stages at two tiles from G = 3 (the operand prefetch of G <= 2 needs three)
// another 1-3 % at M = 33..68.
template <int T>
__host__ __device__ constexpr int pf_stages(int G) {
  return T == 1   ? (G <= 1 ? 5 : 4)
         : T == 2 ? (G <= 2 ? 3 : 2)
                  : (G <= 3 ? 3 : 2);
}

struct StreamArgs {
  const void* x;      // [M][K] BF16 or FP16
  const float* xinv;  // [M] row scales of an FP16 copy, or null
  int M, K, C;        // C = K / 128
  int P;              // logical workgroups (all segments)
  int TG;             // tile groups (all segments)
  short T;            // tiles per wave (the kernel's template argument)
  short NR;           // finish workgroups per split tile group (0: the last workgroup to arrive finishes it)
  short count;        // matrices
  short wait_ms;      // finish workgroups: how long to wait for the arrivals before giving up (milliseconds)
  short cs;           // counter stride in ints: 32 puts each counter on a 128-byte line of its own
  const uint8_t* w[kMaxMats];
  const uint8_t* table[kMaxMats];   // coded NVFP4: device scale-code table [64]
  const float* svec[kMaxMats];      // per-channel scales [N] or null
  float sc[kMaxMats];               // scalar scale (used when svec is null)
  void* y[kMaxMats];                // BF16 or FP32 [M][ldy]
  const uint16_t* resid[kMaxMats];  // BF16 residual [M][ldy] or null
  int N[kMaxMats];
  int tg0[kMaxMats + 1];  // first tile group of each matrix; tg0[count] = TG
  // Segments: each matrix of a launch that is not a SiLU*mul pair (a pair is one segment) has its tile groups
  // [tg0[i], tg0[i + 1]) split over its own workgroups [wg0[i], wg0[i + 1]), exactly as a launch of that matrix
  // alone splits them, so a matrix's results do not depend on the matrices beside it. Units (tile group, chunk) of
  // a segment: U = (tg0[i + 1] - tg0[i]) C, with U (P + 1) < 2^31 (the unit arithmetic is 32-bit).
  int wg0[kMaxMats + 1];
  int ldy[kMaxMats];
  float* partials;  // [2 * P][T * G * 4][256] per workgroup slot
  int* counters;    // [TG] (TG + tg: finish workgroups' own), counter i at counters[i * cs]
  unsigned long long* trace;  // [P][16] s_memrealtime stamps per workgroup (LQ_STREAM_TRACE builds), or null
};

// The kernel touches one field per 64-byte line of its arguments at entry (see stream_kernel).
static_assert(sizeof(StreamArgs) <= 320 && offsetof(StreamArgs, trace) < 320 && offsetof(StreamArgs, x) / 64 == 0 &&
                  (offsetof(StreamArgs, w) + 2 * sizeof(void*)) / 64 == 1 &&
                  (offsetof(StreamArgs, svec) + 2 * sizeof(void*)) / 64 == 2 && offsetof(StreamArgs, resid) / 64 == 3 &&
                  (offsetof(StreamArgs, tg0) + 4 * sizeof(int)) / 64 == 4,
              "argument lines touched at kernel entry");

// arr[mi] of an argument array, read as constant-offset argument loads and a select: no argument read waits on
// mi (or on another argument read), so the reads of a prologue or an epilogue batch into one scalar round trip
// instead of a chain of dependent ones.
template <int N, class X>
__device__ __forceinline__ X pick(const X (&arr)[N], int mi) {
  X v = arr[0];
#pragma unroll
  for (int k = 1; k < N; ++k) v = mi == k ? arr[k] : v;
  return v;
}

// Phase stamps of a workgroup for builds with LQ_STREAM_TRACE: kept in registers, written once at exit.
// 0 entry, 1 first chunk computed, 2 stream done, 3 partials published, 4 arrival counted, 5 reduced, 6 exit,
// 7 prologue loads issued, 8 first partial added, 9 reduction loop done, 10 arguments read, 11 tiles set up,
// 12 / 13 first / last epilogue inputs issued, 14 first ring stage issued, 15 activations ready.
#ifdef LQ_STREAM_TRACE
#define LQ_TS(i) (ts[i] = __builtin_amdgcn_s_memrealtime())
#else
#define LQ_TS(i) ((void)0)
#endif

// One chunk of weights for the lane: FP8 32 bytes (two pieces) per tile; NVFP4 16 bytes + 2 scales.
template <int WF, int T>
struct WRegs {
  u32x4 v[T][WF == kFp8 ? 2 : 1];
  uint32_t sc[T];  // NVFP4: the two E4M3 block scales (raw) or the 12-bit code pair (coded)
};

// Buffer resources: a raw (stride 0) descriptor per matrix; lane offsets in one VGPR, the tile/chunk offset
// in an SGPR, so the ring of in-flight loads costs no address registers.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, 0x00020000);
}
constexpr int kNT = 2;  // slc: streaming (non-temporal) weights

template <int WF, int T>
__device__ __forceinline__ void load_w(WRegs<WF, T>& R, const __amdgpu_buffer_rsrc_t (&rs)[T], const int (&toff)[T],
                                       const int (&coff)[T], int c, int lane_off, int slot, unsigned oob) {
#pragma unroll
  for (int i = 0; i < T; ++i) {
    if constexpr (WF == kFp8) {
      const int so = toff[i] + c * kTileBytesFp8;
      R.v[i][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs[i], lane_off, so, kNT));
      R.v[i][1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs[i], lane_off + 512, so, kNT));
    } else if constexpr (WF == kFp4) {
      const int so = toff[i] + c * kTileBytesFp4;
      R.v[i][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs[i], lane_off, so, kNT));
      R.sc[i] = static_cast<uint16_t>(
          __builtin_amdgcn_raw_buffer_load_b16(rs[i], static_cast<int>((1024 + 2 * slot) | oob), so, 0));
    } else {
      const int so = toff[i] + c * kValueBytesFp4;
      R.v[i][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs[i], lane_off, so, kNT));
      // slot s < 32: low byte at 2s, high nibble in the low half of byte 64 + s; slot 32 + L: byte 2L + 1
      // and the high half of byte 64 + L (reference src/core/stream_gemm.cu:740-780).
      const int L = slot & 31, hi = slot >> 5, cso = coff[i] + c * kCodeBytesFp4;
      const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b8(rs[i], static_cast<int>((2 * L + hi) | oob), cso, 0);
      const uint32_t nb = __builtin_amdgcn_raw_buffer_load_b8(rs[i], static_cast<int>((64 + L) | oob), cso, 0);
      R.sc[i] = lo | (((nb >> (4 * hi)) & 15u) << 8);
    }
  }
}

// The A operand of MFMA step s (8 weights, K 32t + 8s .. +8) for tile i.
template <int WF, bool F16, int T>
__device__ __forceinline__ u32x4 a_operand(const WRegs<WF, T>& R, int i, int s, const uint8_t* tab) {
  if constexpr (WF == kFp8) {
    const u32x4& v = R.v[i][s >> 1];
    const uint32_t d0 = (s & 1) ? v.z : v.x, d1 = (s & 1) ? v.w : v.y;
    const u32x2 a = F16 ? fp8x4_to_f16x4(d0) : fp8x4_to_bf16x4(d0);
    const u32x2 b = F16 ? fp8x4_to_f16x4(d1) : fp8x4_to_bf16x4(d1);
    return u32x4{a.x, a.y, b.x, b.y};
  } else {
    // the two block scales (K [32t, +16) and [32t + 16, +32)); steps 0, 1 use the first
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

// LDS image of one chunk of activations: row m's 16 units of 16 bytes (8 values), unit u at (u ^ (m & 15)).
__device__ __forceinline__ int xs_off(int row, int unit) { return row * 256 + ((unit ^ (row & 15)) << 4); }

// One accumulator chain per output tile and row group: a step's T x G MFMAs (T >= 2) are independent of each
// other, which covers the MFMA result latency.
template <int WF, bool F16, int G, int T>
__device__ __forceinline__ void mfma_step(const WRegs<WF, T>& R, int s, const u32x4 (&b)[G], f32x4 (&acc)[T][G],
                                          const uint8_t* const (&tab)[T]) {
#pragma unroll
  for (int i = 0; i < T; ++i) {
    const u32x4 a = a_operand<WF, F16, T>(R, i, s, tab[i]);
#pragma unroll
    for (int g = 0; g < G; ++g) acc[i][g] = mfma16x16x32(a, b[g], acc[i][g], F16);
  }
}

template <int G>
__device__ __forceinline__ void read_b(u32x4 (&b)[G], const uint8_t* xs, int s, int r, int t) {
#pragma unroll
  for (int g = 0; g < G; ++g) b[g] = *reinterpret_cast<const u32x4*>(xs + xs_off(16 * g + r, 4 * t + s));
}

// One chunk with the activation operands read from LDS inside (the next step's while the current computes).
template <int WF, bool F16, int G, int T>
__device__ __forceinline__ void compute_lds(const WRegs<WF, T>& R, const uint8_t* xs, f32x4 (&acc)[T][G], int r,
                                            int t, const uint8_t* const (&tab)[T]) {
  u32x4 b[2][G];
  read_b<G>(b[0], xs, 0, r, t);
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if (s < 3) read_b<G>(b[(s + 1) & 1], xs, s + 1, r, t);
    mfma_step<WF, F16, G, T>(R, s, b[s & 1], acc, tab);
  }
}

// SiLU v / (1 + e^-v), with the hardware reciprocal (1 ulp) in place of the division.
__device__ __forceinline__ float silu(float v) { return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }

// What the epilogue reads besides the sums, for one lane: the output scales of its 4 channels per tile
// (per-channel vector, or the matrix's scalar), the residual's 4 values per tile and token group, and the
// row scales. Loaded in one batch of vector loads (for the range's first and last tile groups at kernel
// start), so finishing a tile group waits on no memory read.
template <int G, int T>
struct EpiIn {
  f32x4 sv[T];
  u32x2 rr[T][G];
  float xi[G];
};

// Tile i's first output row for this lane: PAIR = gate tiles then the same up tiles.
template <bool PAIR, int T>
__device__ __forceinline__ int epi_row(int wtile0, int i, int t) {
  return (wtile0 + (PAIR ? i % (T / 2) : i)) * 16 + 4 * t;
}

template <int G, bool PAIR, bool OUTF32, int T>
__device__ __forceinline__ void epi_load(const StreamArgs& a, int mi, int wtile0, EpiIn<G, T>& e, int r, int t) {
#pragma unroll
  for (int i = 0; i < T; ++i) {
    const int m = PAIR ? (i < T / 2 ? 0 : 1) : mi;
    const int n = epi_row<PAIR, T>(wtile0, i, t);
    const float sc = pick(a.sc, m);
    const float* const svec = pick(a.svec, m);
    const uint16_t* const resid = pick(a.resid, m);
    const int Nm = pick(a.N, m), ldy = pick(a.ldy, m);
    e.sv[i] = f32x4{sc, sc, sc, sc};
    if (svec && n < Nm) e.sv[i] = *reinterpret_cast<const f32x4*>(svec + n);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int tok = 16 * g + r;
      e.rr[i][g] = u32x2{0u, 0u};
      if constexpr (!PAIR && !OUTF32) {
        if (resid && tok < a.M && n < Nm)
          e.rr[i][g] = *reinterpret_cast<const u32x2*>(resid + static_cast<size_t>(tok) * ldy + n);
      }
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int tok = 16 * g + r;
    e.xi[g] = (a.xinv && tok < a.M) ? a.xinv[tok] : 1.0f;
  }
}

// Epilogue of one lane's outputs: acc[i][g][v] is row 16 * tile(i) + 4t + v, token 16g + r. COH: the stores
// write through to memory (agent-coherent), for a consumer on another CU within the same launch.
template <int G, bool PAIR, bool OUTF32, int T, bool COH = false>
__device__ __forceinline__ void epilogue(const StreamArgs& a, int mi, int wtile0, const f32x4 (&acc)[T][G],
                                         const EpiIn<G, T>& e, int r, int t) {
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int tok = 16 * g + r;
    if (tok >= a.M) continue;
    if constexpr (PAIR) {
#pragma unroll
      for (int i = 0; i < T / 2; ++i) {
        const int n = epi_row<PAIR, T>(wtile0, i, t);
        if (n >= a.N[0]) continue;
        uint16_t o[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float gs = acc[i][g][v] * e.sv[i][v];
          const float us = acc[i + T / 2][g][v] * e.sv[i + T / 2][v];
          o[v] = f32_to_bf16(silu(gs) * us);
        }
        uint16_t* dst = reinterpret_cast<uint16_t*>(a.y[0]) + static_cast<size_t>(tok) * a.ldy[0] + n;
        const u32x2 pk{o[0] | (uint32_t(o[1]) << 16), o[2] | (uint32_t(o[3]) << 16)};
        if constexpr (COH)
          __hip_atomic_store(reinterpret_cast<uint64_t*>(dst), __builtin_bit_cast(uint64_t, pk), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        else
          *reinterpret_cast<u32x2*>(dst) = pk;
      }
    } else {
      const int Nm = pick(a.N, mi), ldy = pick(a.ldy, mi);
      void* const y = pick(a.y, mi);
      const uint16_t* const resid = pick(a.resid, mi);
#pragma unroll
      for (int i = 0; i < T; ++i) {
        const int n = epi_row<PAIR, T>(wtile0, i, t);
        if (n >= Nm) continue;
        float vv[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          vv[v] = acc[i][g][v] * e.sv[i][v];
          if (a.xinv) vv[v] = vv[v] * e.xi[g];
        }
        const size_t o = static_cast<size_t>(tok) * ldy + n;
        if constexpr (OUTF32) {
          *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(y) + o) = f32x4{vv[0], vv[1], vv[2], vv[3]};
        } else {
          if (resid) {
            const u32x2 rr = e.rr[i][g];
            vv[0] = vv[0] + bf16_to_f32(rr.x & 0xffff);
            vv[1] = vv[1] + bf16_to_f32(rr.x >> 16);
            vv[2] = vv[2] + bf16_to_f32(rr.y & 0xffff);
            vv[3] = vv[3] + bf16_to_f32(rr.y >> 16);
          }
          *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(y) + o) =
              u32x2{f32_to_bf16(vv[0]) | (uint32_t(f32_to_bf16(vv[1])) << 16),
                    f32_to_bf16(vv[2]) | (uint32_t(f32_to_bf16(vv[3])) << 16)};
        }
      }
    }
  }
}

// Workgroup p's units are [unit_start(p), unit_start(p + 1)); wg_of_unit is the workgroup of unit u.
__device__ __forceinline__ int wg_of_unit(int u, int P, int U) { return ((u + 1) * P - 1) / U; }
__device__ __forceinline__ int unit_start(int p, int P, int U) { return p * U / P; }

// A segment's first tile group and workgroup, its workgroups P and its units U (see StreamArgs::wg0).
struct SegSplit {
  int tgb, wgb, P, U;
};
// ONESEG: the launch is one segment (a SiLU*mul pair, or a single matrix): segment 0, tile groups [0, TG), workgroups
// [0, P); no argument array is then indexed by a run-time segment (such an index makes the compiler chain dependent
// argument reads at kernel entry).
template <bool ONESEG>
__device__ __forceinline__ SegSplit seg_split(const StreamArgs& a, int i) {
  SegSplit s;
  s.tgb = ONESEG ? 0 : pick(a.tg0, i);
  const int tge = ONESEG ? a.TG : pick(a.tg0, i + 1);
  s.wgb = pick(a.wg0, i);
  s.P = pick(a.wg0, i + 1) - s.wgb;
  s.U = (tge - s.tgb) * a.C;
  return s;
}
// The segment holding workgroup b (raw or logical: the permutation stays inside a segment), or tile group tg.
template <bool ONESEG>
__device__ __forceinline__ int seg_of_wg(const StreamArgs& a, int b) {
  int i = 0;
  if constexpr (!ONESEG) {
#pragma unroll
    for (int k = 1; k < kMaxMats; ++k) i += (k < a.count && b >= a.wg0[k]) ? 1 : 0;
  }
  return i;
}
template <bool ONESEG>
__device__ __forceinline__ int seg_of_tg(const StreamArgs& a, int tg) {
  int i = 0;
  if constexpr (!ONESEG) {
#pragma unroll
    for (int k = 1; k < kMaxMats; ++k) i += (k < a.count && tg >= a.tg0[k]) ? 1 : 0;
  }
  return i;
}

// Tiles of tile group tg that this wave streams: PAIR = gate tile wtile0 then the same up tile; else tiles
// wtile0 .. of matrix mi.
template <int WF, int T, bool PAIR>
struct SegTiles {
  int mi, wtile0;
  __amdgpu_buffer_rsrc_t rs[T];
  int toff[T], coff[T];
};

template <int WF, int T, bool PAIR, bool ONE = false>
__device__ __forceinline__ void seg_tiles(const StreamArgs& a, int tg, int wave, SegTiles<WF, T, PAIR>& s) {
  // the matrix of tile group tg: the last mi < count with tg0[mi] <= tg (tg0 is increasing), counted without a
  // loop whose argument reads would wait on each other
  int mi = 0;
  if constexpr (!PAIR && !ONE) {
#pragma unroll
    for (int k = 1; k < kMaxMats; ++k) mi += (k < a.count && tg >= a.tg0[k]) ? 1 : 0;
  }
  s.mi = mi;
  s.wtile0 = (tg - pick(a.tg0, mi)) * (group_rows(T, PAIR) / 16) + wave * (PAIR ? T / 2 : T);
#pragma unroll
  for (int i = 0; i < T; ++i) {
    const int m = PAIR ? (i < T / 2 ? 0 : 1) : mi;
    const int Nm = pick(a.N, m);
    const int tile = min((PAIR ? s.wtile0 + (i % (T / 2)) : s.wtile0 + i), Nm / 16 - 1);
    const int blk = WF == kFp8 ? kTileBytesFp8 : WF == kFp4 ? kTileBytesFp4 : kValueBytesFp4;
    s.rs[i] = make_rsrc(pick(a.w, m));
    s.toff[i] = tile * a.C * blk;
    s.coff[i] = (Nm / 16) * a.C * kValueBytesFp4 + tile * a.C * kCodeBytesFp4;
  }
}

// Partial sums of a split tile group: workgroup q's slot w (0: its range's first tile group, 1: its last)
// holds thread tid's T x G accumulator vectors at [j = i * G + g][tid], 16 bytes each. They are written and
// read with agent-coherent (sc1) buffer accesses: stores write through past the XCD's L2 and loads do not
// hit a stale L2 line, so the exchange needs no cache-wide writeback or invalidate.
constexpr int kSc1 = 16;  // cache-policy operand: SC1

template <int G, int T>
__device__ __forceinline__ int slot_off(int q, int which) {
  return (2 * q + which) * (T * G * 16 * kThreads) + static_cast<int>(threadIdx.x) * 16;
}

// Where the partials of tile group tg are: workgroups pf .. pl touch it; a workgroup's partial of tg is in
// its slot 0 when tg is its range's first tile group (every workgroup after pf starts inside tg; pf itself
// only when its range starts exactly at tg's first chunk), else in slot 1.
struct SplitInfo {
  int pf, pl;
  bool pf_first;
};
template <bool ONESEG>
__device__ __forceinline__ SplitInfo split_info(const StreamArgs& a, int tg) {
  const SegSplit g = seg_split<ONESEG>(a, seg_of_tg<ONESEG>(a, tg));
  const int u = (tg - g.tgb) * a.C;
  SplitInfo s;
  s.pf = g.wgb + wg_of_unit(u, g.P, g.U);
  s.pl = g.wgb + wg_of_unit(u + a.C - 1, g.P, g.U);
  s.pf_first = unit_start(s.pf - g.wgb, g.P, g.U) == u;
  return s;
}

// The finishing step of split tile groups: the last workgroup to arrive adds every workgroup's partial in
// workgroup order. Every workgroup (the finisher included) published its partial before arriving, so all of
// them are read back from memory, D partials of each group per batch: a batch's loads (of both groups, when
// this workgroup finishes its first and its last tile group) are all issued before its adds, so a fan-in of up
// to D costs one memory round trip. D is 16 (8 per group when finishing two) for four accumulator vectors at
// one or two tiles per wave: the FP8 kernels' fan-in of up to 8 then takes one round trip. At four NVFP4 tiles
// per wave the deeper batch measured slower, so it stays at 8.
template <int G, int T, int NG>
__device__ __forceinline__ void reduce_partials(const StreamArgs& a, const SplitInfo* si, f32x4 (*acc[NG])[G], int r,
                                                unsigned long long (&ts)[16]) {
  constexpr int NV = T * G;  // accumulator vectors per thread
  constexpr int D0 = NV <= 4 ? (T <= 2 ? 16 : 8) : NV <= 8 ? 4 : NV <= 10 ? 3 : NV <= 16 ? 2 : 1;
  constexpr int D = NG == 2 ? (D0 + 1) / 2 : D0;
  const __amdgpu_buffer_rsrc_t prs = make_rsrc(a.partials);
  int n[NG];
  int nmax = 0;
#pragma unroll
  for (int h = 0; h < NG; ++h) {
    n[h] = si[h].pl - si[h].pf + 1;
    nmax = max(nmax, n[h]);
  }
  // rows past M read nothing (an out-of-range offset returns zeros): they only reach outputs never stored
  unsigned rowmask[G];
#pragma unroll
  for (int g = 0; g < G; ++g) rowmask[g] = 16 * g + r < a.M ? 0u : 0x80000000u;
  f32x4 ring[NG][D][NV];
  // Only positions that exist are loaded (out-of-range buffer loads are not free: a burst of them delays the
  // wanted ones).
  auto issue = [&](int h, int k, int b) {
    if (k >= n[h]) return;
    const int off = slot_off<G, T>(si[h].pf + k, (k > 0 || si[h].pf_first) ? 0 : 1);
#pragma unroll
    for (int i = 0; i < T; ++i)
#pragma unroll
      for (int g = 0; g < G; ++g)
        ring[h][b][i * G + g] = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       prs, static_cast<int>((off + (i * G + g) * 16 * kThreads) | rowmask[g]), 0, kSc1));
  };
  for (int q0 = 0; q0 < nmax; q0 += D) {
#pragma unroll
    for (int h = 0; h < NG; ++h)
#pragma unroll
      for (int b = 0; b < D; ++b) issue(h, q0 + b, b);
#pragma unroll
    for (int h = 0; h < NG; ++h)
#pragma unroll
      for (int b = 0; b < D; ++b) {
        const int k = q0 + b;
        if (k < n[h]) {
#pragma unroll
          for (int i = 0; i < T; ++i)
#pragma unroll
            for (int g = 0; g < G; ++g)
              acc[h][i][g] = k == 0 ? ring[h][b][i * G + g] : acc[h][i][g] + ring[h][b][i * G + g];
          if (k == 0) LQ_TS(8);
        }
      }
  }
}

template <int G, int T>
__device__ __forceinline__ void publish_partial(const StreamArgs& a, int p, int which, const f32x4 (&acc)[T][G],
                                                int r) {
  const __amdgpu_buffer_rsrc_t prs = make_rsrc(a.partials);
  const int off = slot_off<G, T>(p, which);
#pragma unroll
  for (int i = 0; i < T; ++i)
#pragma unroll
    for (int g = 0; g < G; ++g)
      if (16 * g + r < a.M)
        __builtin_amdgcn_raw_buffer_store_b128(acc[i][g], prs, off + (i * G + g) * 16 * kThreads, 0, kSc1);
}

// Finish workgroups (StreamArgs::NR > 0, for launches whose tile groups each span several workgroups): launch
// workgroup P + f finishes share f % NR of split tile group f / NR, the accumulator vectors that streaming wave
// f % NR holds (NR = 4). The streaming workgroups publish their partials as in the last-arriver form, count
// themselves on counters[tg] (an atomic whose result nobody waits for) and exit; each finish workgroup waits
// for the full count, adds its share's partials in workgroup order and runs the epilogue on it, element for
// element the last-arriver form's arithmetic. Four workgroups on four CUs read what one finisher read, and no
// streaming workgroup spends its tail finishing two tile groups in a row. When all NR finish workgroups of tg
// have seen the full count (counters[TG + tg] counts them), the last one clears both counters for the next
// launch. A finish workgroup never holds up a streaming one: the dispatcher places workgroups in index order, so
// every streaming workgroup has its CU before any finish workgroup starts waiting. The wait gives up after a
// second (StreamArgs::wait_ms, on s_memrealtime at 100 MHz), which a launch whose streaming workgroups run never
// reaches; if it does
// (the GPU preempted for that long), the workgroup records it in g_wait_expired (reported and cleared by
// lq_stream_ffn_deadline_status) and finishes anyway; the arrival counter is then brought back by subtracting the
// expected count, so late arrivals leave it at zero for later launches.
constexpr int kFinishShares = 4;
__device__ int g_wait_expired = 0;  // per device: a bounded in-kernel wait gave up (results not valid)

template <int G, int T, bool PAIR, bool OUTF32, bool ONE = false>
__device__ __forceinline__ void finish_share(const StreamArgs& a, int f) {
  const int tg = f / kFinishShares, share = f % kFinishShares;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  unsigned long long ts[16] = {};
  LQ_TS(0);
#ifdef LQ_STREAM_TRACE
  struct Flush {
    const StreamArgs& a;
    int f;
    unsigned long long (&ts)[16];
    __device__ ~Flush() {
      LQ_TS(6);
      if (a.trace && threadIdx.x == 0)
        for (int k = 0; k < 16; ++k) a.trace[(a.P + f) * 16 + k] = ts[k];
    }
  } flush{a, f, ts};
#else
  (void)ts;
#endif
  const int r = lane & 15, t = lane >> 4;
  if (tg >= a.TG) return;
  const SplitInfo si = split_info<PAIR || ONE>(a, tg);
  if (si.pf == si.pl) return;  // streamed whole by one workgroup, which finished it
  const int n = si.pl - si.pf + 1;
  const int mi = seg_of_tg<PAIR || ONE>(a, tg);
  const int wtile0 = (tg - pick(a.tg0, mi)) * (group_rows(T, PAIR) / 16) + share * (PAIR ? T / 2 : T);
  // units of the share: (tile, group) vectors, a SiLU*mul pair's gate and up vector together; wave w takes
  // units w, w + 4, ...
  constexpr int NU = (PAIR ? T / 2 : T) * G;
  constexpr int UW = (NU + 3) / 4;
  constexpr int SLOT = T * G * 16 * kThreads;  // bytes of one workgroup slot
  const int vtid = share * 64 + lane;          // the streaming thread whose vectors these are
  const int Nm = PAIR ? a.N[0] : pick(a.N, mi);
  const float* const svec = PAIR ? nullptr : pick(a.svec, mi);
  const uint16_t* const resid = PAIR ? nullptr : pick(a.resid, mi);
  const int ldy = PAIR ? a.ldy[0] : pick(a.ldy, mi);

  // epilogue inputs first (they do not depend on the partials)
  f32x4 sv[UW][2];
  u32x2 rr[UW];
  float xi[UW];
#pragma unroll
  for (int k = 0; k < UW; ++k) {
    const int u = wave + 4 * k;
    const int i = u / G, g = u % G, tok = 16 * g + r;
    const int col = (wtile0 + i) * 16 + 4 * t;
    rr[k] = u32x2{0u, 0u};
    xi[k] = 1.0f;
    if constexpr (PAIR) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float sc = a.sc[h];
        sv[k][h] = f32x4{sc, sc, sc, sc};
        if (u < NU && a.svec[h] && col < Nm) sv[k][h] = *reinterpret_cast<const f32x4*>(a.svec[h] + col);
      }
    } else {
      const float sc = pick(a.sc, mi);
      sv[k][0] = f32x4{sc, sc, sc, sc};
      if (u < NU && svec && col < Nm) sv[k][0] = *reinterpret_cast<const f32x4*>(svec + col);
      if constexpr (!OUTF32)
        if (u < NU && resid && tok < a.M && col < Nm)
          rr[k] = *reinterpret_cast<const u32x2*>(resid + static_cast<size_t>(tok) * ldy + col);
      if (u < NU && a.xinv && tok < a.M) xi[k] = a.xinv[tok];
    }
  }

  // every streaming workgroup of tg has published and counted itself (one wave polls, about every half
  // microsecond: the polls of all finish workgroups land on a few cache lines)
  if (wave == 0 && a.wait_ms == 0) {
    // zero limit (a test hook): give up at once, so the expired-wait path below is taken on every launch
    __hip_atomic_store(&g_wait_expired, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else if (wave == 0) {
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    while (__builtin_amdgcn_readfirstlane(__hip_atomic_load(a.counters + tg * a.cs, __ATOMIC_RELAXED,
                                                             __HIP_MEMORY_SCOPE_AGENT)) < n) {
      if (__builtin_amdgcn_s_memrealtime() - t0 > static_cast<unsigned long long>(a.wait_ms) * 100'000ull) {
        __hip_atomic_store(&g_wait_expired, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(16);
    }
  }
  __syncthreads();
  LQ_TS(1);
  if (threadIdx.x == 0) {
    const int old = __hip_atomic_fetch_add(a.counters + (a.TG + tg) * a.cs, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == kFinishShares - 1) {
      // minus the n arrivals rather than a store of zero: after an expired wait, arrivals still to come bring the
      // counter back to exactly zero instead of leaving a count for the next launch
      __hip_atomic_fetch_add(a.counters + tg * a.cs, -n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.counters + (a.TG + tg) * a.cs, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  const __amdgpu_buffer_rsrc_t prs = make_rsrc(a.partials);
  constexpr int NH = PAIR ? 2 : 1;
  constexpr int B = 8;  // partials per batch of loads
#pragma unroll
  for (int k = 0; k < UW; ++k) {
    const int u = wave + 4 * k;
    if (u >= NU) break;  // (uniform over the wave)
    const int i = u / G, g = u % G, tok = 16 * g + r;
    const unsigned rowmask = tok < a.M ? 0u : 0x80000000u;
    f32x4 acc[NH];
    for (int q0 = 0; q0 < n; q0 += B) {
      f32x4 ring[B][NH];
#pragma unroll
      for (int b = 0; b < B; ++b) {
        const int q = si.pf + q0 + b;
        const int which = (q0 + b == 0 && !si.pf_first) ? 1 : 0;
        const unsigned oob = (q0 + b < n ? 0u : 0x80000000u) | rowmask;
#pragma unroll
        for (int h = 0; h < NH; ++h) {
          const int j = (i + h * (T / 2)) * G + g;
          ring[b][h] = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                         prs, static_cast<int>(((2 * q + which) * SLOT + vtid * 16 + j * 16 * kThreads) | oob), 0,
                         kSc1));
        }
      }
#pragma unroll
      for (int b = 0; b < B; ++b)
        if (q0 + b < n)
#pragma unroll
          for (int h = 0; h < NH; ++h) acc[h] = q0 + b == 0 ? ring[b][h] : acc[h] + ring[b][h];
    }
    if (k == 0) LQ_TS(2);
    const int col = (wtile0 + i) * 16 + 4 * t;
    if (tok >= a.M || col >= Nm) continue;
    if constexpr (PAIR) {
      uint16_t o[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float gs = acc[0][v] * sv[k][0][v];
        const float us = acc[NH - 1][v] * sv[k][NH - 1][v];
        o[v] = f32_to_bf16(silu(gs) * us);
      }
      *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(a.y[0]) + static_cast<size_t>(tok) * ldy + col) =
          u32x2{o[0] | (uint32_t(o[1]) << 16), o[2] | (uint32_t(o[3]) << 16)};
    } else {
      float vv[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        vv[v] = acc[0][v] * sv[k][0][v];
        if (a.xinv) vv[v] = vv[v] * xi[k];
      }
      void* const y = pick(a.y, mi);
      const size_t o = static_cast<size_t>(tok) * ldy + col;
      if constexpr (OUTF32) {
        *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(y) + o) = f32x4{vv[0], vv[1], vv[2], vv[3]};
      } else {
        if (resid) {
          vv[0] = vv[0] + bf16_to_f32(rr[k].x & 0xffff);
          vv[1] = vv[1] + bf16_to_f32(rr[k].x >> 16);
          vv[2] = vv[2] + bf16_to_f32(rr[k].y & 0xffff);
          vv[3] = vv[3] + bf16_to_f32(rr[k].y >> 16);
        }
        *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(y) + o) =
            u32x2{f32_to_bf16(vv[0]) | (uint32_t(f32_to_bf16(vv[1])) << 16),
                  f32_to_bf16(vv[2]) | (uint32_t(f32_to_bf16(vv[3])) << 16)};
      }
    }
  }
}

// G <= 2: a chunk's activation operands (all four steps) are read from LDS one chunk ahead, into registers,
// through a ring of three LDS slots; larger G reads them within the chunk from a ring of two.
template <int G>
struct Smem {
  static constexpr bool BPRE = G <= 2;
  static constexpr int NSLOT = BPRE ? 3 : 2;
  static constexpr int XS_BYTES = 16 * G * 256;  // one chunk of activations, 16G rows
  uint8_t xs[NSLOT][XS_BYTES];
  float xsc[NSLOT][16 * G];  // kCvt: 2^(e - 15) of each row's chunk in the slot
  uint8_t tabs[kMaxMats][64];
  int last_flag[2];
};

// Body modes: kYCoh = the pair epilogue's stores write through (a later phase of the same launch reads them);
// kXCoh = activations are read agent-coherently and only after `ready()` returns (the weight ring's first
// stages are issued before the wait); kCvt = BF16 activations become FP16 as each chunk is staged, with a
// power-of-two scale per row and chunk (from the chunk's largest magnitude, as to_half_rows does per row) that
// each chunk's MFMA sums are multiplied back by, in FP32, before they join the running sums.
constexpr int kYCoh = 1, kXCoh = 2, kCvt = 4;

// kCvt staging of one thread's 8 activations (a 16-byte unit of row `row`; the row's 16 units of the chunk are
// in 16 consecutive lanes): returns them as FP16 scaled by 2^(15 - e), e = exponent of the chunk's largest
// magnitude in the row (0 when that is zero or not finite), and stores 2^(e - 15) for the row.
__device__ __forceinline__ u32x4 stage_cvt(const u32x4& v, float* xsc_row, bool writer) {
  float f[8];
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    f[2 * k] = __uint_as_float(w[k] << 16);
    f[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
  }
  float m = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) m = fmaxf(m, fabsf(f[k]));
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
  int e = 0;
  if (m > 0.f && isfinite(m)) frexpf(m, &e);
  const float sc = ldexpf(1.f, 15 - e);
  if (writer) *xsc_row = ldexpf(1.f, e - 15);
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    o[k] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(f[2 * k] * sc, f[2 * k + 1] * sc));
  return u32x4{o[0], o[1], o[2], o[3]};
}

struct NoWait {
  __device__ void operator()() const {}
};

// Logical workgroup id: blockIdx.x % 8 is the XCD the hardware places it on; consecutive logical ids share an
// XCD, so a tile group's partials are exchanged within one L2.
template <bool ONESEG>
__device__ __forceinline__ int logical_wg(const StreamArgs& a) {
  const int b = blockIdx.x;
  const SegSplit g = seg_split<ONESEG>(a, seg_of_wg<ONESEG>(a, b));
  const int bl = b - g.wgb;
  int p = bl;
  if ((g.P & 7) == 0 && (g.wgb & 7) == 0) p = (bl & 7) * (g.P >> 3) + (bl >> 3);
  return g.wgb + p;
}

}  // namespace lq
