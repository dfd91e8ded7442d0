// Weight-streaming ("skinny") GEMMs for 1..80 rows on gfx950: decode, speculative verify, drafter.
//
//   y[m][n] = epilogue( sum_k x[m][k] * Wq[n][k] ),  Wq = FP8 E4M3 or NVFP4 (E2M1 x E4M3 block scale) codes
//
// The weights are read once from HBM in the reference's tiled layout (a 16-row x 128-value block is
// contiguous); activations and partial sums stay on chip or in the caches. Design:
//
//  * MFMA v_mfma_f32_16x16x32_{bf16,f16}: A = 16 weight rows x 32 K, B = 32 K x 16 activation rows.
//    Lane l (r = l % 16, t = l / 16) owns weight row r of a tile and K range [32t, 32t + 32) of each
//    128-value chunk. An FP8 block's 16-byte pieces for that row/range sit at ((h*2+q)*8+g)*4+t
//    (g = r % 8, h = r / 8, q = 0, 1) and an NVFP4 block's at slot r*4+t, so each load instruction of the
//    wave covers whole 512-byte (FP8) or 1024-byte (NVFP4) runs of the block. The MFMA's logical k of
//    step s maps to physical K 32t + 8s + j for the weights and the activations alike.
//  * Dequantization in registers, exact: FP8 -> BF16/FP16 with v_cvt_scalef32_pk_*_fp8 (scale 1.0);
//    NVFP4 -> FP16 with v_cvt_scalef32_pk_f16_fp4 (scale 1.0) then one v_pk_mul_f16 by the E4M3 block
//    scale (e2m1 * e4m3 has at most 5 significant bits: exact in FP16). The per-channel / global scale
//    is applied in FP32 in the epilogue.
//  * A workgroup is 4 waves over a tile group of 16 tiles (256 weight rows); wave w owns tiles
//    4w .. 4w + 3 and all waves walk the same K chunks in lock step. Each chunk's activations are staged
//    once per workgroup in LDS (each wave loads a quarter; 16-byte units XOR-swizzled by row so the
//    MFMA operand reads are conflict free), while each wave streams its own weights through a ring of PF
//    chunks in registers. Loads retire in issue order, so a chunk's activation share is issued before its
//    weights and the stages are consumed oldest first: every wait leaves the newer stages in flight.
//  * Work split: units = (tile group, K chunk); P workgroups each take a contiguous, equal range of
//    units (a stream-K split), so every CU streams the same number of bytes whatever N and K are. A tile
//    group split across workgroups is finished by the last workgroup to arrive (an arrival counter per
//    group), which adds the partial sums in workgroup order and applies the epilogue.
//  * Determinism and row invariance: P, the tile grouping and the chunk order depend only on N, K and
//    the device's CU count, never on M, and an MFMA's column j depends only on activation row j; so a
//    row's result is bit for bit the same at any M, as the reference guarantees
//    (reference src/core/stream_gemm.cu:10-13).
//  * XCD-aware placement: workgroup ids are permuted so that consecutive ranges of units (and the
//    partials exchanged between them) stay on one XCD's L2.
#include "stream_common.hpp"

#include <algorithm>
#include <atomic>
#include <cstddef>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <type_traits>
#include <utility>

namespace lq {
// FP8 launches whose kernels run faster with MFMA accumulators in VGPRs (-mllvm -amdgpu-mfma-vgpr-form, a
// per-translation-unit switch): this file is compiled a second time with it and LQ_STREAM_VGPR_TU defined,
// keeping only the kernels and launch_g_vgpr. Measured per kernel against the AGPR form (rocprofv3, the
// verify, decode-step, shape and fc workloads): 0.4-9 % faster for every FP8 kernel with one or two tiles per
// wave up to three token groups and with one tile per wave at four or five (verify gate|up 2.3 %, down 3.2 %),
// the verify step at M = 49 and 64 (two tiles, four groups) 5 % faster, 2-4 % slower with two tiles at five;
// the NVFP4 kernels do not change. The same arithmetic either way.
template <int G, int WF, int TW, bool F16, bool PAIR, bool OUTF32, bool CVT>
int launch_g_vgpr(const StreamArgs& a, hipStream_t s);
constexpr bool vgpr_form(int G, int WF, int TW) { return WF == kFp8 && (G <= 4 || TW == 1); }
// The one-launch FFN (phase A: a gate|up pair, phase B: a single matrix, two tiles per wave each) likewise up
// to four token groups (ffn_kernel<2> 56.3 -> 55.2 us, rocprofv3).
template <int G>
void launch_ffn_vgpr(const StreamArgs& a, const StreamArgs& b, int* sync, hipStream_t s);

namespace {
// NPRE (with kXCoh only): the range's first NPRE chunks run ahead (see the prologue), with their activation images and
// wave 0's weights in xpre.
template <int G, int WF, int TW, bool F16, bool PAIR, bool OUTF32, int MODE, bool ONE = false, int NPRE = 0,
          class Ready>
__device__ __forceinline__ void stream_body(const StreamArgs& a, int p, Smem<G>& sm, Ready&& ready,
                                            uint8_t* xpre = nullptr) {
  constexpr int T = TW;
  constexpr int PF = pf_stages<T>(G);
  constexpr bool BPRE = Smem<G>::BPRE;
  constexpr int NSLOT = Smem<G>::NSLOT;
  constexpr bool YCOH = (MODE & kYCoh) != 0, XCOH = (MODE & kXCoh) != 0;
  constexpr int XPOL = XCOH ? kSc1 : 0;
  constexpr bool CVT = (MODE & kCvt) != 0;
  static_assert(!CVT || F16, "converted activations feed the FP16 MFMA");
  static_assert(!BPRE || PF >= 3, "the operand prefetch needs a chunk of lookahead");
  static_assert(NPRE == 0 || (XCOH && !CVT), "run-ahead chunks are for the activation-waiting form");
  constexpr int NP1 = NPRE > 0 ? NPRE : 1;
  auto& xs = sm.xs;
  auto& tabs = sm.tabs;
  auto& last_flag = sm.last_flag;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, t = lane >> 4;
  unsigned long long ts[16] = {};
  LQ_TS(0);
  // One field of every 64-byte line of the arguments, read in one batch: later argument reads then hit the
  // scalar cache instead of making dependent cold round trips (about a microsecond each) before the first
  // weight load can issue.
  asm volatile("" ::"s"(a.x), "s"(a.w[2]), "s"(a.svec[2]), "s"(a.resid[0]), "s"(a.tg0[4]));
  LQ_TS(10);
  auto flush_trace = [&](int pid) {
#ifdef LQ_STREAM_TRACE
    LQ_TS(6);
    if (a.trace && threadIdx.x == 0)
      for (int k = 0; k < 16; ++k) a.trace[pid * 16 + k] = ts[k];
#else
    (void)pid;
    (void)ts;
#endif
  };

  if constexpr (WF == kFp4Coded) {
    for (int i = threadIdx.x; i < a.count * 64; i += kThreads) tabs[i >> 6][i & 63] = a.table[i >> 6][i & 63];
    __syncthreads();
  }

  // this workgroup's units, in the global (tile group, chunk) numbering
  const SegSplit seg = seg_split<PAIR || ONE>(a, seg_of_wg<PAIR || ONE>(a, p));
  const int u0 = seg.tgb * a.C + unit_start(p - seg.wgb, seg.P, seg.U);
  const int u1 = seg.tgb * a.C + unit_start(p - seg.wgb + 1, seg.P, seg.U);
  const int n_it = u1 - u0;  // chunks this workgroup streams
  if (n_it <= 0) {
    flush_trace(p);
    return;
  }
  const int tg_first = u0 / a.C, tg_last = (u1 - 1) / a.C;
  const int cfirst = u0 - tg_first * a.C;

  // This thread's share of a chunk's activations: units q = i * 256 + tid of the 16G x 16 units (row q / 16,
  // 16-byte unit q % 16). Rows past M read as zeros from out-of-range offsets (their MFMA columns are never
  // stored).
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x);
  int xsrc[G], xdst[G];
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int q = i * kThreads + static_cast<int>(threadIdx.x), row = q >> 4, u = q & 15;
    xsrc[i] = row < a.M ? (row * a.K) * 2 + u * 16 : static_cast<int>(0x80000000u);
    xdst[i] = xs_off(row, u);
  }
  // weight lane offset: FP8 piece ((h*2 + 0)*8 + g)*4 + t (q = 1 is 512 bytes on); NVFP4 slot r*4 + t
  const int slot = r * 4 + t;
  const int lane_off = WF == kFp8 ? (((r >> 3) * 16 + (r & 7)) * 4 + t) * 16 : slot * 16;

  // The workgroup's units form one continuous stream through the register ring, across tile-group
  // boundaries: the load cursor (ltg, lc) runs PF - 1 chunks ahead of the compute cursor (ctg, cc).
  int ltg = tg_first, lc = cfirst, lleft = n_it;
  SegTiles<WF, T, PAIR> L;
  seg_tiles<WF, T, PAIR, ONE>(a, ltg, wave, L);
  LQ_TS(11);
  int ctg = tg_first, cc = cfirst;
  int cmi = L.mi, cwtile0 = L.wtile0;

  WRegs<WF, T> wr[PF];
  u32x4 xr[PF][G];
  // Every ring load is issued unconditionally (the wait counts then hold on every path); a load past the
  // stream's end is turned into an out-of-range buffer load (offset >= num_records), which returns zeros and
  // touches no memory.
  auto load_x = [&](int j, int lcj, unsigned oob) {
#pragma unroll
    for (int i = 0; i < G; ++i)
      xr[j][i] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, static_cast<int>(xsrc[i] | oob), lcj * 256, XPOL));
  };
  auto advance = [&]() {
    if (lleft > 0) {
      --lleft;
      if (++lc == a.C) {
        lc = 0;
        ++ltg;
        if (lleft > 0) seg_tiles<WF, T, PAIR, ONE>(a, ltg, wave, L);
      }
    }
  };
  auto load_stage = [&](int j) {
    const unsigned oob = lleft > 0 ? 0u : 0x80000000u;
    // scheduling barriers keep the issue order (activations, then weights, chunk after chunk) that the
    // in-order wait counts rely on
    __builtin_amdgcn_sched_barrier(0);
    load_x(j, lc, oob);
    __builtin_amdgcn_sched_barrier(0);
    load_w<WF, T>(wr[j], L.rs, L.toff, L.coff, lc, static_cast<int>(lane_off | oob), slot, oob);
    __builtin_amdgcn_sched_barrier(0);
    advance();
  };
  // The same stage in two parts, as the main loops issue it: the activation share before the chunk's barrier,
  // the weights after it. The activations of every wave then reach the memory pipeline while the waves gather at
  // the barrier, instead of all of a chunk's loads leaving in one burst behind it (measured: the M=68 launches
  // 3-5 % faster, M=17 about 1 %).
  unsigned stage_oob = 0u;
  auto load_stage_x = [&](int j) {
    stage_oob = lleft > 0 ? 0u : 0x80000000u;
    __builtin_amdgcn_sched_barrier(0);
    load_x(j, lc, stage_oob);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto load_stage_w = [&](int j) {
    __builtin_amdgcn_sched_barrier(0);
    load_w<WF, T>(wr[j], L.rs, L.toff, L.coff, lc, static_cast<int>(lane_off | stage_oob), slot, stage_oob);
    __builtin_amdgcn_sched_barrier(0);
    advance();
  };
  auto put_x = [&](int j, int sl) {
#pragma unroll
    for (int i = 0; i < G; ++i) {
      if constexpr (CVT) {
        const int row = (i * kThreads + static_cast<int>(threadIdx.x)) >> 4;
        *reinterpret_cast<u32x4*>(xs[sl] + xdst[i]) = stage_cvt(xr[j][i], &sm.xsc[sl][row], (threadIdx.x & 15) == 0);
      } else {
        *reinterpret_cast<u32x4*>(xs[sl] + xdst[i]) = xr[j][i];
      }
    }
  };
  // kCvt: a chunk's MFMA sums (accc) join the running sums (acc2) times the row's chunk scale.
  f32x4 accc[T][G];
  auto clear_c = [&]() {
#pragma unroll
    for (int i = 0; i < T; ++i)
#pragma unroll
      for (int g = 0; g < G; ++g) accc[i][g] = f32x4{0.f, 0.f, 0.f, 0.f};
  };
  auto chunk_scales = [&](float (&scs)[G], int sl) {
#pragma unroll
    for (int g = 0; g < G; ++g) scs[g] = sm.xsc[sl][16 * g + r];
  };

  // The first tile group's sums wait in accF for the end of the stream; a tile group wholly inside the range
  // is finished where it ends.
  f32x4 acc2[T][G], accF[T][G];
#pragma unroll
  for (int i = 0; i < T; ++i)
#pragma unroll
    for (int g = 0; g < G; ++g) acc2[i][g] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto fold_c = [&](const float (&scs)[G]) {
#pragma unroll
    for (int i = 0; i < T; ++i)
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc2[i][g][v] = __builtin_fmaf(accc[i][g][v], scs[g], acc2[i][g][v]);
  };
  auto fold = [&](f32x4 (&out)[T][G]) {
#pragma unroll
    for (int i = 0; i < T; ++i)
#pragma unroll
      for (int g = 0; g < G; ++g) {
        out[i][g] = acc2[i][g];
        acc2[i][g] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
  };
  auto after_chunk = [&](int it) {
    if (++cc == a.C && it + 1 < n_it) {
      if (ctg == tg_first) {
        fold(accF);
      } else {
        f32x4 accM[T][G];
        fold(accM);
        EpiIn<G, T> eM;
        epi_load<G, PAIR, OUTF32, T>(a, cmi, cwtile0, eM, r, t);
        epilogue<G, PAIR, OUTF32, T, YCOH>(a, cmi, cwtile0, accM, eM, r, t);
        // Let these stores complete here: with stores of unknown completion order in flight, every later wait
        // on the ring would have to drain it (vmcnt(0)); after this wait the ring's waits stay partial.
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0), expcnt and lgkmcnt unconstrained (gfx9 encoding)
      }
      ++ctg;
      cc = 0;
      SegTiles<WF, T, PAIR> s;
      seg_tiles<WF, T, PAIR, ONE>(a, ctg, wave, s);
      cmi = s.mi;
      cwtile0 = s.wtile0;
    }
  };
  auto tables = [&](const uint8_t* (&tab)[T]) {
#pragma unroll
    for (int i = 0; i < T; ++i) tab[i] = tabs[PAIR ? (i < T / 2 ? 0 : 1) : cmi];
  };

  // The epilogue inputs of the range's first and last tile groups, read ahead of the weight stream.
  SegTiles<WF, T, PAIR> sF, sL;
  seg_tiles<WF, T, PAIR, ONE>(a, tg_first, wave, sF);
  seg_tiles<WF, T, PAIR, ONE>(a, tg_last, wave, sL);
  EpiIn<G, T> eF, eL;
  epi_load<G, PAIR, OUTF32, T>(a, sF.mi, sF.wtile0, eF, r, t);
  LQ_TS(12);
  epi_load<G, PAIR, OUTF32, T>(a, sL.mi, sL.wtile0, eL, r, t);
  LQ_TS(13);

  // the ring streams the chunks after the NPRE run-ahead ones (n_ring of them)
  const int n_ring = max(n_it - NPRE, 0);
  const int npad = (n_ring + PF - 1) / PF * PF;
  WRegs<WF, T> pr[NP1];
  if constexpr (XCOH && NPRE > 0) {
    // Run-ahead: before the wait for the activations, waves 1-3 load the weights of the range's first NPRE chunks and
    // of the ring's first stages into registers. Wave 0 issues no load before the wait, so that its polls in ready()
    // return at the memory's latency (a poll's result waits for every load the wave issued before it), and loads its
    // share right after. Then the run-ahead chunks' activation images come straight into LDS, the ring's activations
    // follow, and the run-ahead chunks are computed while the ring's loads are in flight.
    static_assert(WF == kFp8, "the run-ahead form streams FP8 weights");
    int plc[NP1];
    unsigned poob[NP1];
    SegTiles<WF, T, PAIR> Lp[NP1];
#pragma unroll
    for (int c = 0; c < NPRE; ++c) {
      poob[c] = lleft > 0 ? 0u : 0x80000000u;
      plc[c] = lc;
      Lp[c] = L;
      if (wave != 0) load_w<WF, T>(pr[c], L.rs, L.toff, L.coff, lc, static_cast<int>(lane_off | poob[c]), slot, poob[c]);
      advance();
    }
    int lcs[PF - 1];
    unsigned oobs[PF - 1];
    SegTiles<WF, T, PAIR> Lr[PF - 1];
#pragma unroll
    for (int j = 0; j < PF - 1; ++j) {
      oobs[j] = lleft > 0 ? 0u : 0x80000000u;
      lcs[j] = lc;
      Lr[j] = L;
      if (wave != 0) load_w<WF, T>(wr[j], L.rs, L.toff, L.coff, lc, static_cast<int>(lane_off | oobs[j]), slot, oobs[j]);
      advance();
    }
    ready();
    LQ_TS(15);
    if (wave == 0) {
#pragma unroll
      for (int c = 0; c < NPRE; ++c)
        load_w<WF, T>(pr[c], Lp[c].rs, Lp[c].toff, Lp[c].coff, plc[c], static_cast<int>(lane_off | poob[c]), slot,
                      poob[c]);
    }
    // chunk c's image: 16G rows x 16 units of 16 bytes, as put_x lays it out (unit u of row m at u ^ (m & 15));
    // load k of wave w fills 64 consecutive units (rows 4 (4k + w) .. +4), each lane fetching the source unit that
    // belongs at its place
#pragma unroll
    for (int c = 0; c < NPRE; ++c)
#pragma unroll
      for (int k = 0; k < G; ++k) {
        const int row = 4 * (4 * k + wave) + (lane >> 4), u = (lane & 15) ^ (row & 15);
        const unsigned src = row < a.M ? static_cast<unsigned>((row * a.K) * 2 + u * 16) : 0x80000000u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            xrs, (__attribute__((address_space(3))) void*)(xpre + c * Smem<G>::XS_BYTES + (4 * k + wave) * 1024), 16,
            static_cast<int>(src | poob[c]), __builtin_amdgcn_readfirstlane(plc[c] * 256), 0, XPOL);
      }
    if (wave == 0) {
#pragma unroll
      for (int j = 0; j < PF - 1; ++j)
        load_w<WF, T>(wr[j], Lr[j].rs, Lr[j].toff, Lr[j].coff, lcs[j], static_cast<int>(lane_off | oobs[j]), slot,
                      oobs[j]);
    }
#pragma unroll
    for (int j = 0; j < PF - 1; ++j) load_x(j, lcs[j], oobs[j]);
    // the run-ahead images have landed (only the ring's loads, issued after them, may still be in flight)
    constexpr int kLater = (PF - 1) * G, kLater0 = (PF - 1) * (G + 2 * T);
    static_assert(kLater0 < 64, "vmcnt holds at most 63");
    if (wave == 0)
      __builtin_amdgcn_s_waitcnt(0x0f70 | (kLater0 & 15) | ((kLater0 >> 4) << 14));
    else
      __builtin_amdgcn_s_waitcnt(0x0f70 | (kLater & 15) | ((kLater >> 4) << 14));
    __syncthreads();
#pragma unroll
    for (int c = 0; c < NPRE; ++c) {
      if (c < n_it) {
        const uint8_t* tab[T];
        tables(tab);
        compute_lds<WF, F16, G, T>(pr[c], xpre + c * Smem<G>::XS_BYTES, acc2, r, t, tab);
        if (c == 0) LQ_TS(1);
        after_chunk(c);
      }
    }
  } else if constexpr (XCOH) {
    // weights of the first stages first, then the wait for the activations, then their loads
    int lcs[PF - 1];
    unsigned oobs[PF - 1];
#pragma unroll
    for (int j = 0; j < PF - 1; ++j) {
      oobs[j] = lleft > 0 ? 0u : 0x80000000u;
      lcs[j] = lc;
      load_w<WF, T>(wr[j], L.rs, L.toff, L.coff, lc, static_cast<int>(lane_off | oobs[j]), slot, oobs[j]);
      advance();
    }
    ready();
    LQ_TS(15);
#pragma unroll
    for (int j = 0; j < PF - 1; ++j) load_x(j, lcs[j], oobs[j]);
  } else {
#pragma unroll
    for (int j = 0; j < PF - 1; ++j) {
      load_stage(j);
      if (j == 0) LQ_TS(14);
    }
  }
  LQ_TS(7);
  if constexpr (BPRE) {
    u32x4 bc[4][G], bn[4][G];
    float scc[G], scn[G];
    put_x(0, 0);
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 4; ++s) read_b<G>(bc[s], xs[0], s, r, t);
    if constexpr (CVT) chunk_scales(scc, 0);
    for (int base = 0; base < npad; base += PF) {
#pragma unroll
      for (int j = 0; j < PF; ++j) {
        const int it = base + j;
        const int sl = (it + 1) % NSLOT;
        put_x((j + 1) % PF, sl);
        load_stage_x((j + PF - 1) % PF);
        __syncthreads();
        load_stage_w((j + PF - 1) % PF);
#pragma unroll
        for (int s = 0; s < 4; ++s) read_b<G>(bn[s], xs[sl], s, r, t);
        if constexpr (CVT) chunk_scales(scn, sl);
        if (it < n_ring) {
          const uint8_t* tab[T];
          tables(tab);
          if constexpr (CVT) {
            clear_c();
#pragma unroll
            for (int s = 0; s < 4; ++s) mfma_step<WF, F16, G, T>(wr[j], s, bc[s], accc, tab);
            fold_c(scc);
          } else {
#pragma unroll
            for (int s = 0; s < 4; ++s) mfma_step<WF, F16, G, T>(wr[j], s, bc[s], acc2, tab);
          }
          if (NPRE == 0 && it == 0) LQ_TS(1);
          after_chunk(NPRE + it);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int g = 0; g < G; ++g) bc[s][g] = bn[s][g];
        if constexpr (CVT) {
#pragma unroll
          for (int g = 0; g < G; ++g) scc[g] = scn[g];
        }
      }
    }
  } else {
    for (int base = 0; base < npad; base += PF) {
#pragma unroll
      for (int j = 0; j < PF; ++j) {
        const int it = base + j;
        put_x(j, it & 1);
        load_stage_x((j + PF - 1) % PF);
        __syncthreads();
        load_stage_w((j + PF - 1) % PF);
        if (it < n_ring) {
          const uint8_t* tab[T];
          tables(tab);
          if constexpr (CVT) {
            float scs[G];
            chunk_scales(scs, it & 1);
            clear_c();
            compute_lds<WF, F16, G, T>(wr[j], xs[it & 1], accc, r, t, tab);
            fold_c(scs);
          } else {
            compute_lds<WF, F16, G, T>(wr[j], xs[it & 1], acc2, r, t, tab);
          }
          if (NPRE == 0 && it == 0) LQ_TS(1);
          after_chunk(NPRE + it);
        }
      }
    }
  }
  f32x4 accL[T][G];
  fold(accL);
  LQ_TS(2);

  // Finish the first and the last tile group of the range: a whole one directly, a split one through the
  // partial exchange (every workgroup publishes, counts its arrival, and the last to arrive adds them).
  const bool one = tg_first == tg_last;
  const bool splitF = !one && cfirst != 0;
  const int lbeg = one ? cfirst : 0;
  const int lend = u1 - tg_last * a.C;
  const bool splitL = !(lbeg == 0 && lend == a.C);
  if (!one) {
    if (splitF) publish_partial<G, T>(a, p, 0, accF, r);
    else epilogue<G, PAIR, OUTF32, T, YCOH>(a, sF.mi, sF.wtile0, accF, eF, r, t);
  }
  // Where tile groups span two workgroups or more, a workgroup with two partials counts its first group's
  // arrival before it publishes the second: otherwise it arrives last at both groups more often than not (it has
  // the most to publish) and then finishes both in a row, the slowest finish there is (measured: down at M=17 and
  // the M=68 projections 3-6 % faster). The gate|up pair, where nearly every workgroup has two partials, keeps
  // the single wait (the extra one measured 1 % slower there).
  const bool early = !PAIR && !a.NR && splitF && splitL && seg.P >= 2 * (seg.U / a.C);
  int oldF = 0;
  if (early) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
      oldF = __hip_atomic_fetch_add(a.counters + tg_first * a.cs, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (splitL) publish_partial<G, T>(a, p, one ? 0 : 1, accL, r);
  else epilogue<G, PAIR, OUTF32, T, YCOH>(a, sL.mi, sL.wtile0, accL, eL, r, t);
  if (!splitF && !splitL) {
    flush_trace(p);
    return;
  }
  // Each thread waits for its own partial stores to complete before the barrier; only then does thread 0
  // count the workgroup's arrival.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  LQ_TS(3);
  if (a.NR) {  // the finish workgroups add the partials
    if (threadIdx.x == 0) {
      if (splitF) __hip_atomic_fetch_add(a.counters + tg_first * a.cs, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (splitL) __hip_atomic_fetch_add(a.counters + tg_last * a.cs, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    flush_trace(p);
    return;
  }
  const SplitInfo si[2] = {split_info<PAIR || ONE>(a, tg_first), split_info<PAIR || ONE>(a, tg_last)};
  // (selects rather than indexing si by thread: a thread-indexed local array would be placed in LDS)
  if (threadIdx.x < 2) {
    const bool h = threadIdx.x != 0;
    const int tg = h ? tg_last : tg_first;
    const int span = h ? si[1].pl - si[1].pf : si[0].pl - si[0].pf;
    int last = 0;
    if (h ? splitL : splitF) {
      const int old = (!h && early) ? oldF
                                    : __hip_atomic_fetch_add(a.counters + tg * a.cs, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = old == span;
      if (last) __hip_atomic_store(a.counters + tg * a.cs, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    last_flag[h ? 1 : 0] = last;
  }
  __syncthreads();
  const bool doit[2] = {last_flag[0] != 0, last_flag[1] != 0};
  LQ_TS(4);
  if (!doit[0] && !doit[1]) {
    flush_trace(p);
    return;
  }
  // Both groups' reductions share their round trips when their rings fit in registers (T x G <= 8).
  if (T * G <= 8 && doit[0] && doit[1]) {
    f32x4 (*accs[2])[G] = {accF, accL};
    reduce_partials<G, T, (T * G <= 8 ? 2 : 1)>(a, si, accs, r, ts);
  } else {
    if (doit[0]) {
      f32x4 (*accs[1])[G] = {accF};
      reduce_partials<G, T, 1>(a, si, accs, r, ts);
    }
    if (doit[1]) {
      f32x4 (*accs[1])[G] = {accL};
      reduce_partials<G, T, 1>(a, si + 1, accs, r, ts);
    }
  }
  LQ_TS(9);
  if (doit[0]) epilogue<G, PAIR, OUTF32, T, YCOH>(a, sF.mi, sF.wtile0, accF, eF, r, t);
  if (doit[1]) epilogue<G, PAIR, OUTF32, T, YCOH>(a, sL.mi, sL.wtile0, accL, eL, r, t);
  LQ_TS(5);
  flush_trace(p);
}

template <int G, int WF, int TW, bool F16, bool PAIR, bool OUTF32, bool CVT = false, bool ONE = false>
__global__ void __launch_bounds__(kThreads) stream_kernel(const StreamArgs a) {
  __shared__ __attribute__((aligned(16))) Smem<G> sm;
  if (static_cast<int>(blockIdx.x) >= a.P) {
    finish_share<G, TW, PAIR, OUTF32, ONE>(a, static_cast<int>(blockIdx.x) - a.P);
    return;
  }
  stream_body<G, WF, TW, F16, PAIR, OUTF32, CVT ? kCvt : 0, ONE>(a, logical_wg<PAIR || ONE>(a), sm, NoWait{});
}

// The FFN step in one launch (reference persistent FFN, src/core/stream_gemm.cu:841-1072): phase A = gate|up
// with SiLU(gate) * up into h (a), phase B = down (+ residual) from h (b). Both phases use the same P and the
// same split as two separate launches, so every output is bit for bit theirs. Each workgroup ends phase A
// with its h stores complete and counts itself on sync[0]; phase B issues its first weight stages, then waits
// until all P have arrived (a workgroup that finished phase A early spends the wait with weights in flight),
// then reads h agent-coherently. Requires all P workgroups to be resident at once (P <= #CUs, one launch of
// this kernel per device at a time); a wait past its deadline records sync[2] = 1 and goes on, so the
// kernel always exits. The last workgroup out resets the counters (no memset node in a captured graph).
constexpr unsigned long long kFfnDeadlineTicks = 10'000'000ull;  // s_memrealtime at 100 MHz: 100 ms
constexpr int kFfnFlag = 32;  // sync[32]: phase B may read h (128 bytes past the counters)

#ifndef LQ_NPRE2
#define LQ_NPRE2 4
#endif
// Phase B's run-ahead chunks (weights in registers, their activation images in LDS), by register budget.
template <int G>
constexpr int ffn_run_ahead() { return LQ_NPRE2; }

template <int G>
__global__ void __launch_bounds__(kThreads) ffn_kernel(const StreamArgs a, const StreamArgs b, int* sync) {
  __shared__ __attribute__((aligned(16))) Smem<G> sm;
  constexpr int NPRE = ffn_run_ahead<G>();
  __shared__ __attribute__((aligned(16))) uint8_t xpre[(NPRE > 0 ? NPRE : 1) * Smem<G>::XS_BYTES];  // run-ahead activation images
  const int p = logical_wg<true>(a);
  stream_body<G, kFp8, 2, false, true, false, kYCoh>(a, p, sm, NoWait{});
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's h stores have completed
  __syncthreads();
  // The hand-over of h: every h store is a write-through store (sc1) and has completed (the wait above, before the
  // barrier) when thread 0 counts the workgroup's arrival; phase B reads h with loads that bypass the non-coherent
  // caches (sc1) only after it has seen all P arrivals. So no cache needs a writeback or an invalidation: a release
  // / acquire pair at agent scope adds an L2 writeback to each arrival and an L2 invalidation to each poll, which
  // measured 10 us slower per step than these relaxed atomics.
  // The last to arrive raises the ready flag (sync[kFfnFlag], a cache line of its own): the pollers read the flag, so
  // that their reads do not queue with the arrivals' atomics on the counter.
  const int P = a.P;
  if (threadIdx.x == 0 && __hip_atomic_fetch_add(sync, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == P - 1)
    __hip_atomic_store(sync + kFfnFlag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  auto ready = [&]() {
    if (threadIdx.x == 0) {
      const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
      while (__hip_atomic_load(sync + kFfnFlag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0) {
        __builtin_amdgcn_s_sleep(8);
        if (__builtin_amdgcn_s_memrealtime() - t0 > kFfnDeadlineTicks) {
          __hip_atomic_store(sync + 2, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
      }
    }
    __syncthreads();
  };
  // Phase B runs on its own split's b.P <= P workgroups (the first b.P blocks, mapped as a launch of b alone would
  // map them); the rest only count themselves out below.
  if (static_cast<int>(blockIdx.x) < b.P)
    stream_body<G, kFp8, 2, false, false, false, kXCoh, true, NPRE>(b, logical_wg<true>(b), sm, ready, xpre);
  __syncthreads();
  if (threadIdx.x == 0 &&
      __hip_atomic_fetch_add(sync + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == P - 1) {
    __hip_atomic_store(sync, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(sync + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(sync + kFfnFlag, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

#ifndef LQ_STREAM_VGPR_TU
// ---------------- gathered rows (reference stream_gemm_gather_nvfp4, src/core/stream_gemm.cu:1902-1923) -------------
// y[m][i] = scale2 * x[m] . W[rows[i]] * xinv[m] for i < *nrows, -inf for nrows <= i < cap, with every element's
// arithmetic that of the full NVFP4 launch over all N rows (so a selected row's logit is bit for bit the full
// head's): the same 16 value bytes and 2 scale bytes per chunk (a coded blob's raw-scale copy holds exactly the
// bytes its codes stand for), the same MFMA steps in chunk order, the accumulator cut where the full launch's
// stream-K split cuts that row's tile group (workgroup boundaries of the full launch's P and units), and the
// segments added left to right as its finisher adds them. A wave computes 16 gathered rows; a lane's four
// output rows may belong to different tile groups, so each keeps its own next cut.
// Calls f(integral_constant<int, 0>) .. f(integral_constant<int, N - 1>) in order: a body unrolled at compile time,
// so register arrays indexed by the constant stay in registers.
template <class F, int... J>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, J...>) {
  (f(std::integral_constant<int, J>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

struct GatherArgs {
  const void* x;      // FP16 [M][K]
  const float* xinv;  // [M]
  int M, K, C;
  const uint8_t* w;    // tiled NVFP4 blob (raw: 1152 B blocks; coded: 1024 B value blocks)
  const uint8_t* raw;  // coded blob's raw scales (128 B per block), or null for a raw blob
  float scale2;
  const int* rows;
  const int* nrows;
  int cap, N;        // N: the full matrix's rows
  int P, U, TGR;     // the full launch's workgroups, units and rows per tile group
  float* y;          // [M][cap]
};

// One wave per workgroup and no LDS: a lane's B operand for a chunk is 64 contiguous bytes of one activation row
// (row 16g + r, halves 32t .. 32t + 31 of the chunk, the four MFMA steps' 16-byte pieces in order), loaded from
// L2 straight into registers. Loads run D chunks ahead of the MFMA steps, so a wave's serial path per chunk is
// its MFMA chain alone, and the waves never wait on each other.
constexpr int kGatherThreads = 64;
template <int G>
struct GatherDepth {
  static constexpr int D = G == 1 ? 8 : G == 2 ? 4 : 2;  // chunks in flight: 16 * G * D activation VGPRs
};

// ONE (M % 16 == 1: the last token group holds a single row, M - 1): that row's four 16-byte pieces of a chunk
// come in one load (lane r < 4 takes piece r) and a row shift of the lanes hands piece s to lane 0; the other
// lanes of the group get values of rows past M, whose MFMA columns are never stored. The MFMA operands of every
// stored column are the same as with four loads, so the results are too; it saves three of the wave's loads per
// chunk.
// SPLIT: one token group per workgroup (blockIdx.y): a wave per 16 gathered rows and 16 tokens, so M = 17..80
// fills 2..5 times the waves of one wave carrying every group. An MFMA output column's sum depends on that
// column's operands only, so each element is the same either way.
// amdgpu_waves_per_eu(2) caps the kernel at 256 registers, so its MFMAs accumulate in VGPRs (251 used, no
// AGPRs): with the accumulator in AGPRs the compiler copies it out before every cut test, which waits for the
// chunk's whole MFMA chain.
template <int G, bool ONE, bool SPLIT = false>
__global__ void __launch_bounds__(kGatherThreads) __attribute__((amdgpu_waves_per_eu(2))) gather_kernel(const GatherArgs a) {
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, t = lane >> 4;
  const int cnt = min(max(*a.nrows, 0), a.cap);
  const int i0 = static_cast<int>(blockIdx.x) * 16;  // this wave's first gathered row
  const int m0 = SPLIT ? 16 * static_cast<int>(blockIdx.y) : 0;  // this wave's first token
  // epilogue rows of this lane: gathered i = i0 + 4t + v, token m0 + 16g + r
  auto store = [&](const float (&val)[G][4]) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int m = m0 + 16 * g + r;
      if (m >= a.M) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = i0 + 4 * t + v;
        if (i < a.cap) a.y[static_cast<size_t>(m) * a.cap + i] = i < cnt ? val[g][v] : -INFINITY;
      }
    }
  };
  if (i0 >= cnt) {  // uniform over the wave
    float ninf[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int v = 0; v < 4; ++v) ninf[g][v] = -INFINITY;
    store(ninf);
    return;
  }
  const int blk_bytes = a.raw ? kValueBytesFp4 : kTileBytesFp4;
  const __amdgpu_buffer_rsrc_t wrs = make_rsrc(a.w);
  const __amdgpu_buffer_rsrc_t srs = make_rsrc(a.raw ? a.raw : a.w);
  // the lane's A row (loads): gathered row i0 + r; an invalid or unselected row reads as zeros
  const int ia = i0 + r;
  const int na = ia < cnt ? a.rows[ia] : -1;
  const unsigned aoob = (na >= 0 && na < a.N) ? 0u : 0x80000000u;
  const int nac = aoob ? 0 : na;
  const int slot = (nac & 15) * 4 + t;
  // the lane's output rows: their tile groups and next cuts
  // (wg_of_unit and unit_start by div_by_rcp: the host bounds U below 2^19 and (U + 1) * (P + 1) below 2^31, and a cut
  // inside the chunk loop then costs a few instructions, not two integer divisions on the wave's serial path)
  const float rP = 1.f / static_cast<float>(a.P), rU = 1.f / static_cast<float>(a.U);
  auto next_cut = [&](int u, int tg0) {  // the last chunk of the workgroup that holds unit u, relative to tg0
    const int p = div_by_rcp((u + 1) * a.P - 1, a.U, rU);
    return min(a.C - 1, div_by_rcp((p + 1) * a.U, a.P, rP) - 1 - tg0);
  };
  int tgc[4], nb[4];
  bool first[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int io = i0 + 4 * t + v;
    int no = io < cnt ? a.rows[io] : 0;
    no = (no >= 0 && no < a.N) ? no : 0;
    tgc[v] = (no / a.TGR) * a.C;
    nb[v] = next_cut(tgc[v], tgc[v]);
    first[v] = true;
  }
  // the lane's activation bytes: row 16g + r from byte 64t of each chunk (rows >= M read as zeros)
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x);
  unsigned xoff[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int m = m0 + 16 * g + r;
    xoff[g] = m < a.M ? static_cast<unsigned>(m * a.K * 2 + t * 64) : 0x80000000u;
  }
  // ONE: lane r < 4 of the last group loads piece r of row M - 1 (16 * (G - 1))
  const unsigned xone = r < 4 ? static_cast<unsigned>((16 * (G - 1)) * a.K * 2 + t * 64 + r * 16) : 0x80000000u;
  f32x4 acc[1][G];
  float tot[G][4];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    acc[0][g] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int v = 0; v < 4; ++v) tot[g][v] = 0.f;
  }
  const uint8_t* const tab[1] = {nullptr};
  constexpr int D = GatherDepth<G>::D;
  u32x4 xr[D][G][4], wv[D];
  uint32_t wsc[D];
  const size_t row_blk = static_cast<size_t>(nac >> 4) * a.C;
  auto issue = [&](auto J, int cc) {
    constexpr int j = decltype(J)::value;
    const unsigned o = cc < a.C ? 0u : 0x80000000u;  // past the last chunk: out of range, reads as zeros
    const int cl = min(cc, a.C - 1);
    const size_t blk = row_blk + cl;
    wv[j] = __builtin_bit_cast(
        u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, static_cast<int>((blk * blk_bytes + slot * 16) | aoob | o), 0, 0));
    const size_t so = a.raw ? blk * 128 + slot * 2 : blk * kTileBytesFp4 + 1024 + slot * 2;
    wsc[j] = static_cast<uint16_t>(__builtin_amdgcn_raw_buffer_load_b16(srs, static_cast<int>(so | aoob | o), 0, 0));
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (ONE && g == G - 1) {
        xr[j][g][0] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, static_cast<int>(xone | o), cl * 256, 0));
        continue;
      }
#pragma unroll
      for (int s = 0; s < 4; ++s)
        xr[j][g][s] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, static_cast<int>(xoff[g] | o), cl * 256 + s * 16, 0));
    }
  };
  static_for<D>([&](auto J) { issue(J, J); });
  for (int c0 = 0; c0 < a.C; c0 += D) {
    static_for<D>([&](auto J) {
      constexpr int j = decltype(J)::value;
      // a chunk past the last one (C % D != 0) reads zeros and adds +0 to an accumulator no cut reads: no branch,
      // so the ring's loads stay in flight across the chunk
      const int c = c0 + j;
      WRegs<kFp4, 1> R;
      R.v[0][0] = wv[j];
      R.sc[0] = wsc[j];
      u32x4 xb[G][4];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        if (ONE && g == G - 1) {
          // piece s from lane r + s of the 16-lane row (row_shl:s; lanes past the row read 0)
          const u32x4 v = xr[j][g][0];
          xb[g][0] = v;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            xb[g][1][q] = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v[q]), 0x101, 0xf, 0xf, true));
            xb[g][2][q] = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v[q]), 0x102, 0xf, 0xf, true));
            xb[g][3][q] = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v[q]), 0x103, 0xf, 0xf, true));
          }
          continue;
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) xb[g][s] = xr[j][g][s];
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        u32x4 b[G];
#pragma unroll
        for (int g = 0; g < G; ++g) b[g] = xb[g][s];
        mfma_step<kFp4, true, G, 1>(R, s, b, acc, tab);
      }
      // refill slot j only after its operands are consumed: issued before the MFMAs, the new and the old values
      // are live together, and the compiler reconciles the two register sets with copies at the loop's back
      // edge that wait for every load in flight, draining the ring every D chunks
      issue(J, c + D);
      // a cut is rare (a row's tile group ends or its workgroup changes): one wave-uniform test first, so the
      // common path never reads the accumulator (a read waits for the chunk's whole MFMA chain, and without
      // the test the compiler hoists the reads out of the per-row branches)
      bool cut = false;
#pragma unroll
      for (int v = 0; v < 4; ++v) cut |= c == nb[v];
      if (__builtin_amdgcn_ballot_w64(cut)) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          if (c == nb[v]) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
              tot[g][v] = first[v] ? acc[0][g][v] : tot[g][v] + acc[0][g][v];
              acc[0][g][v] = 0.f;
            }
            first[v] = false;
            if (c + 1 < a.C) nb[v] = next_cut(tgc[v] + c + 1, tgc[v]);
          }
        }
      }
    });
  }
  float val[G][4];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int m = m0 + 16 * g + r;
    const float xi = m < a.M ? a.xinv[m] : 1.f;
#pragma unroll
    for (int v = 0; v < 4; ++v) val[g][v] = (tot[g][v] * a.scale2) * xi;
  }
  store(val);
}

// ---------------- cache run-ahead (reference l2_prefetch_tiles_kernel, src/core/stream_gemm.cu:822-840) ----------
// Reads (and discards) what a stream GEMM over the same matrix reads first: for each of the launch's P workgroups,
// the first nc units (tile group x chunk) of its stream-K range, block by block, one 4-byte load per 64-byte piece
// so every cache line is fetched. Workgroup b takes the range the GEMM's workgroup b takes (the same XCD-aware
// permutation), so on a part that deals workgroups to XCDs by index the lines land in the L2 that GEMM workgroup
// reads through. Nothing is written; the GEMM that follows computes the same bits.
__global__ void __launch_bounds__(256) prefetch_units_kernel(const uint8_t* __restrict__ w, int C, int P, int U,
                                                             int tpg, int tiles, int blk, long long code_base,
                                                             int nc) {
  const int b = static_cast<int>(blockIdx.x);
  const int p = (P & 7) == 0 ? (b & 7) * (P >> 3) + (b >> 3) : b;
  const int u0 = unit_start(p, P, U), n = min(nc, unit_start(p + 1, P, U) - u0);
  const int pieces = tpg * blk / 64;  // 64-byte pieces of one unit's blocks
  uint32_t sink = 0;
  for (int k = 0; k < n; ++k) {
    const int u = u0 + k, tg = u / C, c = u - tg * C;
    for (int i = static_cast<int>(threadIdx.x); i < pieces; i += 256) {
      const int ti = i * 64 / blk, tile = tg * tpg + ti;
      if (tile < tiles)
        sink += *reinterpret_cast<const uint32_t*>(w + (static_cast<size_t>(tile) * C + c) * blk + (i * 64 - ti * blk));
    }
    // coded NVFP4: each tile's 96 code bytes of the chunk, in the blob's code region (two 64-byte pieces)
    if (code_base >= 0 && static_cast<int>(threadIdx.x) < 2 * tpg) {
      const int tile = tg * tpg + (static_cast<int>(threadIdx.x) >> 1);
      if (tile < tiles)
        sink += *reinterpret_cast<const uint32_t*>(w + code_base + (static_cast<size_t>(tile) * C + c) * kCodeBytesFp4 +
                                                   (threadIdx.x & 1) * 64);
    }
  }
  asm volatile("" ::"v"(sink));  // keeps the loads
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

// The same with one block per row and the row held in registers (NPT values per thread, thread t holding values
// t + 256 j): one read of the row, whose loads are all issued before the maximum is taken. Same arithmetic per
// element as half_rows_kernel. Rows up to 256 * NPT values.
template <bool BF16IN, int NPT>
__global__ void __launch_bounds__(256) half_rows_reg_kernel(const void* __restrict__ x, int K,
                                                            _Float16* __restrict__ out, float* __restrict__ xinv) {
  __shared__ float red[4];
  const size_t m = blockIdx.x;
  float v[NPT];
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int k = static_cast<int>(threadIdx.x) + 256 * j;
    if constexpr (BF16IN) v[j] = k < K ? bf16_to_f32(reinterpret_cast<const uint16_t*>(x)[m * K + k]) : 0.f;
    else v[j] = k < K ? reinterpret_cast<const float*>(x)[m * K + k] : 0.f;
  }
  float mx = 0.f;
#pragma unroll
  for (int j = 0; j < NPT; ++j) mx = fmaxf(mx, fabsf(v[j]));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int e = 0;
  if (mx > 0.f && isfinite(mx)) frexpf(mx, &e);
  const float s = ldexpf(1.f, 15 - e);
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int k = static_cast<int>(threadIdx.x) + 256 * j;
    if (k < K) out[m * K + k] = static_cast<_Float16>(v[j] * s);
  }
  if (threadIdx.x == 0) xinv[m] = ldexpf(1.f, e - 15);
}

// RMSNorm of each row into FP32 `out` and the FP16 row copy the stream GEMM reads (reference
// src/core/stream_gemm.cu:380-418): rstd = 1 / sqrt(sum(x^2) / H + eps), v = x * rstd * w' with w' = 1 + w
// (Gemma) or w, then xh = f16_rn(v * 2^(15 - e)), xinv = 2^(e - 15) from the row's largest |v| (the values
// to_half_rows makes from `out`). One block per row; the FP16 pass recomputes v exactly as the first pass did.
__global__ void __launch_bounds__(256) rmsnorm_half_kernel(const float* __restrict__ x, const uint16_t* __restrict__ w,
                                                           float* __restrict__ out, _Float16* __restrict__ xh,
                                                           float* __restrict__ xinv, int H, float eps, bool gemma) {
  __shared__ float red[4];
  const size_t r = blockIdx.x;
  const float* row = x + r * H;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  float ss = 0.f;
  for (int h = tid; h < H; h += 256) ss += row[h] * row[h];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  if (lane == 0) red[wv] = ss;
  __syncthreads();
  const float tot = (red[0] + red[1]) + (red[2] + red[3]);
  const float rstd = 1.f / sqrtf(tot / static_cast<float>(H) + eps);
  auto val = [&](int h) {
    const float wf = bf16_to_f32(w[h]);
    return row[h] * rstd * (gemma ? 1.f + wf : wf);
  };
  float mx = 0.f;
  for (int h = tid; h < H; h += 256) {
    const float v = val(h);
    out[r * H + h] = v;
    mx = fmaxf(mx, fabsf(v));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  __syncthreads();
  if (lane == 0) red[wv] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int e = 0;
  if (mx > 0.f && isfinite(mx)) frexpf(mx, &e);
  const float sc = ldexpf(1.f, 15 - e);
  for (int h = tid; h < H; h += 256) xh[r * H + h] = static_cast<_Float16>(val(h) * sc);
  if (tid == 0) xinv[r] = ldexpf(1.f, e - 15);
}

// The same with the row and its weights held in registers (NPT values per thread, thread t holding values
// t + 256 j): one read of each, the same sum order (h ascending per thread) and the same arithmetic per element
// as rmsnorm_half_kernel. Rows up to 256 * NPT values.
template <int NPT>
__global__ void __launch_bounds__(256) rmsnorm_half_reg_kernel(const float* __restrict__ x,
                                                               const uint16_t* __restrict__ w, float* __restrict__ out,
                                                               _Float16* __restrict__ xh, float* __restrict__ xinv,
                                                               int H, float eps, bool gemma) {
  __shared__ float red[4];
  const size_t r = blockIdx.x;
  const float* row = x + r * H;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  float v[NPT], wf[NPT];
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int h = tid + 256 * j;
    v[j] = h < H ? row[h] : 0.f;
    wf[j] = h < H ? bf16_to_f32(w[h]) : 0.f;
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NPT; ++j)
    if (tid + 256 * j < H) ss += v[j] * v[j];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  if (lane == 0) red[wv] = ss;
  __syncthreads();
  const float tot = (red[0] + red[1]) + (red[2] + red[3]);
  const float rstd = 1.f / sqrtf(tot / static_cast<float>(H) + eps);
  float mx = 0.f;
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int h = tid + 256 * j;
    if (h < H) {
      v[j] = v[j] * rstd * (gemma ? 1.f + wf[j] : wf[j]);
      out[r * H + h] = v[j];
      mx = fmaxf(mx, fabsf(v[j]));
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  __syncthreads();
  if (lane == 0) red[wv] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int e = 0;
  if (mx > 0.f && isfinite(mx)) frexpf(mx, &e);
  const float sc = ldexpf(1.f, 15 - e);
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int h = tid + 256 * j;
    if (h < H) xh[r * H + h] = static_cast<_Float16>(v[j] * sc);
  }
  if (tid == 0) xinv[r] = ldexpf(1.f, e - 15);
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

// Workgroups per launch: one per CU (a workgroup's four waves fill its SIMDs), a multiple of 8 (one share per
// XCD), never more than the units.
// Depends only on the unit count and the device, never on M (row invariance).
int choose_wgs(long long U) {
  int dev = 0;
  (void)hipGetDevice(&dev);
  long long P = static_cast<long long>(device_cus(dev));
  if (P > U) P = U;
  if (P >= 8) P -= P % 8;
  return static_cast<int>(std::max<long long>(P, 1));
}

#endif  // LQ_STREAM_VGPR_TU

template <int G, int WF, int TW, bool F16, bool PAIR, bool OUTF32, bool CVT>
int launch_g_here(const StreamArgs& a, hipStream_t s) {
  // One matrix (or one pair): its segment is 0 at compile time, so no argument read waits on a computed segment
  // index (about 1 us less before the first weight load). Only the FP16-in, FP32-out entry points take several
  // matrices per launch (stream_gemm_multi); only they also instantiate the general form.
  const dim3 grid(a.P + a.NR * a.TG);
  if constexpr (PAIR) {
    hipLaunchKernelGGL((stream_kernel<G, WF, TW, F16, PAIR, OUTF32, CVT>), grid, dim3(kThreads), 0, s, a);
  } else if constexpr (F16 && OUTF32 && !CVT) {
    if (a.count == 1)
      hipLaunchKernelGGL((stream_kernel<G, WF, TW, F16, PAIR, OUTF32, CVT, true>), grid, dim3(kThreads), 0, s, a);
    else
      hipLaunchKernelGGL((stream_kernel<G, WF, TW, F16, PAIR, OUTF32, CVT>), grid, dim3(kThreads), 0, s, a);
  } else {
    if (a.count != 1) return fail(LQ_ERR_ARG, "stream_gemm: one matrix per launch with BF16 activations or output");
    hipLaunchKernelGGL((stream_kernel<G, WF, TW, F16, PAIR, OUTF32, CVT, true>), grid, dim3(kThreads), 0, s, a);
  }
  return check_launch("stream_gemm");
}

#ifndef LQ_STREAM_VGPR_TU
template <int G, int WF, int TW, bool F16, bool PAIR, bool OUTF32, bool CVT>
int launch_g(const StreamArgs& a, hipStream_t s) {
  if constexpr (vgpr_form(G, WF, TW))
    return launch_g_vgpr<G, WF, TW, F16, PAIR, OUTF32, CVT>(a, s);
  else
    return launch_g_here<G, WF, TW, F16, PAIR, OUTF32, CVT>(a, s);
}

template <int WF, int TW, bool F16, bool PAIR, bool OUTF32, bool CVT>
int launch_mt(const StreamArgs& a, hipStream_t s) {
  switch (cdiv(a.M, 16)) {
    case 1: return launch_g<1, WF, TW, F16, PAIR, OUTF32, CVT>(a, s);
    case 2: return launch_g<2, WF, TW, F16, PAIR, OUTF32, CVT>(a, s);
    case 3: return launch_g<3, WF, TW, F16, PAIR, OUTF32, CVT>(a, s);
    case 4: return launch_g<4, WF, TW, F16, PAIR, OUTF32, CVT>(a, s);
    default: return launch_g<5, WF, TW, F16, PAIR, OUTF32, CVT>(a, s);
  }
}

// Dispatch on the tiles per wave stream_args chose (only FP8 single matrices have a choice).
template <int WF, bool F16, bool PAIR, bool OUTF32, bool CVT = false>
int launch_m(const StreamArgs& a, hipStream_t s) {
  if constexpr (WF == kFp8 && !PAIR) {
    if (a.T == 1) return launch_mt<WF, 1, F16, PAIR, OUTF32, CVT>(a, s);
  }
  return launch_mt<WF, tiles_per_wave(WF, PAIR), F16, PAIR, OUTF32, CVT>(a, s);
}

// Validates, fills the launch arguments and launches. `fmt`: weight format; `f16`: activations are an
// FP16 row copy (with xinv) rather than BF16; `pair`: mats = {gate, up} with the SiLU*mul epilogue.
std::atomic<int> g_finish_wait_ms{1000};  // StreamArgs::wait_ms of later launches (lq_debug_finish_wait_ms)
#ifdef LQ_STREAM_TRACE
unsigned long long* g_trace = nullptr;  // device buffer of P x 8 stamps for the next launches
#endif

// FP32 floats of one partial slot (one workgroup's T x G accumulator vectors for 256 threads).
size_t slot_floats(int T, int M) { return static_cast<size_t>(T) * cdiv(M, 16) * 4 * kThreads; }

// Tiles per wave, tile groups and workgroups of one matrix (or one SiLU*mul pair) launched alone. One FP8 tile per
// wave when a workgroup's range would be short (under 10 chunks at two tiles) and a tile group would span six
// workgroups or more: there the finish dominates, and one tile per wave halves its fan-in and partial size. A lower
// fan-in does not pay for the activations one tile per wave stages per weight byte (twice as many): 7168 x 5120
// (fan-in 4.6) is 2 % slower over the M = 68 decode-step pass with one tile, 5120 x 6144 (fan-in 6) 3-6 % faster at
// M = 17..68. Depends on the matrix's N, K and the device only, never on M (row invariance).
void matrix_split(int fmt, bool pair, int N, int C, int& T, int& tg, int& P) {
  T = tiles_per_wave(fmt, pair);
  auto go = [&]() {
    tg = cdiv(N, group_rows(T, pair));
    P = choose_wgs(static_cast<long long>(tg) * C);
    // Whole tile groups per workgroup count: where that idles at most 1/16 of the workgroups, P is rounded down to a
    // multiple of tg, so every tile group is split over the same number of workgroups and none of them finishes
    // two tile groups (measured, FP8 at M = 1..68: 3-7 % faster where it applies, e.g. 5120 x 6144 at M = 17
    // 16.1 -> 15.0 us; the M = 68 decode-step pass 8.30 -> 8.05 ms).
    if (!pair && P >= 3 * tg && (P % tg) * 16 <= P) P -= P % tg;
  };
  go();
  if (fmt == kFp8 && !pair && static_cast<long long>(tg) * C < 10LL * P && P > 5 * tg) {
    T = 1;
    go();
  }
}

// The segments of a launch (sets a.T, a.TG, a.P, tg0, wg0): each matrix (a pair: both) split as it would be alone,
// its workgroups after the previous matrix's. Returns kMixedTiles (nothing set) when the matrices want different
// tiles per wave: the caller then launches them in groups.
constexpr int kMixedTiles = -1;  // (distinct from every LQ_ERR_* status)
int choose_tiles(const char* name, int fmt, bool pair, const int* Ns, int n, StreamArgs& a) {
  const int nseg = pair ? 1 : n;
  int T0 = -1, tgs = 0, wgs = 0;
  for (int i = 0; i < nseg; ++i) {
    int T, tg, P;
    matrix_split(fmt, pair, Ns[i], a.C, T, tg, P);
    if (T0 >= 0 && T != T0) return kMixedTiles;
    T0 = T;
    if (static_cast<long long>(tg) * a.C * (P + 1) >= (1LL << 31) || tgs + static_cast<long long>(tg) >= (1LL << 30))
      return fail(LQ_ERR_SHAPE, std::string(name) + ": matrices too large for one launch");
    // the kernels address a weight blob and the activations with 32-bit byte offsets
    const long long blk = fmt == kFp8 ? kTileBytesFp8 : fmt == kFp4 ? kTileBytesFp4 : kValueBytesFp4 + kCodeBytesFp4;
    if (static_cast<long long>(Ns[i] / 16) * a.C * blk >= (1LL << 31) ||
        static_cast<long long>(a.M) * a.C * kChunk * 2 >= (1LL << 31))
      return fail(LQ_ERR_SHAPE, std::string(name) + ": weight blob and activations must be below 2^31 bytes");
    a.tg0[i] = tgs;
    a.wg0[i] = wgs;
    tgs += tg;
    wgs += P;
  }
  if (pair) a.tg0[1] = 0;
  a.tg0[pair ? 2 : n] = tgs;
  a.wg0[nseg] = wgs;
  a.T = T0;
  a.TG = tgs;
  a.P = wgs;
  return LQ_OK;
}

// Validates and fills the launch arguments except the workspace pointers.
int stream_args(const char* name, int fmt, bool f16, bool pair, bool outf32, const void* x, const float* xinv, int M,
                const Mat* mats, int n, int K, StreamArgs& a) {
  const std::string nm(name);
  if (K <= 0 || K % kChunk != 0) return fail(LQ_ERR_SHAPE, nm + ": K must be a multiple of 128");
  if (M < 1 || M > LQ_MAX_STREAM_ROWS) return fail(LQ_ERR_SHAPE, nm + ": M must be in [1, 80]");
  if (n < 1 || n > kMaxMats) return fail(LQ_ERR_SHAPE, nm + ": 1 to 4 matrices per launch");
  if (!x) return fail(LQ_ERR_ARG, nm + ": null activations");
  if (f16 && !xinv) return fail(LQ_ERR_ARG, nm + ": null xinv");
  a = StreamArgs{};
  a.x = x;
  a.xinv = xinv;
  a.M = M;
  a.K = K;
  a.C = K / kChunk;
  a.count = static_cast<short>(n);
  int Ns[kMaxMats];
  for (int i = 0; i < n; ++i) {
    const Mat& m = mats[i];
    if (m.N <= 0 || m.N % 16 != 0) return fail(LQ_ERR_SHAPE, nm + ": N % 16 and K % 128 must be 0");
    if (!m.w || !m.y) return fail(LQ_ERR_ARG, nm + ": null weight or output");
    if (fmt == kFp4Coded && !m.table) return fail(LQ_ERR_ARG, nm + ": null scale-code table");
    // the epilogue reads 4 channels' scales as one 16-byte load and writes 4 outputs as one 8- or 16-byte store
    if (reinterpret_cast<uintptr_t>(m.svec) % 16 != 0 || reinterpret_cast<uintptr_t>(m.y) % (outf32 ? 16 : 8) != 0 ||
        reinterpret_cast<uintptr_t>(m.resid) % 8 != 0 || m.ldy % 4 != 0)
      return fail(LQ_ERR_ARG, nm + ": scales must be 16-byte aligned, outputs and residual 8-byte aligned");
    a.w[i] = m.w;
    a.table[i] = m.table;
    a.svec[i] = m.svec;
    a.sc[i] = m.sc;
    a.y[i] = m.y;
    a.resid[i] = m.resid;
    a.N[i] = m.N;
    a.ldy[i] = m.ldy;
    Ns[i] = m.N;
  }
  if (pair && (n != 2 || mats[0].N != mats[1].N)) return fail(LQ_ERR_SHAPE, nm + ": gate and up must have the same N");
  if (!pair && fmt != kFp8 && !f16 && outf32) return fail(LQ_ERR_ARG, nm + ": BF16 activations with NVFP4 give BF16 out");
  return choose_tiles(name, fmt, pair, Ns, n, a);  // (kMixedTiles: the matrices want different tiles per wave)
}

// Finish workgroups when a finisher's reads would be long: a tile group spans three workgroups or more (so all
// are split) and its partials hold (P / TG + 1) x T x G >= 24 vectors per thread. They start only as streaming
// workgroups leave their CUs (a streaming workgroup's registers fill its CU) and see the count a memory round
// trip later, about 2 us after the last arrival, which pays off only when one finisher's reads take longer.
// Measured (graph-timed, FP8 with residual): down 5120 x 17408 gains 4 % at M = 17 and 3 % at M = 33 (28
// vectors), 13 % at M = 68; the NVFP4 25600-wide fc at M = 16 2 %. A threshold of 16 also takes K = 6144 at
// M = 68 (20 vectors, 12 % slower) and 1024-wide matrices at M = 1 (8 % slower). The results are the same either
// way.
bool finish_wgs(const StreamArgs& a) {
  const int G = cdiv(a.M, 16);
  return a.P >= 3 * a.TG && (a.P / a.TG + 1) * a.T * G >= 24;
}

// Arrival counters one 128-byte line apart (a stride of 32 ints) when the counter memory holds them that way, else
// packed: the arrivals of every workgroup land on the counters at about the same time, and atomics on one line are
// performed one after another (measured: the M = 17 down projection's tail). kOwnCounters: what lq_init reserves in
// the library's own workspace.
constexpr size_t kOwnCounters = size_t(1) << 20;
int counter_stride(size_t n, size_t capacity) { return n * 32 <= capacity ? 32 : 1; }

// A fixed scratch region in place of the workspace (the no-allocation entry point): partials and counters, with
// their capacities; the launch is rejected when it needs more.
struct FixedScratch {
  float* partials;
  size_t partial_bytes;
  int* counters;
  size_t counter_count;
};

int stream_launch(const char* name, int fmt, bool f16, bool pair, bool outf32, const void* x, const float* xinv, int M,
                  const Mat* mats, int n, int K, hipStream_t s, const FixedScratch* fixed = nullptr) {
  StreamArgs a;
  int rc = stream_args(name, fmt, f16, pair, outf32, x, xinv, M, mats, n, K, a);
  if (rc == kMixedTiles) {
    // matrices that want different tiles per wave: one launch per group of equal T, each matrix split as alone
    for (int T : {1, 2, 4}) {
      Mat sub[kMaxMats];
      int k = 0;
      for (int i = 0; i < n; ++i) {
        int Ti, tg, P;
        matrix_split(fmt, false, mats[i].N, K / kChunk, Ti, tg, P);
        if (Ti == T) sub[k++] = mats[i];
      }
      if (k && (rc = stream_launch(name, fmt, f16, pair, outf32, x, xinv, M, sub, k, K, s, fixed))) return rc;
    }
    return LQ_OK;
  }
  if (rc) return rc;
  a.NR = static_cast<short>(finish_wgs(a) ? kFinishShares : 0);
  a.wait_ms = static_cast<short>(g_finish_wait_ms.load(std::memory_order_relaxed));
  const size_t nc = static_cast<size_t>(a.TG) * (a.NR ? 2 : 1);
  const size_t pbytes = 2 * static_cast<size_t>(a.P) * slot_floats(a.T, M) * sizeof(float);
  a.cs = static_cast<short>(counter_stride(nc, fixed ? fixed->counter_count : kOwnCounters));
  const size_t ncnt = nc * a.cs;
  if (fixed) {
    if (pbytes > fixed->partial_bytes || ncnt > fixed->counter_count)
      return fail(LQ_ERR_SHAPE, std::string(name) + ": the launch needs " + std::to_string(pbytes) +
                                    " bytes of partial sums and " + std::to_string(ncnt) +
                                    " counters; the fixed scratch holds " + std::to_string(fixed->partial_bytes) +
                                    " and " + std::to_string(fixed->counter_count));
    a.partials = fixed->partials;
    a.counters = fixed->counters;
  } else {
    Workspace* ws = workspace_for_current_device();
    if (!ws) return LQ_ERR_DEVICE;
    rc = ws->reserve_stream(pbytes, ncnt);
    if (rc) return rc;
    a.partials = ws->partials;
    a.counters = ws->counters;
  }
#ifdef LQ_STREAM_TRACE
  a.trace = g_trace;
#endif
  if (pair) return f16 ? launch_m<kFp8, true, true, false>(a, s) : launch_m<kFp8, false, true, false>(a, s);
  if (fmt == kFp8) {
    if (f16) return outf32 ? launch_m<kFp8, true, false, true>(a, s) : launch_m<kFp8, true, false, false>(a, s);
    return outf32 ? launch_m<kFp8, false, false, true>(a, s) : launch_m<kFp8, false, false, false>(a, s);
  }
  // NVFP4 runs on the FP16 MFMA: BF16 activations are converted chunk by chunk in the kernel
  if (!f16) return fmt == kFp4 ? launch_m<kFp4, true, false, false, true>(a, s)
                               : launch_m<kFp4Coded, true, false, false, true>(a, s);
  if (fmt == kFp4) return outf32 ? launch_m<kFp4, true, false, true>(a, s) : launch_m<kFp4, true, false, false>(a, s);
  return outf32 ? launch_m<kFp4Coded, true, false, true>(a, s) : launch_m<kFp4Coded, true, false, false>(a, s);
}

// The FFN step (gate|up + SiLU*mul into h, down + residual into y) as one launch when both phases get the same
// number of workgroups, else as the two launches it equals bit for bit.
int ffn_launch(const char* name, const uint16_t* x, int M, const Mat (&gu)[2], const Mat& dn, const uint16_t* h,
               hipStream_t s) {
  StreamArgs a, b;
  int rc = stream_args(name, kFp8, false, true, false, x, nullptr, M, gu, 2, dn.N, a);
  if (rc) return rc;
  rc = stream_args(name, kFp8, false, false, false, h, nullptr, M, &dn, 1, gu[0].N, b);
  if (rc) return rc;
  // (the one-launch form runs both phases at two tiles per wave, phase B on at most phase A's workgroups)
  if (b.P > a.P || a.T != 2 || b.T != 2) {
    rc = stream_launch(name, kFp8, false, true, false, x, nullptr, M, gu, 2, dn.N, s);
    return rc ? rc : stream_launch(name, kFp8, false, false, false, h, nullptr, M, &dn, 1, gu[0].N, s);
  }
  Workspace* ws = workspace_for_current_device();
  if (!ws) return LQ_ERR_DEVICE;
  const size_t fa = 2 * static_cast<size_t>(a.P) * slot_floats(a.T, M);
  const size_t fb = 2 * static_cast<size_t>(b.P) * slot_floats(b.T, M);
  a.cs = b.cs = static_cast<short>(counter_stride(static_cast<size_t>(a.TG) + b.TG, ws->external ? ws->counter_count : kOwnCounters));
  rc = ws->reserve_stream((fa + fb) * sizeof(float), (static_cast<size_t>(a.TG) + b.TG) * a.cs);
  if (rc) return rc;
  a.partials = ws->partials;
  a.counters = ws->counters;
  b.partials = ws->partials + fa;
  b.counters = ws->counters + static_cast<size_t>(a.TG) * a.cs;
#ifdef LQ_STREAM_TRACE
  a.trace = g_trace;
  b.trace = g_trace ? g_trace + 16 * static_cast<size_t>(a.P) : nullptr;
#endif
  switch (cdiv(M, 16)) {
    case 1: launch_ffn_vgpr<1>(a, b, ws->sync, s); break;
    case 2: launch_ffn_vgpr<2>(a, b, ws->sync, s); break;
    case 3: launch_ffn_vgpr<3>(a, b, ws->sync, s); break;
    case 4: launch_ffn_vgpr<4>(a, b, ws->sync, s); break;
    default: hipLaunchKernelGGL(ffn_kernel<5>, dim3(a.P), dim3(kThreads), 0, s, a, b, ws->sync); break;
  }
  return check_launch(name);
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
  // rows of up to 32768 values: one block per row, the row in registers
  auto reg = [&](auto npt) {
    constexpr int NPT = decltype(npt)::value;
    if (bf16in)
      hipLaunchKernelGGL((half_rows_reg_kernel<true, NPT>), dim3(M), dim3(256), 0, s, x, K,
                         reinterpret_cast<_Float16*>(xh), xinv);
    else
      hipLaunchKernelGGL((half_rows_reg_kernel<false, NPT>), dim3(M), dim3(256), 0, s, x, K,
                         reinterpret_cast<_Float16*>(xh), xinv);
    return check_launch(nm);
  };
  if (K <= 1024) return reg(std::integral_constant<int, 4>{});
  if (K <= 2048) return reg(std::integral_constant<int, 8>{});
  if (K <= 4096) return reg(std::integral_constant<int, 16>{});
  if (K <= 8192) return reg(std::integral_constant<int, 32>{});
  if (K <= 16384) return reg(std::integral_constant<int, 64>{});
  if (K <= 32768) return reg(std::integral_constant<int, 128>{});
  const int split = std::max(1, std::min(K / 1024, cdiv(192, M)));
  const int slice = cdiv(K, split);
  const dim3 grid(M, cdiv(K, slice));
  if (bf16in)
    hipLaunchKernelGGL(half_rows_kernel<true>, grid, dim3(256), 0, s, x, K, slice, reinterpret_cast<_Float16*>(xh), xinv);
  else
    hipLaunchKernelGGL(half_rows_kernel<false>, grid, dim3(256), 0, s, x, K, slice, reinterpret_cast<_Float16*>(xh), xinv);
  return check_launch(nm);
}

__global__ void __launch_bounds__(256) zero_ints_kernel(int* p, int n) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0;
}

}  // namespace
}  // namespace lq

// ---------------- the no-allocation entry point's scratch ----------------
// lq_stream_fp8_pc_noalloc keeps its split-K partial sums and arrival counters in this file-scope device array
// instead of the library's workspace: 25 MiB of partials (two slots per workgroup at up to 320 workgroups, one per CU,
// two tiles per wave and five row groups: M <= 80, on devices of up to 320 CUs) and 64 Ki counters. Every GPU the library runs on holds its own copy until the
// process ends. Host code never passes the array's name to a kernel (on the host it is only a stand-in): its
// device address is looked up once per device (noalloc_scratch) and that address is used.
constexpr size_t kScratchPartialBytes = size_t(25) << 20;  // 2 x 320 x 40 KiB
constexpr size_t kScratchCounters = size_t(1) << 16;
static __device__ __align__(256) unsigned char scratch[kScratchPartialBytes + 4 * kScratchCounters];

namespace lq {
namespace {
std::mutex g_scratch_mutex;
constexpr int kScratchDevices = 64;
unsigned char* g_scratch_ptr[kScratchDevices] = {};
bool g_scratch_zeroed[kScratchDevices] = {};

// The current device's scratch address (looked up on the first call per device), with its counters cleared once:
// by lq_init (synchronously), or else by a fill kernel on `s` ahead of the first launch (captured into a graph if
// the first call is captured). The counters are zero again at the end of every launch.
int noalloc_scratch(hipStream_t s, bool sync, FixedScratch& fs) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchDevices)
    return fail(LQ_ERR_DEVICE, "stream_fp8_pc_noalloc: no current device");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(LQ_ERR_DEVICE, std::string("stream_fp8_pc_noalloc: scratch address lookup failed: ") +
                                     hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<unsigned char*>(p);
  }
  fs.partials = reinterpret_cast<float*>(g_scratch_ptr[dev]);
  fs.partial_bytes = kScratchPartialBytes;
  fs.counters = reinterpret_cast<int*>(g_scratch_ptr[dev] + kScratchPartialBytes);
  fs.counter_count = kScratchCounters;
  if (!g_scratch_zeroed[dev]) {
    hipLaunchKernelGGL(zero_ints_kernel, dim3(64), dim3(256), 0, s, fs.counters, static_cast<int>(kScratchCounters));
    if (int rc = check_launch("stream_fp8_pc_noalloc")) return rc;
    if (sync && hipStreamSynchronize(s) != hipSuccess)
      return fail(LQ_ERR_DEVICE, "stream_fp8_pc_noalloc: clearing the scratch counters failed");
    g_scratch_zeroed[dev] = true;
  }
  return LQ_OK;
}
}  // namespace

int noalloc_init_current_device() {
  FixedScratch fs;
  return noalloc_scratch(nullptr, true, fs);
}
}  // namespace lq

using namespace lq;

extern "C" {

// Test hook (not part of the interface): the finish workgroups' wait limit for later launches, in milliseconds
// (default 1000; 0 makes every finish workgroup give up without waiting, so tests reach the expired-wait path
// deterministically without a stalled GPU). Returns the previous limit, or -1 for a value outside [0, 32767].
int lq_debug_finish_wait_ms(int ms) {
  if (ms < 0 || ms > 32767) return -1;
  return g_finish_wait_ms.exchange(ms);
}

#ifdef LQ_STREAM_TRACE
// Trace builds only: stream launches record per-workgroup phase stamps into `buf` ([P][8] u64, device).
int lq_debug_stream_trace(unsigned long long* buf) {
  g_trace = buf;
  return LQ_OK;
}
#endif

int lq_to_half_rows(const float* x, int M, int K, uint16_t* xh, float* xinv, void* stream) {
  return half_rows(false, x, M, K, xh, xinv, static_cast<hipStream_t>(stream));
}

int lq_bf16_to_half_rows(const uint16_t* x, int M, int K, uint16_t* xh, float* xinv, void* stream) {
  return half_rows(true, x, M, K, xh, xinv, static_cast<hipStream_t>(stream));
}

int lq_rmsnorm_half(const float* x, const uint16_t* w, float* out, uint16_t* xh, float* xinv, int rows, int H, float eps,
                    int gemma, void* stream) {
  if (rows < 1 || H < 1) return fail(LQ_ERR_SHAPE, "rmsnorm_half: rows and H must be positive");
  if (!x || !w || !out || !xh || !xinv) return fail(LQ_ERR_ARG, "rmsnorm_half: null pointer");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  _Float16* const xh16 = reinterpret_cast<_Float16*>(xh);
  // rows of up to 8192 values: the row and its weights in registers
  if (H <= 1024) hipLaunchKernelGGL(rmsnorm_half_reg_kernel<4>, dim3(rows), dim3(256), 0, s, x, w, out, xh16, xinv, H, eps, gemma != 0);
  else if (H <= 2048) hipLaunchKernelGGL(rmsnorm_half_reg_kernel<8>, dim3(rows), dim3(256), 0, s, x, w, out, xh16, xinv, H, eps, gemma != 0);
  else if (H <= 4096) hipLaunchKernelGGL(rmsnorm_half_reg_kernel<16>, dim3(rows), dim3(256), 0, s, x, w, out, xh16, xinv, H, eps, gemma != 0);
  else if (H <= 8192) hipLaunchKernelGGL(rmsnorm_half_reg_kernel<32>, dim3(rows), dim3(256), 0, s, x, w, out, xh16, xinv, H, eps, gemma != 0);
  else hipLaunchKernelGGL(rmsnorm_half_kernel, dim3(rows), dim3(256), 0, s, x, w, out, xh16, xinv, H, eps, gemma != 0);
  return check_launch("rmsnorm_half");
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

int lq_stream_fp8_pc_noalloc(const uint16_t* x, int M, const uint8_t* w, const float* wscale_n, uint16_t* y, int N,
                             int K, void* stream) {
  if (int rc = check_rows("stream_fp8_pc_noalloc", M, N, K)) return rc;
  if (!wscale_n) return fail(LQ_ERR_ARG, "stream_fp8_pc_noalloc: null scales");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  FixedScratch fs;
  if (int rc = noalloc_scratch(s, false, fs)) return rc;
  const Mat m{w, nullptr, wscale_n, 0.f, y, nullptr, N, N};
  return stream_launch("stream_fp8_pc_noalloc", kFp8, false, false, false, x, nullptr, M, &m, 1, K, s, &fs);
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

int lq_stream_fp8_pc_ffn(const uint16_t* x, int M, const uint8_t* w_gate, const float* s_gate, const uint8_t* w_up,
                         const float* s_up, const uint8_t* w_down, const float* s_down, const uint16_t* resid,
                         uint16_t* h, uint16_t* y, int I, int H, void* stream) {
  if (int rc = check_rows("stream_fp8_pc_ffn", M, I, H)) return rc;
  if (int rc = check_rows("stream_fp8_pc_ffn", M, H, I)) return rc;
  if (!s_gate || !s_up || !s_down || !resid || !h) return fail(LQ_ERR_ARG, "stream_fp8_pc_ffn: null scales, residual or h");
  const Mat gu[2] = {{w_gate, nullptr, s_gate, 0.f, h, nullptr, I, I}, {w_up, nullptr, s_up, 0.f, h, nullptr, I, I}};
  const Mat dn{w_down, nullptr, s_down, 0.f, y, resid, H, H};
  return ffn_launch("stream_fp8_pc_ffn", x, M, gu, dn, h, static_cast<hipStream_t>(stream));
}

int lq_stream_gemm_gather_nvfp4(const uint16_t* xh, const float* xinv, int M, const uint8_t* w,
                                const uint8_t* raw_scales, float scale2, const int* rows, const int* nrows, int cap,
                                float* y, int K, int N, void* stream) {
  const std::string nm = "stream_gemm_gather";
  if (K <= 0 || K % kChunk != 0 || cap <= 0 || cap % 32 != 0)
    return fail(LQ_ERR_SHAPE, nm + ": K % 128 and cap % 32 must be 0");
  if (M < 1 || M > LQ_MAX_STREAM_ROWS) return fail(LQ_ERR_SHAPE, nm + ": M must be in [1, 80]");
  if (N <= 0 || N % 16 != 0) return fail(LQ_ERR_SHAPE, nm + ": N % 16 and K % 128 must be 0");
  // the kernel addresses the blob and the activations with 32-bit byte offsets (bit 31 marks a read out of range)
  if (static_cast<long long>(N / 16) * (K / kChunk) * kTileBytesFp4 >= (1LL << 31) ||
      static_cast<long long>(M) * K * 2 >= (1LL << 31))
    return fail(LQ_ERR_SHAPE, nm + ": weight blob and activations must be below 2^31 bytes");
  if (!xh || !xinv || !w || !rows || !nrows || !y) return fail(LQ_ERR_ARG, nm + ": null pointer");
  GatherArgs a{};
  a.x = xh;
  a.xinv = xinv;
  a.M = M;
  a.K = K;
  a.C = K / kChunk;
  a.w = w;
  a.raw = raw_scales;
  a.scale2 = scale2;
  a.rows = rows;
  a.nrows = nrows;
  a.cap = cap;
  a.N = N;
  a.y = y;
  // the full launch's split (the matrix alone): its tiles per wave, tile groups, workgroups and units
  int fT, ftg, fP;
  matrix_split(kFp4, false, N, a.C, fT, ftg, fP);
  a.TGR = group_rows(fT, false);
  a.P = fP;
  a.U = ftg * a.C;
  if (a.U >= (1 << 19) || (static_cast<long long>(a.U) + 1) * (a.P + 1) >= (1LL << 31))
    return fail(LQ_ERR_SHAPE, nm + ": too many units for the gather's split arithmetic");
  const dim3 grid(cap / 16), blk(kGatherThreads);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  // one token group per workgroup row; a single token takes the one-row form
  if (M == 1)
    hipLaunchKernelGGL((gather_kernel<1, true>), grid, blk, 0, s, a);
  else
    hipLaunchKernelGGL((gather_kernel<1, false, true>), dim3(cap / 16, cdiv(M, 16)), blk, 0, s, a);
  return check_launch("stream_gemm_gather");
}

int lq_l2_prefetch_weights(const uint8_t* w, int fp4, int coded, int N, int K, size_t bytes, void* stream) {
  if (!w || bytes == 0) return LQ_OK;  // as the reference: nothing asked, nothing done
  if (N <= 0 || N % 16 != 0 || K <= 0 || K % kChunk != 0)
    return fail(LQ_ERR_SHAPE, "l2_prefetch_weights: N % 16 and K % 128 must be 0");
  const int fmt = fp4 ? (coded ? kFp4Coded : kFp4) : kFp8;
  const int C = K / kChunk, tiles = N / 16;
  int T, tg, P;
  matrix_split(fmt, false, N, C, T, tg, P);
  const int tpg = group_rows(T, false) / 16;
  const int blk = fmt == kFp8 ? kTileBytesFp8 : fmt == kFp4 ? kTileBytesFp4 : kValueBytesFp4;
  const long long per_round = static_cast<long long>(P) * tpg * (blk + (coded && fp4 ? kCodeBytesFp4 : 0));
  const long long want = static_cast<long long>(bytes) / per_round;
  const int nc = static_cast<int>(std::min<long long>(C, std::max<long long>(1, want)));
  const long long code_base = fmt == kFp4Coded ? static_cast<long long>(tiles) * C * kValueBytesFp4 : -1;
  hipLaunchKernelGGL(prefetch_units_kernel, dim3(P), dim3(256), 0, static_cast<hipStream_t>(stream), w, C, P,
                     tg * C, tpg, tiles, blk, code_base, nc);
  return check_launch("l2_prefetch_weights");
}

int lq_stream_ffn_deadline_status(int* hit) {
  if (!hit) return fail(LQ_ERR_ARG, "stream_ffn_deadline_status: null pointer");
  Workspace* ws = workspace_for_current_device();
  if (!ws) return LQ_ERR_DEVICE;
  *hit = 0;
  // reading clears the flags: a later report names only launches after this one
  const int zero = 0;
  if (ws->sync) {
    if (hipMemcpy(hit, ws->sync + 2, sizeof(int), hipMemcpyDeviceToHost) != hipSuccess)
      return fail(LQ_ERR_DEVICE, "stream_ffn_deadline_status: copy failed");
    if (*hit && hipMemcpy(ws->sync + 2, &zero, sizeof(int), hipMemcpyHostToDevice) != hipSuccess)
      return fail(LQ_ERR_DEVICE, "stream_ffn_deadline_status: clear failed");
  }
  int fin = 0;  // a finish workgroup's wait
  if (hipMemcpyFromSymbol(&fin, HIP_SYMBOL(g_wait_expired), sizeof(int)) != hipSuccess)
    return fail(LQ_ERR_DEVICE, "stream_ffn_deadline_status: copy failed");
  if (fin && hipMemcpyToSymbol(HIP_SYMBOL(g_wait_expired), &zero, sizeof(int)) != hipSuccess)
    return fail(LQ_ERR_DEVICE, "stream_ffn_deadline_status: clear failed");
  *hit = *hit || fin;
  return LQ_OK;
}

int lq_stream_nvfp4_bf16(const uint16_t* x, int M, const uint8_t* w, const uint8_t* table, float scale2, uint16_t* y,
                         int N, int K, void* stream) {
  if (int rc = check_rows("stream_nvfp4_bf16", M, N, K)) return rc;
  const Mat m{w, table, nullptr, scale2, y, nullptr, N, N};
  return stream_launch("stream_nvfp4_bf16", table ? kFp4Coded : kFp4, false, false, false, x, nullptr, M, &m, 1, K,
                       static_cast<hipStream_t>(stream));
}

}  // extern "C"

#else  // LQ_STREAM_VGPR_TU: the FP8 kernels vgpr_form selects, compiled with VGPR accumulators

}  // namespace

template <int G, int WF, int TW, bool F16, bool PAIR, bool OUTF32, bool CVT>
int launch_g_vgpr(const StreamArgs& a, hipStream_t s) {
  return launch_g_here<G, WF, TW, F16, PAIR, OUTF32, CVT>(a, s);
}

template <int G>
void launch_ffn_vgpr(const StreamArgs& a, const StreamArgs& b, int* sync, hipStream_t s) {
  hipLaunchKernelGGL(ffn_kernel<G>, dim3(a.P), dim3(kThreads), 0, s, a, b, sync);
}
template void launch_ffn_vgpr<1>(const StreamArgs&, const StreamArgs&, int*, hipStream_t);
template void launch_ffn_vgpr<2>(const StreamArgs&, const StreamArgs&, int*, hipStream_t);
template void launch_ffn_vgpr<3>(const StreamArgs&, const StreamArgs&, int*, hipStream_t);
template void launch_ffn_vgpr<4>(const StreamArgs&, const StreamArgs&, int*, hipStream_t);

// every launch the main translation unit routes here: single matrices (BF16 or FP16 activations, BF16 or FP32
// output) at one or two tiles per wave, SiLU*mul pairs at two (two tiles only up to four token groups)
#define LQ_VGPR_SINGLE(G, TW)                                                                       \
  template int launch_g_vgpr<G, kFp8, TW, false, false, false, false>(const StreamArgs&, hipStream_t); \
  template int launch_g_vgpr<G, kFp8, TW, false, false, true, false>(const StreamArgs&, hipStream_t);  \
  template int launch_g_vgpr<G, kFp8, TW, true, false, false, false>(const StreamArgs&, hipStream_t);  \
  template int launch_g_vgpr<G, kFp8, TW, true, false, true, false>(const StreamArgs&, hipStream_t);
#define LQ_VGPR_PAIR(G)                                                                            \
  template int launch_g_vgpr<G, kFp8, 2, false, true, false, false>(const StreamArgs&, hipStream_t); \
  template int launch_g_vgpr<G, kFp8, 2, true, true, false, false>(const StreamArgs&, hipStream_t);
LQ_VGPR_SINGLE(1, 1) LQ_VGPR_SINGLE(2, 1) LQ_VGPR_SINGLE(3, 1) LQ_VGPR_SINGLE(4, 1) LQ_VGPR_SINGLE(5, 1)
LQ_VGPR_SINGLE(1, 2) LQ_VGPR_SINGLE(2, 2) LQ_VGPR_SINGLE(3, 2) LQ_VGPR_SINGLE(4, 2)
LQ_VGPR_PAIR(1) LQ_VGPR_PAIR(2) LQ_VGPR_PAIR(3) LQ_VGPR_PAIR(4)
static_assert(vgpr_form(4, kFp8, 2) && vgpr_form(5, kFp8, 1) && !vgpr_form(5, kFp8, 2) && !vgpr_form(1, kFp4, 4),
              "the instantiations above cover vgpr_form");
}  // namespace lq
#endif  // LQ_STREAM_VGPR_TU
