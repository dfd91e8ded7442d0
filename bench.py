"""Benchmark of the fused quantized GEMM path on one MI355X.

Headline metric: the speculative-verify MLP at M = 17 rows (config 2): gate|up
(K = 5120, N = 2 x 17408, FP8 per-channel) with the SiLU*mul epilogue, then down (K = 17408, N = 5120) with the
BF16 residual add. A step is one such pass (two launches); `value` is algorithmic HBM bytes per second of the whole
step (the same pass as the one-launch FFN kernel is reported beside it).
Weights rotate over copies totalling >= 1 GB so neither L2 nor the 256 MB MALL serves the next step's weights.
Inputs are synthetic and follow the configs' recipes: activations N(0, 1) in BF16; weights N(0, 0.02) quantized by the
library's host quantizers (FP8 with one scale per output channel, NVFP4 round-to-nearest, FP8 in 128 x 128 blocks for
the prefill, whose activations the device quantizer groups 1 x 128). Rotation copies are device clones of one matrix
per role (distinct addresses, so no cache serves the next step's weights).

Also reported beside it (same JSON line): decode M = 1 (config 1), the NVFP4 drafter fc (config 3), the full M = 68
decode-step weight pass (config 5), and the block-scaled prefill GEMM at M = 4096 (config 4) in TFLOP/s.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "ling-engine_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, published
FP8_DENSE_TFLOPS = 5000.0   # MI355X dense FP8 MFMA, published (no sparsity)
ROTATE_BYTES = 1 << 30


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--only", default="", help="comma list of extra sections to run (default: all)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--vendor-reference", action="store_true",
                    help="also time hipBLASLt's per-tensor FP8 GEMM (torch._scaled_mm) on the config-4 shapes, for comparison")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a 1 GiB device copy (the known-size kernel that scales HBM byte counters)")
    return ap.parse_args()


class Timer:
    """HIP events on the current stream around individual launches."""

    def __init__(self, torch, n):
        self.torch = torch
        self.ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
        self.i = 0

    def start(self):
        self.ev[self.i][0].record()

    def stop(self):
        self.ev[self.i][1].record()
        self.i += 1

    def mean_ms(self):
        return sum(a.elapsed_time(b) for a, b in self.ev[:self.i]) / max(1, self.i)


PREFILL_WARM_S = 2.0


def warm_until(torch, fn, seconds=None):
    """Runs fn in batches of 10 launches until `seconds` (PREFILL_WARM_S) of wall time have passed, then syncs."""
    seconds = PREFILL_WARM_S if seconds is None else seconds
    t0 = time.time()
    while True:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
        if time.time() - t0 >= seconds:
            return


_WCACHE = {}


def fp8_weight(torch, L, N, K, seed, dev):
    """A weight of the configs' data: W ~ N(0, 0.02) (numpy's generator, seeded), quantized to FP8 E4M3 with one
    FP32 scale per output channel by the library's host quantizer (amax / 448, the benchmark recipe), in the tiled
    layout. One quantized matrix per (N, K, seed % 1000); further copies are device clones (distinct addresses, so
    the rotation still defeats the caches)."""
    import numpy as np
    key = (N, K, seed % 1000)
    if key not in _WCACHE:
        w = (np.random.default_rng(seed % 1000).standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
        q, s = L.quantize_fp8_channel(w)
        del w
        _WCACHE[key] = (L.retile_fp8(torch.from_numpy(q).to(dev)), torch.from_numpy(s).to(dev))
        del q
    tw, s = _WCACHE[key]
    return tw.clone(), s.clone()


def drop_weight_cache(torch):
    _WCACHE.clear()
    torch.cuda.empty_cache()


def graph_per_launch_ms(torch, fn, copies, per_graph=None, replays=10):
    """Mean time per launch of fn(i) with the launches captured in one HIP graph (per_graph launches rotating over
    `copies`), replayed `replays` times: the GPU's time, without the host's per-call dispatch cost."""
    per_graph = per_graph or max(copies, 20)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(per_graph):
            fn(i % copies)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(per_graph):
            fn(i % copies)
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(replays):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / (replays * per_graph)


def bench_verify_mlp(torch, L, O, args, dev):
    """Config 2: M = 17; the step as two launches, the same step as one FFN launch, and the gate|up kernel alone."""
    import numpy as np
    M, H, F = 17, 5120, 17408
    per_set = 2 * F * H + H * F
    copies = max(2, -(-ROTATE_BYTES // per_set))
    log(f"[bench] verify MLP M={M}: {copies} weight copies x {per_set / 1e6:.1f} MB")
    sets = []
    for c in range(copies):
        wg, sg = fp8_weight(torch, L, F, H, 100, dev)
        wu, su = fp8_weight(torch, L, F, H, 101, dev)
        wd, sd = fp8_weight(torch, L, H, F, 102, dev)
        sets.append((wg, sg, wu, su, wd, sd))
    x = torch.from_numpy(O.normal_bf16(0x4C510002, 1.0, (M, H)).view(np.int16)).to(dev).view(torch.bfloat16)
    r0 = torch.from_numpy(O.normal_bf16(0x4C510003, 1.0, (M, H)).view(np.int16)).to(dev).view(torch.bfloat16)
    h = torch.empty((M, F), dtype=torch.bfloat16, device=dev)
    r = r0.clone()

    def step(i):
        wg, sg, wu, su, wd, sd = sets[i % copies]
        L.stream_fp8_pc_ffn(x, wg, sg, wu, su, wd, sd, r, F, h=h, y=r)

    def step2(i, tg=None, td=None):
        wg, sg, wu, su, wd, sd = sets[i % copies]
        if tg: tg.start()
        L.stream_fp8_pc_silu_mul(x, wg, sg, wu, su, F, h=h)
        if tg: tg.stop()
        if td: td.start()
        L.stream_fp8_pc_residual(h, wd, sd, r, H, y=r)
        if td: td.stop()

    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)

    def timed(fn):
        for i in range(args.warmup):
            fn(i)
        torch.cuda.synchronize()
        t0.record()
        for i in range(args.steps):
            fn(i)
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / args.steps

    # The step: gate|up + SiLU*mul, then down + residual, launched back to back over the rotating weight copies
    # on this stream; HIP events around the loop give the mean step time. The same step as the one-launch FFN
    # kernel is timed the same way and reported beside it.
    ms = timed(step2)
    ms1 = timed(step)
    tg, td = Timer(torch, args.steps), Timer(torch, args.steps)
    for i in range(args.steps):
        step2(i, tg, td)
    torch.cuda.synchronize()

    def gu_only(i):
        wg, sg, wu, su, _, _ = sets[i % copies]
        L.stream_fp8_pc_silu_mul(x, wg, sg, wu, su, F, h=h)
    gu_b2b = timed(gu_only)

    def dn_only(i):
        _, _, _, _, wd, sd = sets[i % copies]
        L.stream_fp8_pc_residual(h, wd, sd, r, H, y=r)
    dn_b2b = timed(dn_only)
    # algorithmic bytes: weights + scales + activations in/out (+ residual read and write); h counted as the
    # gate|up output and the down input
    b_gu = 2 * F * H + 2 * F * 4 + M * H * 2 + M * F * 2
    b_dn = H * F + H * 4 + M * F * 2 + 2 * M * H * 2
    gb_s = (b_gu + b_dn) / (ms * 1e-3) / 1e9
    gu_ms, dn_ms = tg.mean_ms(), td.mean_ms()
    res = {
        "ms_per_step": ms,
        "gb_s": gb_s,
        "bytes_per_step": b_gu + b_dn,
        "one_launch": {"ms": ms1, "gb_s": (b_gu + b_dn) / (ms1 * 1e-3) / 1e9},
        "gate_up": {"ms": gu_b2b, "bytes": b_gu, "gb_s": b_gu / (gu_b2b * 1e-3) / 1e9,
                    "ms_event_pair": gu_ms, "gb_s_event_pair": b_gu / (gu_ms * 1e-3) / 1e9},
        "down": {"ms": dn_b2b, "bytes": b_dn, "gb_s": b_dn / (dn_b2b * 1e-3) / 1e9,
                 "ms_event_pair": dn_ms, "gb_s_event_pair": b_dn / (dn_ms * 1e-3) / 1e9},
        "rotation_copies": copies,
        "deadline_hit": L.stream_ffn_deadline_status(),
    }
    del sets
    drop_weight_cache(torch)
    return res


def bench_skinny(torch, L, O, args, dev, name, M, N, K, fmt):
    """A single skinny GEMM over rotating copies of one weight of the configs' data (FP8 per-channel, or NVFP4
    round-to-nearest of W ~ N(0, 0.02) by the library's host quantizer): ms per launch from HIP events around a
    captured graph of launches (the GPU's time; the host's ctypes dispatch is slower than these kernels), and GB/s."""
    import numpy as np
    if fmt == "fp8":
        wbytes, sbytes = N * K, N * 4
    else:
        wbytes, sbytes = N * K // 2 + N * K // 16, 0
    copies = max(2, -(-ROTATE_BYTES // wbytes))
    ws = []
    if fmt == "fp8":
        for c in range(copies):
            ws.append(fp8_weight(torch, L, N, K, 200, dev))
        g2 = None
    else:
        wb = O.f32_to_bf16(np.random.default_rng(300).standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
        v, sc, g2, _ = L.quantize_nvfp4(wb)
        del wb
        blob = L.retile_nvfp4(torch.from_numpy(v).to(dev), torch.from_numpy(sc).to(dev))
        ws = [(blob.clone(), None) for _ in range(copies)]
        del blob
    x = torch.from_numpy(O.normal_bf16(0x4C510000 + M, 1.0, (M, K)).view(np.int16)).to(dev).view(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

    def run(i):
        w, s = ws[i % copies]
        if fmt == "fp8":
            L.stream_fp8_pc(x, w, s, N, y=y)
        else:
            L.stream_nvfp4_bf16(x, w, None, g2, N, y=y)

    for i in range(args.warmup):
        run(i)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(args.steps):
        run(i)
    t1.record()
    torch.cuda.synchronize()
    ms_stream = t0.elapsed_time(t1) / args.steps
    ms = graph_per_launch_ms(torch, run, copies)
    b = wbytes + sbytes + M * K * 2 + M * N * 2
    del ws
    drop_weight_cache(torch)
    return {"M": M, "N": N, "K": K, "format": fmt, "ms": ms, "bytes": b, "gb_s": b / (ms * 1e-3) / 1e9,
            "frac_hbm": b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, "timing": "HIP graph of launches",
            "ms_stream_launches": ms_stream}


def bench_decode_step(torch, L, O, args, dev):
    """Config 5: M = 68 through 64 layers (48 DeltaNet, 16 attention, 64 MLP) + lm_head, FP8 per-channel."""
    import numpy as np
    M, H, F = 68, 5120, 17408
    mats = []  # (kind, N, K): kind "plain", "silu" (pairs), "resid"
    for li in range(64):
        if li % 4 == 3:
            mats += [("plain", 7168, H), ("resid", H, 6144)]
        else:
            mats += [("plain", 12352, H), ("resid", H, 6144)]
        mats += [("silu", F, H), ("resid", H, F)]
    mats.append(("plain", 151936, H))
    total = 0
    weights = []
    for i, (kind, N, K) in enumerate(mats):
        n_mats = 2 if kind == "silu" else 1
        ws = [fp8_weight(torch, L, N, K, 500 + j, dev) for j in range(n_mats)]
        total += n_mats * (N * K + N * 4)
        weights.append(ws)
    xs = {K: torch.from_numpy(O.normal_bf16(0x4C510005 + K, 1.0, (M, K)).view(np.int16)).to(dev).view(torch.bfloat16)
          for K in (H, 6144, F)}
    ys = {}

    def out(N):
        if N not in ys:
            ys[N] = torch.zeros((M, N), dtype=torch.bfloat16, device=dev)
        return ys[N]

    def step():
        for (kind, N, K), ws in zip(mats, weights):
            if kind == "plain":
                L.stream_fp8_pc(xs[K], ws[0][0], ws[0][1], N, y=out(N))
            elif kind == "silu":
                L.stream_fp8_pc_silu_mul(xs[K], ws[0][0], ws[0][1], ws[1][0], ws[1][1], N, h=out(N))
            else:
                r = out(N)
                L.stream_fp8_pc_residual(xs[K], ws[0][0], ws[0][1], r, N, y=r)

    steps = max(3, min(args.steps // 20, 10))
    step()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        step()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    del weights
    drop_weight_cache(torch)
    return {"M": M, "launches": len(mats), "weight_bytes": total, "ms": ms, "gb_s": total / (ms * 1e-3) / 1e9,
            "frac_hbm": total / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, "steps": steps}


def bench_prefill(torch, L, O, args, dev):
    """Config 4: M = 4096 FP8 x FP8 block-scaled GEMMs (gate|up as one N = 34816 GEMM, down), BF16 out."""
    if not hasattr(L, "prefill_fp8_block"):
        return None
    M, H, F = 4096, 5120, 17408
    res = {}
    total_flop, total_ms = 0.0, 0.0
    import numpy as np
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    for name, N, K in (("gate_up", 2 * F, H), ("down", H, F)):
        # the configs' data: W ~ N(0, 0.02) in 128 x 128 FP8 blocks (the library's host quantizer), activations
        # x ~ N(0, 1) in BF16 quantized in 1 x 128 groups by the library's device quantizer
        wf = np.random.default_rng(700 + K).standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
        qw, sw = L.quantize_fp8_block128(wf)
        del wf
        w = L.retile_fp8(torch.from_numpy(qw).to(dev))
        ws = torch.from_numpy(sw).to(dev)
        del qw
        xb = torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16)
        a, xs = L.quant_act_fp8_g128(xb)
        del xb
        y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        steps = max(10, args.steps // 2)
        # steady state: the part raises its clock over about a second of sustained MFMA load, so a few launches
        # from idle read 15-20 % slow; warm up on the same GEMM for PREFILL_WARM_S seconds first
        warm_until(torch, lambda: L.prefill_fp8_block(a, xs, w, ws, N, y=y))
        tm = Timer(torch, steps)
        for _ in range(steps):
            tm.start()
            L.prefill_fp8_block(a, xs, w, ws, N, y=y)
            tm.stop()
        torch.cuda.synchronize()
        ms = tm.mean_ms()
        flop = 2.0 * M * N * K
        res[name] = {"M": M, "N": N, "K": K, "ms": ms, "tflops": flop / (ms * 1e-3) / 1e12,
                     "frac_mfma": flop / (ms * 1e-3) / 1e12 / FP8_DENSE_TFLOPS}
        total_flop += flop
        total_ms += ms
        del w, a, xs, y
    res["total"] = {"flop": total_flop, "ms": total_ms, "tflops": total_flop / (total_ms * 1e-3) / 1e12,
                    "frac_mfma": total_flop / (total_ms * 1e-3) / 1e12 / FP8_DENSE_TFLOPS}
    if args.vendor_reference:
        # a comparison point only (not this library's path): the vendor GEMM with one scale per tensor, and this
        # library's two forms on the same operands
        ref = {}
        for name, N, K in (("gate_up", 2 * F, H), ("down", H, F)):
            a = torch.randn(M, K, device=dev).to(torch.float8_e4m3fn)
            b = torch.randn(N, K, device=dev).to(torch.float8_e4m3fn)
            one = torch.tensor(1.0, device=dev)
            # the same operands through this library: the per-tensor form and the block-scaled one (unit scales)
            w = L.retile_fp8(b.view(torch.uint8).contiguous())
            xs1 = torch.ones((M, K // 128), device=dev)
            ws1 = torch.ones((N // 128, K // 128), device=dev)
            yb = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
            runs = {"hipblaslt_per_tensor": lambda: torch._scaled_mm(a, b.t(), scale_a=one, scale_b=one,
                                                                     out_dtype=torch.bfloat16),
                    "per_tensor_here": lambda: L.prefill_gemm_fp8_bf16out(a.view(torch.uint8), w, 1.0, N, y=yb),
                    "block_scaled_here": lambda: L.prefill_fp8_block(a.view(torch.uint8), xs1, w, ws1, N, y=yb)}
            ref[name] = {}
            for key, fn in runs.items():
                warm_until(torch, fn)
                t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                t0.record()
                for _ in range(20):
                    fn()
                t1.record()
                torch.cuda.synchronize()
                ms = t0.elapsed_time(t1) / 20
                ref[name][key] = {"ms": ms, "tflops": 2.0 * M * N * K / (ms * 1e-3) / 1e12}
            del a, b, w, yb
        res["hipblaslt_fp8_per_tensor"] = ref
    torch.cuda.empty_cache()
    return res


def bench_prefill_nvfp4(torch, L, args, dev):
    """The NVFP4 prefill GEMM on config 4's gate|up shape (M = 4096, N = 2 x 17408, K = 5120) and the fused SwiGLU
    form (gate and up, N = 17408 each, into NVFP4): a beside-line, not one of the benchmark configs (their prefill is FP8)."""
    M, H, F = 4096, 5120, 17408
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    res = {}

    import numpy as np

    def blob(N, K, seed):
        # W ~ N(0, 0.02) rounded to NVFP4 by the library's host quantizer
        wb = (np.random.default_rng(seed).standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
        wb = (wb.view(np.uint32) + 0x7FFF + ((wb.view(np.uint32) >> 16) & 1)) >> 16  # BF16, round to nearest even
        v, sc, _, _ = L.quantize_nvfp4(wb.astype(np.uint16))
        return L.retile_nvfp4(torch.from_numpy(v).to(dev), torch.from_numpy(sc).to(dev))

    # activations x ~ N(0, 1) quantized to NVFP4 by the library's device quantizer
    xq, xs = L.quant_act_nvfp4(torch.randn((M, H), device=dev, generator=g), 1.0)
    steps = max(10, args.steps // 2)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn):
        warm_until(torch, fn)  # steady-state clock, as for the FP8 prefill
        t0.record()
        for _ in range(steps):
            fn()
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / steps

    w = blob(2 * F, H, 801)
    y = torch.empty((M, 2 * F), dtype=torch.float32, device=dev)
    ms = timed(lambda: L.prefill_gemm_nvfp4(xq, xs, w, 1.0, 2 * F, y=y))
    flop = 2.0 * M * 2 * F * H
    res["gemm_gate_up"] = {"M": M, "N": 2 * F, "K": H, "ms": ms, "tflops": flop / (ms * 1e-3) / 1e12}
    del w, y
    gw, uw = blob(F, H, 802), blob(F, H, 803)
    ms = timed(lambda: L.prefill_swiglu_nvfp4(xq, xs, gw, 1.0, uw, 1.0, F, 0.05))
    res["swiglu_gate_up"] = {"M": M, "N": F, "K": H, "ms": ms, "tflops": flop / (ms * 1e-3) / 1e12}
    del gw, uw
    torch.cuda.empty_cache()
    return res


def cpu_baseline(O):
    """The oracle's whole CPU path (dequantize to FP32, FP32 accumulate in k order, BF16 out) on the headline
    workload's shapes: one verify-MLP pass at M = 17 (gate 5120->17408, up 5120->17408, down 17408->5120), on
    every host core, best of 3; reported in the metric's unit (GB/s of weight + activation bytes)."""
    import numpy as np
    M, H, F = 17, 5120, 17408
    threads = O.hardware_threads()
    rng = np.random.default_rng(0x4C510006)
    x = O.normal_bf16(0x4C510002, 1.0, (M, H))
    h = O.normal_bf16(0x4C510003, 1.0, (M, F))
    def codes(n, k):
        q = rng.integers(0, 256, (n, k), dtype=np.uint8)
        q[(q & 0x7F) == 0x7F] = 0x3C
        return q
    qg, qu, qd = codes(F, H), codes(F, H), codes(H, F)
    sg = np.full(F, 2e-4, np.float32)
    sd = np.full(H, 2e-4, np.float32)
    best = None
    for _ in range(3):
        t = time.perf_counter()
        O.stream_fp8_pc_bf16(x, qg, sg, threads=threads)
        O.stream_fp8_pc_bf16(x, qu, sg, threads=threads)
        O.stream_fp8_pc_bf16(h, qd, sd, threads=threads)
        dt = time.perf_counter() - t
        best = dt if best is None else min(best, dt)
    b = (2 * F * H + 2 * F * 4 + M * H * 2 + M * F * 2) + (H * F + H * 4 + M * F * 2 + 2 * M * H * 2)
    # the model string, with the family / model / stepping numbers (a virtual machine's model string can be generic)
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                k, _, v = ln.partition(":")
                k = k.strip()
                if k in ("model name", "cpu family", "model", "stepping") and k not in info:
                    info[k] = v.strip()
                if not ln.strip() and info:
                    break
    except OSError:
        pass
    cpu = info.get("model name", "unknown")
    if "cpu family" in info:
        cpu += f" (family {info['cpu family']}, model {info.get('model', '?')}, stepping {info.get('stepping', '?')})"
    return {"value": round(b / best / 1e9, 3), "unit": "GB/s", "cores": threads, "cpu": cpu, "kind": "port",
            "sample": f"one full verify-MLP pass (M=17; gate and up 5120->17408, down 17408->5120; FP8 per-channel) "
                      f"through the oracle's C path, best of 3: {best:.2f} s per pass, "
                      f"{best * threads:.1f} core-seconds"}


def bench_producers(torch, L, dev):
    """The activation producers at config 4's shapes (M = 4096 tokens) and the sparse-head gather (M = 17, 2048
    of 151936 vocabulary rows of a 5120-wide NVFP4 head): all HBM-bound, so each reports its bytes moved (inputs
    read once, outputs written once), the time per launch (HIP events around a captured graph of launches rotating
    over input copies of >= 1 GB: the GPU's time, not the host's call rate) and the fraction of 8 TB/s. The gather's eight row sets touch 48 MB of the head, which
    the 256 MB MALL can hold across repetitions; the gather is latency-bound either way (timed alike with rows in
    order or repeated)."""
    M, H, F = 4096, 5120, 17408
    g = torch.Generator(device=dev)
    g.manual_seed(0x4C51000A)

    def timed(fn, copies):
        return graph_per_launch_ms(torch, fn, copies)

    def line(name, nbytes, ms):
        return {"bytes": nbytes, "us": round(ms * 1e3, 2), "gb_s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                "frac_hbm": round(nbytes / (ms * 1e-3) / 8e12, 4)}

    out = {}
    nb = M * H
    # 1x128 FP8 group quantizer: BF16 in, FP8 + FP32 group scales out
    c = max(2, -(-(1 << 30) // (2 * nb)))
    xs = [torch.randn(M, H, device=dev, generator=g).to(torch.bfloat16) for _ in range(c)]
    byt = 2 * nb + nb + nb // 128 * 4
    out["quant_act_fp8_g128"] = line("g128", byt, timed(lambda i: L.quant_act_fp8_g128(xs[i]), c))
    del xs
    # NVFP4 quantizer and RMSNorm into NVFP4 (no FP32 copy): FP32 in, packed E2M1 + E4M3 block scales out
    c = max(2, -(-(1 << 30) // (4 * nb)))
    xf = [torch.randn(M, H, device=dev, generator=g) for _ in range(c)]
    byt = 4 * nb + nb // 2 + nb // 16
    out["quant_act_nvfp4"] = line("nvfp4", byt, timed(lambda i: L.quant_act_nvfp4(xf[i], 0.01), c))
    w = (torch.randn(H, device=dev, generator=g) * 0.1).to(torch.bfloat16).view(torch.int16)
    out["rmsnorm_quant_nvfp4"] = line("rmsq", byt + 2 * H, timed(
        lambda i: L.rmsnorm_quant(xf[i], w, 1e-6, True, 0.01, with_out=False), c))
    # per-tensor FP8 quantizer and RMSNorm into FP8: FP32 in, FP8 out
    out["quant_act_fp8"] = line("fp8", 5 * nb, timed(lambda i: L.quant_act_fp8(xf[i], 0.02), c))
    out["rmsnorm_quant_fp8"] = line("rmsq8", 5 * nb + 2 * H, timed(
        lambda i: L.rmsnorm_quant(xf[i], w, 1e-6, False, 0.02, with_out=False), c))
    # the stream GEMMs' FP16 activation copies, at the largest skinny M (68 rows; latency-bound at this size):
    # FP32 in, FP16 + per-row scale out (RMSNorm also writes FP32)
    ms_ = 68
    xs68 = [xf[i][:ms_].contiguous() for i in range(c)]
    n68 = ms_ * H
    out["to_half_rows_m68"] = line("half", 6 * n68 + 4 * ms_, timed(lambda i: L.to_half_rows(xs68[i]), c))
    out["rmsnorm_half_m68"] = line("rmsh", 10 * n68 + 4 * ms_ + 2 * H, timed(
        lambda i: L.rmsnorm_half(xs68[i], w.view(torch.bfloat16), 1e-6), c))
    del xf
    # silu(g) * u into NVFP4 (the FFN's gate|up outputs, FP32): two inputs
    nf = M * F
    c = 2
    gu = [(torch.randn(M, F, device=dev, generator=g), torch.randn(M, F, device=dev, generator=g)) for _ in range(c)]
    byt = 8 * nf + nf // 2 + nf // 16
    out["silu_mul_quant_nvfp4"] = line("silu", byt, timed(lambda i: L.silu_mul_quant_nvfp4(gu[i][0], gu[i][1], 0.01), c))
    del gu
    # the DeltaNet gated output norm into FP8 (48 value heads of 128 per token) and the attention output's sigmoid
    # gate into FP8 (24 heads of 256 per token): two FP32 inputs each
    rows, qs = M * 48, M * 24 * 256
    c = 2
    xz = [(torch.randn(rows, 128, device=dev, generator=g), torch.randn(rows, 128, device=dev, generator=g))
          for _ in range(c)]
    wn = (torch.randn(128, device=dev, generator=g) * 0.5).to(torch.bfloat16).view(torch.int16)
    out["gated_rmsnorm_fp8"] = line("gnorm", 9 * rows * 128 + 256, timed(
        lambda i: L.gated_rmsnorm_fp8(xz[i][0], xz[i][1], wn, 1e-6, 0.02), c))
    del xz
    xg = [(torch.randn(qs, device=dev, generator=g), torch.randn(qs, device=dev, generator=g)) for _ in range(c)]
    out["sigmoid_mul_fp8"] = line("sigm", 9 * qs, timed(lambda i: L.sigmoid_mul_fp8(xg[i][0], xg[i][1], 0.02), c))
    del xg
    torch.cuda.empty_cache()
    # sparse-head gather: 2048 of 151936 rows of an NVFP4 [151936][5120] head, M = 17 (a verify step's rows)
    V, K, Mg, cap = 151936, 5120, 17, 2048
    vals = torch.randint(0, 256, (V, K // 2), dtype=torch.uint8, device=dev, generator=g)
    scs = torch.randint(0x28, 0x48, (V, K // 16), dtype=torch.uint8, device=dev, generator=g)
    head = L.retile_nvfp4(vals, scs)
    del vals, scs
    xh, xinv = L.bf16_to_half_rows(torch.randn(Mg, K, device=dev, generator=g).to(torch.bfloat16))
    sets = []
    for c2 in range(8):
        rows = torch.randperm(V, device=dev, generator=g)[:cap].to(torch.int32)
        sets.append(rows)
    nrows = torch.tensor([cap], dtype=torch.int32, device=dev)
    y = torch.empty((Mg, cap), dtype=torch.float32, device=dev)
    byt = cap * (K // 2 + K // 16) + Mg * K * 2 + Mg * cap * 4
    out["gather_nvfp4_2048_of_151936"] = line("gather", byt, timed(
        lambda i: L.stream_gemm_gather_nvfp4(xh, xinv, head, None, 1e-3, sets[i], nrows, cap, V, K, y=y), 8))
    del head
    torch.cuda.empty_cache()
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (the path is single-GPU); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch

    import ling_gemm as L
    import oracle as O
    dev = "cuda:0"
    torch.cuda.set_device(0)
    L.init()
    only = set(args.only.split(",")) if args.only else None
    props = torch.cuda.get_device_properties(0)
    log(f"[bench] {props.name} CUs={props.multi_processor_count} mem={props.total_memory / 2**30:.0f} GiB")

    vm = bench_verify_mlp(torch, L, O, args, dev)
    log(f"[bench] verify MLP: {vm['ms_per_step'] * 1e3:.1f} us/step, {vm['gb_s']:.0f} GB/s")
    extra = {}
    if only is None or "decode" in only:
        extra["decode_m1"] = bench_skinny(torch, L, O, args, dev, "decode", 1, 5120, 5120, "fp8")
        log(f"[bench] decode M=1: {extra['decode_m1']}")
    if only is None or "nvfp4" in only:
        extra["drafter_fc_nvfp4_m16"] = bench_skinny(torch, L, O, args, dev, "fc", 16, 5120, 25600, "nvfp4")
        log(f"[bench] nvfp4 fc: {extra['drafter_fc_nvfp4_m16']}")
    if only is None or "step" in only:
        extra["decode_step_m68"] = bench_decode_step(torch, L, O, args, dev)
        log(f"[bench] full step M=68: {extra['decode_step_m68']}")
    if only is None or "prefill" in only:
        pf = bench_prefill(torch, L, O, args, dev)
        if pf:
            extra["prefill_m4096"] = pf
            log(f"[bench] prefill: {pf['total']}")
    if only is None or "nvfp4prefill" in only:
        pn = bench_prefill_nvfp4(torch, L, args, dev)
        extra["prefill_nvfp4_m4096"] = pn
        log(f"[bench] prefill nvfp4: {pn}")
    if only is None or "producers" in only:
        pr = bench_producers(torch, L, dev)
        extra["producers"] = pr
        log(f"[bench] producers: {pr}")
    if args.copy_calibration:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    cpu = None if args.no_cpu else cpu_baseline(O)
    if cpu:
        log(f"[bench] cpu baseline: {cpu}")

    gu = vm["gate_up"]
    # HBM bytes per launch of the gate|up kernel, from the committed rocprofv3 PMC summary (FETCH_SIZE and
    # WRITE_SIZE per dispatch, calibrated on a 1 GiB copy); null when absent
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "stream_gemm_verify_m17_hbm_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f)["kernels"].get("gate_up_silu", {}).get("traffic_bytes")
    line = {
        "metric": "verify GEMM HBM GB/s (% peak) at M=17; prefill block-scaled TFLOP/s",
        "value": round(vm["gb_s"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(vm["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic, the configs' recipes: activations N(0,1) in BF16; weights N(0,0.02) quantized by the "
                "library's host quantizers (FP8 per channel amax/448; NVFP4 round-to-nearest; prefill FP8 in 128x128 "
                "blocks, activations in 1x128 groups by the device quantizer); rotation copies are device clones",
        "config": {"workload": "speculative-verify MLP, M=17: gate|up 5120->2x17408 FP8 per-channel + SiLU*mul, "
                               "down 17408->5120 + BF16 residual (benchmark config 2)",
                   "M": 17, "hidden": 5120, "ffn": 17408, "weight_format": "fp8_e4m3 per-channel",
                   "rotation_copies": vm["rotation_copies"]},
        "frac_hbm": round(vm["gb_s"] / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(gu["gb_s"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu["gb_s"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "stream_kernel (gate|up + SiLU*mul, M=17)", "bytes_per_launch": gu["bytes"],
                     "ms_per_launch": round(gu["ms"], 5),
                     "timing": "HIP events around back-to-back launches of this kernel alone on its stream"},
        "kernels": {"gate_up_silu": gu, "down_residual": vm["down"],
                    "ffn_one_launch": dict(vm["one_launch"], deadline_hit=vm["deadline_hit"])},
        "cpu_baseline": cpu,
    }
    line.update(extra)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
