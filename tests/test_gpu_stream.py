"""Parity of the skinny (stream) GEMMs on the GPU against the CPU oracle, through the C ABI.

Bounds (the path's accuracy target): on BF16 outputs, max relative error <= 1e-2 and mean |got - ref| <= 1e-3, with the
relative error of an element |got - ref| / max(|ref|, rms(ref row)) (robust to outputs near zero; one BF16 ulp is
at most 2^-8 of it),
where ref is the oracle (dequantize to FP32, FP32 accumulate, one BF16 rounding); dequantized weights and the
layout are bit-exact. Rows of every M are bit-identical to the same rows of a larger launch (row invariance,
reference src/core/stream_gemm.cu:10-13, tests/stream_tests.cu:206-224).
"""
import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture(scope="module")
def L():
    import ling_gemm
    ling_gemm.init()
    return ling_gemm


def to_dev(a: np.ndarray, dtype=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    return t.view(dtype) if dtype is not None else t


def bf16_dev(bits: np.ndarray) -> torch.Tensor:
    return to_dev(bits.view(np.int16)).view(torch.bfloat16)


def bf16_host(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def assert_close_bf16(got_bits: np.ndarray, ref_bits: np.ndarray, what: str, row_scaled: bool = False):
    """row_scaled: inputs deliberately scaled far from N(0, 1) per row; the mean absolute error is then taken
    in units of each row's rms."""
    got = O.bf16_to_f32(got_bits).astype(np.float64)
    ref = O.bf16_to_f32(ref_bits).astype(np.float64)
    assert np.isfinite(got).all(), what
    rms = np.sqrt(np.mean(ref * ref, axis=-1, keepdims=True)) + 1e-30
    rel = np.max(np.abs(got - ref) / np.maximum(np.abs(ref), rms))
    mae = np.mean(np.abs(got - ref) / rms) if row_scaled else np.mean(np.abs(got - ref))
    assert rel <= 1e-2, f"{what}: max rel err {rel:.3e}"
    assert mae <= 1e-3, f"{what}: mean abs err {mae:.3e}"
    return rel, mae


def fp8_weights(seed, N, K):
    w = O.normal_f32(seed, 0.02, (N, K))
    return O.quant_fp8_per_channel(w)


# ---------------------------------------------------------------- layout / dequant
@pytest.mark.parametrize("N,K", [(16, 128), (48, 384), (528, 2048)])
def test_retile_fp8_bytes_and_dequant_bit_exact(L, N, K):
    q, s = fp8_weights(1, N, K)
    tw = L.retile_fp8(to_dev(q))
    assert np.array_equal(tw.cpu().numpy(), O.retile_fp8(q))
    got = L.dequant_tiled_fp8_pc_f32(tw, to_dev(s), N, K).cpu().numpy()
    want = O.dequant_fp8_pc(q, s)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    gb = bf16_host(L.dequant_tiled_fp8(tw, 0.021, N, K))
    wb = O.f32_to_bf16(O.dequant_fp8_pc(q, np.full(N, 0.021, np.float32)))
    assert np.array_equal(gb, wb)


@pytest.mark.parametrize("N,K", [(16, 128), (528, 2048)])
def test_retile_nvfp4_raw_and_coded_bytes_and_dequant(L, N, K):
    w = O.normal_bf16(2, 0.02, (N, K))
    v, s, g, _ = O.quant_nvfp4(w)
    tw = L.retile_nvfp4(to_dev(v), to_dev(s))
    assert np.array_equal(tw.cpu().numpy(), O.retile_nvfp4(v, s))
    got = L.dequant_tiled_nvfp4_f32(tw, g, N, K).cpu().numpy()
    want = O.dequant_nvfp4(v, s, g)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(bf16_host(L.dequant_tiled_nvfp4(tw, g, N, K)), O.f32_to_bf16(want))
    ok, table, code_of = O.scale_code_table(s)
    assert ok
    blob, raw = L.retile_nvfp4_coded(to_dev(v), to_dev(s), to_dev(code_of))
    oblob, oraw = O.retile_nvfp4_coded(v, s, code_of)
    assert np.array_equal(blob.cpu().numpy(), oblob)
    assert np.array_equal(raw.cpu().numpy(), oraw)
    got2 = L.dequant_tiled_nvfp4_f32(blob, g, N, K, raw).cpu().numpy()
    assert np.array_equal(got2.view(np.uint32), want.view(np.uint32))


# ---------------------------------------------------------------- BF16 per-channel FP8 path
MS = [1, 2, 7, 15, 16, 17, 24, 31, 32, 33, 48, 64, 68, 80]


@pytest.mark.parametrize("N,K", [(528, 2048), (16, 128), (1040, 384)])
def test_stream_fp8_pc_parity_and_row_invariance(L, N, K):
    q, s = fp8_weights(3, N, K)
    x = O.normal_bf16(4, 1.0, (80, K))
    tw = L.retile_fp8(to_dev(q))
    sd = to_dev(s)
    xd = bf16_dev(x)
    ref = O.stream_fp8_pc_bf16(x, q, s)
    full = bf16_host(L.stream_fp8_pc(xd, tw, sd, N))
    assert_close_bf16(full, ref, f"M=80 N={N} K={K}")
    for M in MS:
        got = bf16_host(L.stream_fp8_pc(xd[:M].contiguous(), tw, sd, N))
        assert np.array_equal(got, full[:M]), f"row invariance M={M}"


def test_stream_fp8_pc_silu_mul(L):
    N, K = 1024, 1280
    qg, sg = fp8_weights(5, N, K)
    qu, su = fp8_weights(6, N, K)
    x = O.normal_bf16(7, 1.0, (68, K))
    twg, twu = L.retile_fp8(to_dev(qg)), L.retile_fp8(to_dev(qu))
    xd = bf16_dev(x)
    xf = O.bf16_to_f32(x)
    gacc = O.gemm_f32(xf, O.dequant_fp8_pc(qg, sg))
    uacc = O.gemm_f32(xf, O.dequant_fp8_pc(qu, su))
    ref = O.epi_silu_mul_bf16(gacc, uacc)
    full = bf16_host(L.stream_fp8_pc_silu_mul(xd, twg, to_dev(sg), twu, to_dev(su), N))
    assert_close_bf16(full, ref, "silu_mul M=68")
    for M in [1, 17, 33]:
        got = bf16_host(L.stream_fp8_pc_silu_mul(xd[:M].contiguous(), twg, to_dev(sg), twu, to_dev(su), N))
        assert np.array_equal(got, full[:M])


def test_stream_fp8_pc_residual_in_place(L):
    N, K = 512, 2048
    q, s = fp8_weights(8, N, K)
    x = O.normal_bf16(9, 1.0, (17, K))
    r = O.normal_bf16(10, 1.0, (17, N))
    tw = L.retile_fp8(to_dev(q))
    acc = O.gemm_f32(O.bf16_to_f32(x), O.dequant_fp8_pc(q, s))
    ref = O.epi_residual_bf16(acc, r)
    rd = bf16_dev(r)
    out = bf16_host(L.stream_fp8_pc_residual(bf16_dev(x), tw, to_dev(s), rd, N))
    assert_close_bf16(out, ref, "residual")
    L.stream_fp8_pc_residual(bf16_dev(x), tw, to_dev(s), rd, N, y=rd)  # in place
    assert np.array_equal(bf16_host(rd), out)


def _ffn_case(L, I, H, seed, Ms):
    qg, sg = fp8_weights(seed, I, H)
    qu, su = fp8_weights(seed + 1, I, H)
    qd, sd = fp8_weights(seed + 2, H, I)
    tg, tu, td = L.retile_fp8(to_dev(qg)), L.retile_fp8(to_dev(qu)), L.retile_fp8(to_dev(qd))
    sg_d, su_d, sd_d = to_dev(sg), to_dev(su), to_dev(sd)
    x = O.normal_bf16(seed + 3, 1.0, (max(Ms), H))
    r = O.normal_bf16(seed + 4, 1.0, (max(Ms), H))
    out = {}
    for M in Ms:
        xd, rd = bf16_dev(x[:M]), bf16_dev(r[:M])
        h_sep = L.stream_fp8_pc_silu_mul(xd, tg, sg_d, tu, su_d, I)
        y_sep = L.stream_fp8_pc_residual(h_sep, td, sd_d, rd, H)
        for rep in range(3):  # repeated launches: the in-kernel counters reset themselves
            h, y = L.stream_fp8_pc_ffn(xd, tg, sg_d, tu, su_d, td, sd_d, rd, I)
            assert np.array_equal(bf16_host(h), bf16_host(h_sep)), f"ffn h M={M} launch {rep}"
            assert np.array_equal(bf16_host(y), bf16_host(y_sep)), f"ffn y M={M} launch {rep}"
        out[M] = (bf16_host(h), bf16_host(y))
    assert L.stream_ffn_deadline_status() == 0
    return (qg, sg, qu, su, qd, sd, x, r), out


def test_stream_fp8_pc_ffn_one_launch(L):
    """The one-launch FFN equals gate|up + SiLU*mul followed by down + residual bit for bit, and the oracle."""
    I, H = 4096, 2048
    (qg, sg, qu, su, qd, sd, x, r), out = _ffn_case(L, I, H, 40, [1, 17, 68])
    M = 17
    xf = O.bf16_to_f32(x[:M])
    href = O.epi_silu_mul_bf16(O.gemm_f32(xf, O.dequant_fp8_pc(qg, sg)), O.gemm_f32(xf, O.dequant_fp8_pc(qu, su)))
    yref = O.epi_residual_bf16(O.gemm_f32(O.bf16_to_f32(out[M][0]), O.dequant_fp8_pc(qd, sd)), r[:M])
    assert_close_bf16(out[M][0], href, "ffn h")
    assert_close_bf16(out[M][1], yref, "ffn y")


def test_stream_fp8_pc_ffn_in_place_full_size(L):
    """Config 2's shapes (I = 17408, H = 5120, M = 17) with the residual updated in place."""
    I, H, M = 17408, 5120, 17
    x = O.normal_bf16(99, 1.0, (M, H))
    r = O.normal_bf16(98, 1.0, (M, H))
    qg, sg = fp8_weights(60, I, H)
    qu, su = fp8_weights(61, I, H)
    qd, sd = fp8_weights(62, H, I)
    tg, tu, td = L.retile_fp8(to_dev(qg)), L.retile_fp8(to_dev(qu)), L.retile_fp8(to_dev(qd))
    xd, rd = bf16_dev(x), bf16_dev(r)
    h_sep = L.stream_fp8_pc_silu_mul(xd, tg, to_dev(sg), tu, to_dev(su), I)
    y_sep = bf16_host(L.stream_fp8_pc_residual(h_sep, td, to_dev(sd), rd, H))
    h, y = L.stream_fp8_pc_ffn(xd, tg, to_dev(sg), tu, to_dev(su), td, to_dev(sd), rd, I, y=rd)
    assert np.array_equal(bf16_host(h), bf16_host(h_sep))
    assert np.array_equal(bf16_host(rd), y_sep)
    assert L.stream_ffn_deadline_status() == 0


# ---------------------------------------------------------------- reference-compatible FP16 path
def reference_rows(x: np.ndarray, wdeq: np.ndarray) -> np.ndarray:
    return (x.astype(np.float64) @ wdeq.astype(np.float64).T)


def test_to_half_rows_bit_exact(L):
    x = O.normal_f32(11, 1.0, (24, 5120))
    x[1] = 0
    x[2, 77] = 3.0e30
    x[3, 5119] = np.inf
    xh, xinv = L.to_half_rows(to_dev(x))
    wh, winv = O.to_half_rows(x)
    assert np.array_equal(xh.view(torch.int16).cpu().numpy().view(np.uint16), wh)
    assert np.array_equal(xinv.cpu().numpy(), winv)
    xb = O.f32_to_bf16(O.normal_f32(12, 1.0, (16, 25600)))
    bh, binv = L.bf16_to_half_rows(bf16_dev(xb))
    wh2, winv2 = O.to_half_rows(O.bf16_to_f32(xb))
    assert np.array_equal(bh.view(torch.int16).cpu().numpy().view(np.uint16), wh2)
    assert np.array_equal(binv.cpu().numpy(), winv2)


@pytest.mark.parametrize("K", [100, 1000, 3000, 8192, 12000, 32768, 40000, 65600])
def test_to_half_rows_row_widths(L, K):
    """Rows held in registers (up to 32768 values a row), including widths that leave a ragged tail, and longer rows
    (the split-grid form: each block converts a slice), from FP32 and from BF16."""
    x = O.normal_f32(13 + K, 1.0, (5, K))
    x[4] = 0
    x[2, K - 1] = 7.0e4  # the row's largest magnitude in the last slice
    xh, xinv = L.to_half_rows(to_dev(x))
    wh, winv = O.to_half_rows(x)
    assert np.array_equal(xh.view(torch.int16).cpu().numpy().view(np.uint16), wh)
    assert np.array_equal(xinv.cpu().numpy(), winv)
    xb = O.f32_to_bf16(x)
    bh, binv = L.bf16_to_half_rows(bf16_dev(xb))
    wh2, winv2 = O.to_half_rows(O.bf16_to_f32(xb))
    assert np.array_equal(bh.view(torch.int16).cpu().numpy().view(np.uint16), wh2)
    assert np.array_equal(binv.cpu().numpy(), winv2)


def reference_style_weights(seed, N, K):
    """tests/stream_tests.cu:147-160: random bytes (no E4M3 NaN), NVFP4 scales 0x28..0x48, x with outliers."""
    rng = np.random.default_rng(seed)
    w8 = rng.integers(0, 256, (N, K), dtype=np.uint8)
    w8[(w8 & 0x7F) == 0x7F] = 0x10
    w4 = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    s4 = rng.integers(0x28, 0x49, (N, K // 16), dtype=np.uint8)
    x = O.normal_f32(seed + 1, 1.0, (32, K))
    x.reshape(-1)[::97] *= 30.0
    return w8, w4, s4, x


def test_stream_gemm_fp8_and_nvfp4_reference_compatible(L):
    N, K = 528, 2048
    w8, w4, s4, x = reference_style_weights(11, N, K)
    gs4, gs8 = 0.37, 0.021
    t8 = L.retile_fp8(to_dev(w8))
    t4 = L.retile_nvfp4(to_dev(w4), to_dev(s4))
    xh, xinv = L.to_half_rows(to_dev(x))
    ref8 = reference_rows(x, O.dequant_fp8_pc(w8, np.full(N, gs8, np.float32)))
    ref4 = reference_rows(x, O.dequant_nvfp4(w4, s4, gs4))
    for fp4, ref in [(False, ref8), (True, ref4)]:
        full = (L.stream_gemm_nvfp4(xh, xinv, t4, None, gs4, N, K) if fp4 else
                L.stream_gemm_fp8(xh, xinv, t8, gs8, N, K)).cpu().numpy()
        rms = np.sqrt(np.mean(ref ** 2, axis=1, keepdims=True))
        # the reference's own bound (tests/stream_tests.cu:211-218)
        assert np.max(np.abs(full - ref) / rms) < 2e-3
        for M in [1, 2, 7, 8, 9, 15, 16, 17, 20, 24, 25, 32]:
            got = (L.stream_gemm_nvfp4(xh[:M].contiguous(), xinv[:M].contiguous(), t4, None, gs4, N, K) if fp4 else
                   L.stream_gemm_fp8(xh[:M].contiguous(), xinv[:M].contiguous(), t8, gs8, N, K)).cpu().numpy()
            assert np.array_equal(got, full[:M])


def test_coded_equals_raw_and_multi_equals_separate(L):
    N, K = 528, 1024
    w = O.normal_bf16(13, 0.02, (N, K))
    v, s, g, _ = O.quant_nvfp4(w)
    ok, table, code_of = O.scale_code_table(s)
    assert ok
    raw = L.retile_nvfp4(to_dev(v), to_dev(s))
    blob, _ = L.retile_nvfp4_coded(to_dev(v), to_dev(s), to_dev(code_of))
    tab = to_dev(table)
    x = O.normal_f32(14, 1.0, (20, K))
    xh, xinv = L.to_half_rows(to_dev(x))
    a = L.stream_gemm_nvfp4(xh, xinv, raw, None, g, N, K).cpu().numpy()
    b = L.stream_gemm_nvfp4(xh, xinv, blob, tab, g, N, K).cpu().numpy()
    assert np.array_equal(a, b)
    q8, _ = fp8_weights(15, 256, K)
    t8 = L.retile_fp8(to_dev(q8))
    y8 = L.stream_gemm_fp8(xh, xinv, t8, 0.5, 256, K).cpu().numpy()
    ya = torch.empty((20, N), dtype=torch.float32, device=DEV)
    yb = torch.empty((20, N), dtype=torch.float32, device=DEV)
    L.stream_gemm_multi(True, xh, xinv, [(raw, None, g, ya, N), (blob, tab, g, yb, N)], K)
    assert np.array_equal(ya.cpu().numpy(), a) and np.array_equal(yb.cpu().numpy(), a)
    y1 = torch.empty((20, 256), dtype=torch.float32, device=DEV)
    y2 = torch.empty((20, 256), dtype=torch.float32, device=DEV)
    L.stream_gemm_multi(False, xh, xinv, [(t8, None, 0.5, y1, 256), (t8, None, 0.5, y2, 256)], K)
    assert np.array_equal(y1.cpu().numpy(), y8) and np.array_equal(y2.cpu().numpy(), y8)


def test_l2_prefetch_weights_changes_nothing(L):
    """The cache run-ahead (reference kernels.cuh:405 l2_prefetch_weights) writes nothing: every GEMM after it gives
    the same bits, FP8 and NVFP4 raw and coded, at budgets from one unit per workgroup to the whole matrix; a null
    blob or a zero budget is a no-op, as in the reference (stream_gemm.cu:1865); a bad shape is an error."""
    N, K = 2048, 5120
    q, s = fp8_weights(77, N, K)
    tw, sd = L.retile_fp8(to_dev(q)), to_dev(s)
    x = bf16_dev(O.normal_bf16(78, 1.0, (17, K)))
    before = bf16_host(L.stream_fp8_pc(x, tw, sd, N))
    for nbytes in (1, 1 << 20, 1 << 40):
        L.l2_prefetch_weights(tw, False, False, N, K, nbytes)
        assert np.array_equal(bf16_host(L.stream_fp8_pc(x, tw, sd, N)), before), f"fp8 nbytes={nbytes}"
    v, sc, g, _ = O.quant_nvfp4(O.normal_bf16(79, 0.02, (N, K)))
    ok, table, code_of = O.scale_code_table(sc)
    assert ok
    raw = L.retile_nvfp4(to_dev(v), to_dev(sc))
    coded, _ = L.retile_nvfp4_coded(to_dev(v), to_dev(sc), to_dev(code_of))
    for blob, tab in ((raw, None), (coded, to_dev(table))):
        ref = bf16_host(L.stream_nvfp4_bf16(x, blob, tab, g, N))
        for nbytes in (1, 1 << 22, 1 << 40):
            L.l2_prefetch_weights(blob, True, tab is not None, N, K, nbytes)
            got = bf16_host(L.stream_nvfp4_bf16(x, blob, tab, g, N))
            assert np.array_equal(got, ref), f"nvfp4 coded={tab is not None} nbytes={nbytes}"
    torch.cuda.synchronize()
    L.l2_prefetch_weights(None, False, False, N, K, 1 << 20)
    L.l2_prefetch_weights(tw, False, False, 17, K, 0)  # zero budget: not even the shape is looked at
    with pytest.raises(L.LingGemmError):
        L.l2_prefetch_weights(tw, False, False, 17, K, 1 << 20)
    with pytest.raises(L.LingGemmError):
        L.l2_prefetch_weights(tw, False, False, N, 100, 1 << 20)


@pytest.mark.parametrize("N,K", [(4096, 2560), (8192, 5120)])
def test_stream_gemm_gather_nvfp4_bit_exact(L, N, K):
    """The sparse head (reference tests/stream_tests.cu:271-300): a row subset, not in order, from the raw blob
    and from the coded blob with its raw scales; each selected row's logits are the full launch's bit for bit,
    columns past the count are -inf (workgroups wholly past it included), an empty selection is all -inf. The
    shapes split every tile group across workgroups, so the full launch's cuts are exercised."""
    w = O.normal_bf16(60 + N, 0.02, (N, K))
    v, s, g, _ = O.quant_nvfp4(w)
    ok, table, code_of = O.scale_code_table(s)
    assert ok
    raw = L.retile_nvfp4(to_dev(v), to_dev(s))
    coded, raw_scales = L.retile_nvfp4_coded(to_dev(v), to_dev(s), to_dev(code_of))
    rows = np.arange(N - 1, -1, -3, dtype=np.int32)
    cnt = rows.size
    cap = (cnt + 96 + 31) // 32 * 32
    drows = to_dev(rows)
    x = O.normal_f32(61, 1.0, (80, K))
    for M in [1, 11, 17, 33, 65, 68, 80]:
        xh, xinv = L.to_half_rows(to_dev(x[:M]))
        full = L.stream_gemm_nvfp4(xh, xinv, raw, None, g, N, K).cpu().numpy()
        for c in [cnt, 5, 0]:
            dcnt = to_dev(np.array([c], np.int32))
            want = np.full((M, cap), -np.inf, np.float32)
            want[:, :c] = full[:, rows[:c]]
            for blob, rs in ((raw, None), (coded, raw_scales)):
                got = L.stream_gemm_gather_nvfp4(xh, xinv, blob, rs, g, drows, dcnt, cap, N, K).cpu().numpy()
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"gather M={M} count={c}"


@pytest.mark.parametrize("N,K", [(512, 2560), (8192, 2560)])
def test_stream_nvfp4_bf16(L, N, K):
    """BF16 activations on the NVFP4 path: each 128-value chunk of a row is staged as FP16 under its own
    power-of-two scale. Rows span 1e-6 .. 3e4 in magnitude, chunks within a row differ by up to 2^12, one row is
    zero; every M is row-invariant against M = 68, raw and coded scales agree. Two shapes: a tile group spread
    over 20 workgroups' ranges (512 rows) and over 8 (8192 rows)."""
    w = O.normal_bf16(16, 0.02, (N, K))
    v, s, g, _ = O.quant_nvfp4(w)
    tw = L.retile_nvfp4(to_dev(v), to_dev(s))
    xf = O.bf16_to_f32(O.normal_bf16(17, 1.0, (68, K))).astype(np.float32)
    row_scale = np.float32(10.0) ** np.linspace(-6, 4.5, 68).astype(np.float32)
    chunk_scale = np.float32(2.0) ** ((np.arange(K) // 128) % 13 - 6).astype(np.float32)
    xf = xf * row_scale[:, None] * chunk_scale[None, :]
    xf[5] = 0
    x = O.f32_to_bf16(xf)
    ref = O.f32_to_bf16(O.gemm_f32(O.bf16_to_f32(x), O.dequant_nvfp4(v, s, g)))
    full = bf16_host(L.stream_nvfp4_bf16(bf16_dev(x), tw, None, g, N))
    assert_close_bf16(full, ref, "nvfp4 bf16 M=68", row_scaled=True)
    assert not full[5].any()
    xs = O.normal_bf16(18, 1.0, (16, K))
    ref16 = O.f32_to_bf16(O.gemm_f32(O.bf16_to_f32(xs), O.dequant_nvfp4(v, s, g)))
    assert_close_bf16(bf16_host(L.stream_nvfp4_bf16(bf16_dev(xs), tw, None, g, N)), ref16, "nvfp4 bf16 N(0,1)")
    for M in [1, 16, 17, 33]:
        got = bf16_host(L.stream_nvfp4_bf16(bf16_dev(x[:M]), tw, None, g, N))
        assert np.array_equal(got, full[:M]), f"nvfp4 bf16 row invariance M={M}"
    ok, table, code_of = O.scale_code_table(s)
    assert ok
    twc, _ = L.retile_nvfp4_coded(to_dev(v), to_dev(s), to_dev(code_of))
    coded = bf16_host(L.stream_nvfp4_bf16(bf16_dev(x), twc, to_dev(table), g, N))
    assert np.array_equal(coded, full)


def test_error_paths(L):
    q, s = fp8_weights(1, 16, 128)
    tw = L.retile_fp8(to_dev(q))
    x = bf16_dev(O.normal_bf16(1, 1.0, (81, 128)))
    with pytest.raises(L.LingGemmError, match=r"M must be in \[1, 80\]"):
        L.stream_fp8_pc(x, tw, to_dev(s), 16)
    with pytest.raises(L.LingGemmError, match="K must be a multiple of 128"):
        L.stream_fp8_pc(bf16_dev(O.normal_bf16(1, 1.0, (2, 100))), tw, to_dev(s), 16)
    with pytest.raises(L.LingGemmError, match="N % 16"):
        L.stream_fp8_pc(x[:2].contiguous(), tw, to_dev(s), 24)
    # a weight blob of 2 GiB or more is refused before launch (the kernels' byte offsets are 32-bit); the small
    # buffers passed are never read
    y = torch.empty((1, 16), dtype=torch.bfloat16, device=DEV)
    rc = L.lib.lq_stream_fp8_pc(x.data_ptr(), 1, tw.data_ptr(), to_dev(s).data_ptr(), y.data_ptr(), 131072, 16384,
                                None)
    assert rc != 0 and b"2^31" in L.lib.lq_last_error()
    rows = torch.zeros(32, dtype=torch.int32, device=DEV)
    yg = torch.empty((1, 32), dtype=torch.float32, device=DEV)
    rc = L.lib.lq_stream_gemm_gather_nvfp4(x.data_ptr(), yg.data_ptr(), 1, tw.data_ptr(), None, 1.0, rows.data_ptr(),
                                           rows.data_ptr(), 32, yg.data_ptr(), 16384, 262144, None)
    assert rc != 0 and b"2^31" in L.lib.lq_last_error()
    # activations of 2 GiB or more (M = 80, K = 104858 chunks) with a small weight blob (N = 16) are refused too
    rc = L.lib.lq_stream_gemm_gather_nvfp4(x.data_ptr(), yg.data_ptr(), 80, tw.data_ptr(), None, 1.0, rows.data_ptr(),
                                           rows.data_ptr(), 32, yg.data_ptr(), 104858 * 128, 16, None)
    assert rc != 0 and b"2^31" in L.lib.lq_last_error()


def test_caller_workspace(L):
    """A caller-owned workspace gives the same bits as the library's own; too small a buffer is an error."""
    N, K, I = 1024, 2048, 2048
    q, s = fp8_weights(71, N, K)
    qg, sg = fp8_weights(72, I, K)
    qu, su = fp8_weights(73, I, K)
    qd, sd = fp8_weights(74, K, I)
    tw, tg, tu, td = (L.retile_fp8(to_dev(a)) for a in (q, qg, qu, qd))
    sdev = [to_dev(a) for a in (s, sg, su, sd)]
    x = bf16_dev(O.f32_to_bf16(O.normal_f32(75, 1.0, (68, K))))
    r = bf16_dev(O.f32_to_bf16(O.normal_f32(76, 1.0, (68, K))))

    def run():
        y = L.stream_fp8_pc(x, tw, sdev[0], N)
        h = L.stream_fp8_pc_silu_mul(x, tg, sdev[1], tu, sdev[2], I)
        h2, out = L.stream_fp8_pc_ffn(x, tg, sdev[1], tu, sdev[2], td, sdev[3], r, I)
        torch.cuda.synchronize()
        return [t.view(torch.int16).cpu() for t in (y, h, h2, out)]

    own = run()
    nbytes = L.stream_workspace_bytes(68)
    assert nbytes > 0
    buf = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    try:
        L.set_workspace(buf)
        got = run()
        assert all(torch.equal(a, b) for a, b in zip(own, got))
        small = torch.empty(2 << 20, dtype=torch.uint8, device=DEV)
        L.set_workspace(small)
        with pytest.raises(L.LingGemmError, match="too small"):
            L.stream_fp8_pc(x, tw, sdev[0], N)
        with pytest.raises(L.LingGemmError, match="aligned and at least"):
            L.set_workspace(small[:1024])
    finally:
        L.set_workspace(None)
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(own, run()))


@pytest.mark.parametrize("N,K", [(5120, 5120), (5120, 6144), (7168, 5120)])
def test_full_size_one_tile_shapes(L, N, K):
    """Config 1's decode GEMV (M = 1, 5120 x 5120) and the short-range shapes of the decode step that run one tile
    per wave: parity at M = 1 and M = 17 against the oracle, and rows of M = 1 and 17 bit-identical to M = 68."""
    q, s = fp8_weights(91, N, K)
    x = O.normal_bf16(92, 1.0, (68, K))
    tw, sd, xd = L.retile_fp8(to_dev(q)), to_dev(s), bf16_dev(x)
    full = bf16_host(L.stream_fp8_pc(xd, tw, sd, N))
    for M in (1, 17):
        got = bf16_host(L.stream_fp8_pc(xd[:M].contiguous(), tw, sd, N))
        assert_close_bf16(got, O.stream_fp8_pc_bf16(x[:M], q, s), f"M={M} N={N} K={K}")
        assert np.array_equal(got, full[:M]), f"row invariance M={M} N={N} K={K}"


@pytest.mark.parametrize("K", [5120, 1024])
def test_multi_is_bit_identical_to_separate_launches(L, K):
    """stream_gemm_multi equals separate calls bit for bit (reference src/core/kernels.cuh:278-280), with matrices of
    different N in one launch: each matrix is split over its own workgroups as it would be alone (q|k|v-like shapes;
    at K = 1024 the short ranges give the FP8 matrices one tile per wave while the NVFP4 ones keep four, and the wide
    one two). FP8 and NVFP4 (raw and coded), M = 17 and 68."""
    x = O.normal_f32(70 + K, 1.0, (68, K))
    for M in (17, 68):
        xh, xinv = L.to_half_rows(to_dev(x[:M]))
        fp8 = []
        for i, N in enumerate((5120, 1024, 1024, 12352)):
            q, _ = fp8_weights(80 + i + K, N, K)
            fp8.append((L.retile_fp8(to_dev(q)), 0.25 + i, N))
        sep = [L.stream_gemm_fp8(xh, xinv, w, sc, N, K).view(torch.int32).cpu().numpy() for w, sc, N in fp8]
        ys = [torch.empty((M, N), dtype=torch.float32, device=DEV) for _, _, N in fp8]
        L.stream_gemm_multi(False, xh, xinv, [(w, None, sc, y, N) for (w, sc, N), y in zip(fp8, ys)], K)
        for i, y in enumerate(ys):
            assert np.array_equal(y.view(torch.int32).cpu().numpy(), sep[i]), f"fp8 multi M={M} matrix {i}"
        f4 = []
        for i, N in enumerate((2048, 512, 6144)):
            v, s, g, _ = O.quant_nvfp4(O.normal_bf16(90 + i + K, 0.02, (N, K)))
            ok, table, code_of = O.scale_code_table(s)
            blob, _ = L.retile_nvfp4_coded(to_dev(v), to_dev(s), to_dev(code_of))
            f4.append((blob, to_dev(table), g, N) if ok and i == 1 else (L.retile_nvfp4(to_dev(v), to_dev(s)), None, g, N))
        sep4 = [L.stream_gemm_nvfp4(xh, xinv, w, tab, g, N, K).view(torch.int32).cpu().numpy() for w, tab, g, N in f4]
        ys = [torch.empty((M, N), dtype=torch.float32, device=DEV) for _, _, _, N in f4]
        L.stream_gemm_multi(True, xh, xinv, [(w, tab, g, y, N) for (w, tab, g, N), y in zip(f4, ys)], K)
        for i, y in enumerate(ys):
            assert np.array_equal(y.view(torch.int32).cpu().numpy(), sep4[i]), f"nvfp4 multi M={M} matrix {i}"


def test_multi_with_finish_workgroups_is_bit_identical(L):
    """A multi launch whose split-K sums are done by finish workgroups (K = 17408 at M = 68: tile groups spread
    over many workgroups, long reductions) equals separate launches bit for bit, and M = 68's first rows equal an
    M = 17 launch, which finishes through its last arrivals."""
    K = 17408
    x = O.normal_f32(171, 1.0, (68, K))
    ws = []
    for i, N in enumerate((5120, 2048)):
        q, _ = fp8_weights(180 + i, N, K)
        ws.append((L.retile_fp8(to_dev(q)), 0.5 + i, N))
    outs = {}
    for M in (68, 17):
        xh, xinv = L.to_half_rows(to_dev(x[:M]))
        sep = [L.stream_gemm_fp8(xh, xinv, w, sc, N, K).view(torch.int32).cpu().numpy() for w, sc, N in ws]
        ys = [torch.empty((M, N), dtype=torch.float32, device=DEV) for _, _, N in ws]
        L.stream_gemm_multi(False, xh, xinv, [(w, None, sc, y, N) for (w, sc, N), y in zip(ws, ys)], K)
        for i, y in enumerate(ys):
            assert np.array_equal(y.view(torch.int32).cpu().numpy(), sep[i]), f"multi M={M} matrix {i}"
        outs[M] = sep
    for i in range(len(ws)):
        assert np.array_equal(outs[68][i][:17], outs[17][i]), f"row invariance matrix {i}"


def test_expired_finish_wait_leaves_counters_consistent(L):
    """Finish workgroups whose wait for the arrivals gives up (forced from the host with a zero wait limit through
    the test hook lq_debug_finish_wait_ms; every kernel still runs to its end) leave the arrival counters
    consistent: the status call reports an expiry once and clears it, and later launches with the normal limit
    equal a launch made before, bit for bit."""
    import ctypes
    K, N, M = 17408, 5120, 68  # tile groups over ~6 workgroups at 5 activation groups: finish workgroups
    x = O.normal_f32(201, 1.0, (M, K))
    q, _ = fp8_weights(202, N, K)
    w = L.retile_fp8(to_dev(q))
    xh, xinv = L.to_half_rows(to_dev(x))
    ref = L.stream_gemm_fp8(xh, xinv, w, 0.5, N, K).view(torch.int32).cpu().numpy()
    assert L.stream_ffn_deadline_status() == 0
    hook = L.lib.lq_debug_finish_wait_ms
    hook.argtypes, hook.restype = [ctypes.c_int], ctypes.c_int
    assert hook(-1) == -1
    prev = hook(0)
    try:
        for _ in range(3):
            L.stream_gemm_fp8(xh, xinv, w, 0.5, N, K)  # outputs not checked: a wait may give up
        torch.cuda.synchronize()
    finally:
        assert hook(prev) == 0
    # a zero limit makes every finish workgroup give up without waiting: the expiry is always reported
    assert L.stream_ffn_deadline_status() == 1
    assert L.stream_ffn_deadline_status() == 0  # reading cleared the flag
    for _ in range(3):
        got = L.stream_gemm_fp8(xh, xinv, w, 0.5, N, K).view(torch.int32).cpu().numpy()
        assert np.array_equal(got, ref)


def test_caller_workspace_holds_a_full_multi_launch(L):
    """lq_stream_workspace_bytes covers the largest skinny launch: a multi launch of four NVFP4 matrices (four tiles
    per wave) at M = 68, each matrix on its own workgroups, so up to four times #CUs workgroups' partials. The
    results equal those from the library's own workspace."""
    K, M = 5120, 68
    x = O.normal_f32(191, 1.0, (M, K))
    xh, xinv = L.to_half_rows(to_dev(x))
    mats = []
    for i in range(4):
        v, sc, g, _ = O.quant_nvfp4(O.normal_bf16(192 + i, 0.02, (2048, K)))
        mats.append((L.retile_nvfp4(to_dev(v), to_dev(sc)), g))

    def run():
        ys = [torch.empty((M, 2048), dtype=torch.float32, device=DEV) for _ in mats]
        L.stream_gemm_multi(True, xh, xinv, [(w, None, g, y, 2048) for (w, g), y in zip(mats, ys)], K)
        torch.cuda.synchronize()
        return [y.view(torch.int32).cpu() for y in ys]

    own = run()
    buf = torch.empty(L.stream_workspace_bytes(M), dtype=torch.uint8, device=DEV)
    try:
        L.set_workspace(buf)
        got = run()
    finally:
        L.set_workspace(None)
    assert all(torch.equal(a, b) for a, b in zip(own, got))
