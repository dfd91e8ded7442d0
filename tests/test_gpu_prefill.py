"""Parity of the block-scaled FP8 prefill GEMM and its 1x128 activation quantizer against the CPU oracle.

The quantizer is bit-exact (codes and scales). The GEMM is checked against the oracle's dequantize-to-FP32,
FP32-accumulate product on the same quantized operands, with the BF16 bounds of the stream GEMMs (max relative
error <= 1e-2 with denominator max(|ref|, rms(row)), mean |err| <= 1e-3), at small sizes in full and at the
config-4 shapes on a row subset; plus size-independent properties (row subsets equal the full launch, zero
rows stay zero, stray columns past N untouched).
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


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def bf16_dev(bits):
    return to_dev(bits.view(np.int16)).view(torch.bfloat16)


def bf16_host(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def check(got_bits, ref_f32, what):
    got = O.bf16_to_f32(got_bits).astype(np.float64)
    ref = O.bf16_to_f32(O.f32_to_bf16(ref_f32)).astype(np.float64)
    rms = np.sqrt(np.mean(ref * ref, axis=-1, keepdims=True)) + 1e-30
    rel = np.max(np.abs(got - ref) / np.maximum(np.abs(ref), rms))
    mae = np.mean(np.abs(got - ref))
    assert rel <= 1e-2, f"{what}: max rel {rel:.3e}"
    assert mae <= 1e-3, f"{what}: mae {mae:.3e}"


@pytest.mark.parametrize("M,K", [(1, 128), (33, 512), (300, 5120)])
def test_quant_act_fp8_g128_bit_exact(L, M, K):
    x = O.normal_bf16(40 + M, 1.0, (M, K))
    x[0, :128] = 0  # an all-zero group
    if M > 2:
        x[2, 5] = O.f32_to_bf16(np.array([3.0e4], np.float32))[0]  # an outlier
    q, s = L.quant_act_fp8_g128(bf16_dev(x))
    wq, ws = O.quant_act_fp8_g128(x)
    assert np.array_equal(s.cpu().numpy(), ws)
    assert np.array_equal(q.cpu().numpy(), wq)


def prefill_case(L, M, N, K, seed):
    w = O.normal_f32(seed, 0.02, (N, K))
    wq, ws = O.quant_fp8_block128(w)
    x = O.normal_bf16(seed + 1, 1.0, (M, K))
    xq, xs = O.quant_act_fp8_g128(x)
    tw = L.retile_fp8(to_dev(wq))
    return wq, ws, xq, xs, tw


# (300, 256, 4096) and (257, 128, 3072): every tile is split along K into 4 / 3 parts (the tail split)
@pytest.mark.parametrize("M,N,K", [(1, 128, 128), (130, 256, 384), (512, 384, 1024), (257, 128, 3072),
                                   (300, 256, 4096)])
def test_prefill_small_full(L, M, N, K):
    wq, ws, xq, xs, tw = prefill_case(L, M, N, K, 50 + M)
    y = L.prefill_fp8_block(to_dev(xq), to_dev(xs), tw, to_dev(ws), N)
    ref = O.prefill_fp8_rows(xq, xs, np.arange(M), wq, ws)
    check(bf16_host(y), ref, f"prefill M={M} N={N} K={K}")
    # split tiles add their parts in a fixed order: a second launch is bit-identical
    y2 = L.prefill_fp8_block(to_dev(xq), to_dev(xs), tw, to_dev(ws), N)
    assert np.array_equal(bf16_host(y), bf16_host(y2))


def test_prefill_stray_columns_and_rows(L):
    M, N, K = 70, 256, 256
    wq, ws, xq, xs, tw = prefill_case(L, M, N, K, 7)
    ldy = N + 64
    y = torch.full((M, ldy), 7.0, dtype=torch.bfloat16, device=DEV)
    L.prefill_fp8_block(to_dev(xq), to_dev(xs), tw, to_dev(ws), N, y=y, ldy=ldy)
    yh = y.float().cpu().numpy()
    assert np.all(yh[:, N:] == 7.0)  # nothing written past N
    ref = O.prefill_fp8_rows(xq, xs, np.arange(M), wq, ws)
    check(bf16_host(y[:, :N].contiguous()), ref, "ldy")
    # a zero activation row gives a zero output row; the launch is row-independent
    xq2 = xq.copy()
    xq2[3] = 0
    y2 = L.prefill_fp8_block(to_dev(xq2), to_dev(xs), tw, to_dev(ws), N)
    assert np.all(y2[3].float().cpu().numpy() == 0)
    y1 = L.prefill_fp8_block(to_dev(xq), to_dev(xs), tw, to_dev(ws), N)
    assert np.array_equal(bf16_host(y1)[4:], bf16_host(y2)[4:])
    sub = L.prefill_fp8_block(to_dev(xq[:17]), to_dev(xs[:17]), tw, to_dev(ws), N)
    assert np.array_equal(bf16_host(sub), bf16_host(y1)[:17])


@pytest.mark.parametrize("N,K", [(34816, 5120), (5120, 17408)])
def test_prefill_config4_shapes_row_subset(L, N, K):
    """The prefill benchmark shape (M = 4096, config 4): the full GEMM on the GPU, checked on every 64th token row."""
    M = 4096
    rng = np.random.default_rng(N)
    wq = rng.integers(0, 256, (N, K), dtype=np.uint8)
    wq[(wq & 0x7F) == 0x7F] = 0x30
    ws = (rng.random((N // 128, K // 128), dtype=np.float32) * 1e-3 + 1e-4).astype(np.float32)
    x = O.normal_bf16(N + 1, 1.0, (M, K))
    xq_d, xs_d = L.quant_act_fp8_g128(bf16_dev(x))
    tw = L.retile_fp8(to_dev(wq))
    y = L.prefill_fp8_block(xq_d, xs_d, tw, to_dev(ws), N)
    rows = np.arange(0, M, 64)
    xq = xq_d.cpu().numpy()
    xs = xs_d.cpu().numpy()
    ref = O.prefill_fp8_rows(xq, xs, rows, wq, ws)
    check(bf16_host(y)[rows], ref, f"config4 N={N} K={K}")


def test_prefill_errors(L):
    xq = torch.zeros((4, 128), dtype=torch.uint8, device=DEV)
    xs = torch.ones((4, 1), dtype=torch.float32, device=DEV)
    with pytest.raises(L.LingGemmError, match="N % 128 and K % 128 must be 0"):
        L.prefill_fp8_block(xq, xs, torch.zeros(64 * 128, dtype=torch.uint8, device=DEV), xs, 64)


# ---------------- per-tensor forms (reference prefill_gemm_fp8 / _bf16out / quant_act_fp8) ----------------
def test_quant_act_fp8_per_tensor_bit_exact(L):
    x = O.normal_f32(61, 3.0, (37, 512))
    x[0, :4] = [0.0, -0.0, 1e6, -1e6]  # zeros and saturation
    q = L.quant_act_fp8(to_dev(x), 0.0123)
    assert np.array_equal(q.cpu().numpy(), O.quant_act_fp8(x, 0.0123))


def pt_case(L, M, N, K, seed):
    rng = np.random.default_rng(seed)
    wq = rng.integers(0, 256, (N, K), dtype=np.uint8)
    wq[(wq & 0x7F) == 0x7F] = 0x38
    xq = rng.integers(0, 256, (M, K), dtype=np.uint8)
    xq[(xq & 0x7F) == 0x7F] = 0x38
    return wq, xq, L.retile_fp8(to_dev(wq))


E4M3 = np.array([O.lib.or_e4m3_decode(c) for c in range(256)], np.float64)


def pt_ref(xq, wq, alpha, rows=None):
    """Exact (float64) alpha * xq . wq^T on the given rows, and alpha * |xq| . |wq|^T (the size of the terms)."""
    rows = np.arange(xq.shape[0]) if rows is None else rows
    xd, wd = E4M3[xq[rows]], E4M3[wq]
    return alpha * (xd @ wd.T), abs(alpha) * (np.abs(xd) @ np.abs(wd).T)


def check_f32(got, ref_abs, what, base=None):
    """FP32 outputs: max |err| / max(|ref|, rms(row)) <= 2e-3. The bound is the FP8 MFMA's: it sums a 128-value
    block's products at reduced precision (measured about 6e-5 of the sum of the terms' magnitudes, a few 1e-4
    of the row's rms), well inside the 1e-2 of the BF16 outputs."""
    ref = ref_abs[0] if base is None else ref_abs[0] + base
    rms = np.sqrt(np.mean(ref * ref, axis=-1, keepdims=True)) + 1e-30
    rel = np.max(np.abs(got - ref) / np.maximum(np.abs(ref), rms))
    assert rel <= 2e-3, f"{what}: max rel {rel:.3e}"


@pytest.mark.parametrize("M,N,K", [(1, 128, 128), (200, 384, 640), (513, 256, 1024), (300, 256, 4096)])
def test_prefill_per_tensor_f32_and_accumulate(L, M, N, K):
    wq, xq, tw = pt_case(L, M, N, K, 70 + M)
    alpha = 3.0e-4
    y = L.prefill_gemm_fp8(to_dev(xq), tw, alpha, N)
    ref = pt_ref(xq, wq, alpha)
    check_f32(y.cpu().numpy().astype(np.float64), ref, f"per-tensor M={M}")
    base = O.normal_f32(M, 1.0, (M, N))
    y2 = torch.from_numpy(base).to(DEV)
    L.prefill_gemm_fp8(to_dev(xq), tw, alpha, N, y=y2, accumulate=True)
    check_f32(y2.cpu().numpy().astype(np.float64), ref, f"accumulate M={M}", base=base.astype(np.float64))


def test_prefill_per_tensor_bf16out_and_ldy(L):
    M, N, K = 90, 256, 512
    wq, xq, tw = pt_case(L, M, N, K, 5)
    ldy = N + 32
    raw = pt_ref(xq, wq, 1.0)[0]
    alpha = float(1.0 / np.sqrt(np.mean(raw * raw)))  # outputs of unit size, as the BF16 bounds assume
    y = torch.full((M, ldy), 5.0, dtype=torch.bfloat16, device=DEV)
    L.prefill_gemm_fp8_bf16out(to_dev(xq), tw, alpha, N, y=y, ldy=ldy)
    assert np.all(y[:, N:].float().cpu().numpy() == 5.0)
    check(bf16_host(y[:, :N].contiguous()), (alpha * raw).astype(np.float32), "bf16out")


def test_prefill_per_tensor_config4_rows(L):
    """Config-4 gate|up shape through the per-tensor form, checked on every 128th row."""
    M, N, K = 4096, 34816, 5120
    wq, xq, tw = pt_case(L, M, N, K, 9)
    y = L.prefill_gemm_fp8(to_dev(xq), tw, 2e-4, N)
    rows = np.arange(0, M, 128)
    check_f32(y.cpu().numpy()[rows].astype(np.float64), pt_ref(xq, wq, 2e-4, rows), "per-tensor config4")


# ---------------- rmsnorm_half (reference stream_gemm.cu:380-418) ----------------
@pytest.mark.parametrize("rows,H,gemma", [(1, 5120, True), (17, 5120, True), (3, 17408, False), (68, 1024, True),
                                         (2, 3000, False)])
def test_rmsnorm_half(L, rows, H, gemma):
    x = O.normal_f32(80 + rows, 2.0, (rows, H))
    w = O.normal_bf16(81 + rows, 0.1, (H,))
    out, xh, xinv = L.rmsnorm_half(to_dev(x), bf16_dev(w), 1e-6, gemma)
    ro, _, _ = O.rmsnorm_half(x, w, 1e-6, gemma)
    o = out.cpu().numpy()
    assert np.max(np.abs(o - ro) / (np.abs(ro) + 1e-6 * np.abs(ro).max())) <= 1e-5
    # the FP16 copy is exactly to_half_rows of the device's own FP32 output
    ch, ci = O.to_half_rows(o)
    assert np.array_equal(xh.view(torch.int16).cpu().numpy().view(np.uint16), ch)
    assert np.array_equal(xinv.cpu().numpy(), ci)


# ---------------- activation producers (reference prefill_gemm.cu:382-459, 607-637) ----------------
def _reference_test_activations(M, K, seed):
    """The reference's own test distribution (tests/prefill_tests.cu:58-60): N(0, 1) * 0.003, every 97th value
    40 times larger."""
    x = O.normal_f32(seed, 1.0, (M, K)).reshape(-1)
    x[::97] *= 40.0
    return (x * 0.003).astype(np.float32).reshape(M, K)


@pytest.mark.parametrize("M,K", [(67, 512), (5, 5120), (1, 16)])
def test_quant_act_nvfp4_bit_exact(L, M, K):
    x = _reference_test_activations(M, K, 21 + M)
    in4 = 0.0019763766  # the reference test's input scale
    q, sf = L.quant_act_nvfp4(to_dev(x), in4)
    rq, rsf = O.quant_act_nvfp4(x, in4)
    assert np.array_equal(sf.cpu().numpy(), rsf), "scales"
    assert np.array_equal(q.cpu().numpy(), rq), "codes"


def test_silu_mul_quant_nvfp4(L):
    """silu(g) * u into NVFP4. The device exp and the oracle's libm expf may round silu differently in the last
    bit, which can move a value across a BF16 rounding boundary: at most a few codes in 10^3 may differ, and
    the scales must agree except where such a value is a block's largest."""
    M, K = 17, 4096
    g = O.normal_f32(31, 2.0, (M, K))
    u = O.normal_f32(32, 1.0, (M, K))
    q, sf = L.silu_mul_quant_nvfp4(to_dev(g), to_dev(u), 0.01)
    rq, rsf = O.silu_mul_quant_nvfp4(g, u, 0.01)
    qd, sfd = q.cpu().numpy(), sf.cpu().numpy()
    assert np.mean(sfd != rsf) <= 1e-3
    assert np.mean(qd != rq) <= 3e-3


@pytest.mark.parametrize("nvfp4", [False, True])
def test_rmsnorm_quant(L, nvfp4):
    M, H = 5, 5120
    x = O.normal_f32(41, 3.0, (M, H))
    w = O.normal_bf16(42, 0.2, (H,))
    scale = 0.01 if nvfp4 else 0.02
    out, q, sf = L.rmsnorm_quant(to_dev(x), to_dev(w.view(np.int16)), 1e-6, nvfp4, scale)
    ref_out, _, _ = O.rmsnorm_quant(x, w, 1e-6, nvfp4, scale)
    outd = out.cpu().numpy()
    assert np.max(np.abs(outd - ref_out)) <= 4e-6 * np.max(np.abs(ref_out))  # FP32 rounding of the norm
    # the quantization of the kernel's own FP32 output is byte for byte the oracle's quantizer
    if nvfp4:
        rq, rsf = O.quant_act_nvfp4(outd, scale)
        assert np.array_equal(sf.cpu().numpy(), rsf)
    else:
        rq = O.quant_act_fp8(outd, scale)
    assert np.array_equal(q.cpu().numpy(), rq)
    # without the FP32 copy the bytes are the same
    _, q2, sf2 = L.rmsnorm_quant(to_dev(x), to_dev(w.view(np.int16)), 1e-6, nvfp4, scale, with_out=False)
    assert np.array_equal(q2.cpu().numpy(), q.cpu().numpy())


@pytest.mark.parametrize("nvfp4", [False, True])
def test_rmsnorm_quant_bf16(L, nvfp4):
    """rmsnorm_quant_bf16 (reference prefill_gemm.cu:640-645): the same codes and scales as rmsnorm_quant, and a BF16
    copy equal to the BF16 rounding of rmsnorm_quant's FP32 output."""
    M, H = 7, 5120
    x = O.normal_f32(43, 3.0, (M, H))
    w = to_dev(O.normal_bf16(44, 0.2, (H,)).view(np.int16))
    scale = 0.01 if nvfp4 else 0.02
    out, q, sf = L.rmsnorm_quant(to_dev(x), w, 1e-6, nvfp4, scale)
    ob, qb, sfb = L.rmsnorm_quant_bf16(to_dev(x), w, 1e-6, nvfp4, scale)
    assert np.array_equal(qb.cpu().numpy(), q.cpu().numpy())
    if nvfp4:
        assert np.array_equal(sfb.cpu().numpy(), sf.cpu().numpy())
    want = O.f32_to_bf16(out.cpu().numpy())
    assert np.array_equal(ob.view(torch.int16).cpu().numpy().view(np.uint16), want)
    _, q2, _ = L.rmsnorm_quant_bf16(to_dev(x), w, 1e-6, nvfp4, scale, with_out=False)
    assert np.array_equal(q2.cpu().numpy(), q.cpu().numpy())


def test_quant_act_fp8_bf16in_bit_exact(L):
    """quant_act_fp8_bf16in (reference prefill_gemm.cu:626-630): the bytes quant_act_fp8 gives for the FP32 values
    the BF16 copy holds."""
    xb = O.f32_to_bf16(O.normal_f32(62, 3.0, (37, 512)))
    xb[0, :4] = O.f32_to_bf16(np.array([0.0, -0.0, 1e6, -1e6], np.float32))
    q = L.quant_act_fp8_bf16in(to_dev(xb.view(np.int16)).view(torch.bfloat16), 0.0123)
    assert np.array_equal(q.cpu().numpy(), O.quant_act_fp8(O.bf16_to_f32(xb), 0.0123))


def test_activation_producer_errors(L):
    x = torch.zeros((2, 24), dtype=torch.float32, device=DEV)
    with pytest.raises(L.LingGemmError, match="K % 16"):
        L.quant_act_nvfp4(x, 1.0)
    w = torch.zeros((1000,), dtype=torch.int16, device=DEV)
    with pytest.raises(L.LingGemmError, match="H % 1024 must be 0"):
        L.rmsnorm_quant(torch.zeros((1, 1000), dtype=torch.float32, device=DEV), w, 1e-6, True, 1.0)


# ---------------- NVFP4 prefill (reference prefill_gemm.cu:344-376, 593-704) ----------------
def _nvfp4_operands(L, M, N, K, seed):
    w = O.normal_bf16(seed, 0.02, (N, K))
    wv, ws, g, _ = O.quant_nvfp4(w)
    x = O.normal_f32(seed + 1, 1.0, (M, K))
    xq, xs = O.quant_act_nvfp4(x, 0.0625)
    return wv, ws, xq, xs


def check_f32_tight(got, ref, what):
    """FP32 outputs of exactly dequantized operands (every product exact in FP32): max |err| / max(|ref|, rms(row))
    <= 1e-5 against the float64 product."""
    rms = np.sqrt(np.mean(ref * ref, axis=-1, keepdims=True)) + 1e-30
    rel = np.max(np.abs(got - ref) / np.maximum(np.abs(ref), rms))
    assert rel <= 1e-5, f"{what}: max rel {rel:.3e}"


@pytest.mark.parametrize("M,N,K", [(1, 128, 128), (130, 384, 512), (300, 256, 2048), (513, 640, 1024)])
def test_prefill_nvfp4(L, M, N, K):
    wv, ws, xq, xs = _nvfp4_operands(L, M, N, K, 80 + M)
    raw = L.retile_nvfp4(to_dev(wv), to_dev(ws))
    alpha = 0.37
    y = L.prefill_gemm_nvfp4(to_dev(xq), to_dev(xs), raw, alpha, N).cpu().numpy()
    ref = O.prefill_nvfp4_rows(xq, xs, np.arange(M), wv, ws, alpha)
    check_f32_tight(y.astype(np.float64), ref, f"nvfp4 prefill M={M} N={N} K={K}")
    # the coded blob with its raw scales gives the same bits
    ok, table, code_of = O.scale_code_table(ws)
    if ok:
        coded, rs = L.retile_nvfp4_coded(to_dev(wv), to_dev(ws), to_dev(code_of))
        y2 = L.prefill_gemm_nvfp4(to_dev(xq), to_dev(xs), coded, alpha, N, wsf=rs).cpu().numpy()
        assert np.array_equal(y2, y)
    # accumulate into rows ldy apart
    ldy = N + 32
    base = torch.full((M, ldy), 0.5, dtype=torch.float32, device=DEV)
    L.prefill_gemm_nvfp4(to_dev(xq), to_dev(xs), raw, alpha, N, y=base, ldy=ldy, accumulate=True)
    b = base.cpu().numpy()
    assert np.all(b[:, N:] == 0.5)
    check_f32_tight(b[:, :N].astype(np.float64), ref + 0.5, "nvfp4 prefill accumulate")


def test_prefill_nvfp4_device_quantized_activations(L):
    """The activations from quant_act_nvfp4 on the GPU, a larger shape, every 16th row checked."""
    M, N, K = 1024, 2048, 2048
    w = O.normal_bf16(90, 0.02, (N, K))
    wv, ws, _, _ = O.quant_nvfp4(w)
    raw = L.retile_nvfp4(to_dev(wv), to_dev(ws))
    x = O.normal_f32(91, 1.0, (M, K))
    xq, xs = L.quant_act_nvfp4(to_dev(x), 0.03)
    y = L.prefill_gemm_nvfp4(xq, xs, raw, 1.0, N).cpu().numpy()
    rows = np.arange(0, M, 16)
    ref = O.prefill_nvfp4_rows(xq.cpu().numpy(), xs.cpu().numpy(), rows, wv, ws, 1.0)
    check_f32_tight(y[rows].astype(np.float64), ref, "nvfp4 prefill device-quantized")


def test_prefill_swiglu_nvfp4(L):
    """gate|up into the down projection's NVFP4 input. The float64 products rounded to FP32 can differ from the
    GPU's FP32 sums in the last bit, which may move a value across a BF16 rounding boundary: at most a few codes
    in 10^3 and scales in 10^3 may differ from the oracle's quantization of the exact products."""
    M, N, K = 300, 384, 1024
    gv_, gs_, xq, xs = _nvfp4_operands(L, M, N, K, 95)
    uw = O.normal_bf16(97, 0.02, (N, K))
    uv_, us_, _, _ = O.quant_nvfp4(uw)
    gate = L.retile_nvfp4(to_dev(gv_), to_dev(gs_))
    up = L.retile_nvfp4(to_dev(uv_), to_dev(us_))
    ag, au, osc = 0.8, 1.3, 0.05
    q, sf = L.prefill_swiglu_nvfp4(to_dev(xq), to_dev(xs), gate, ag, up, au, N, osc)
    g = O.prefill_nvfp4_rows(xq, xs, np.arange(M), gv_, gs_, ag).astype(np.float32)
    u = O.prefill_nvfp4_rows(xq, xs, np.arange(M), uv_, us_, au).astype(np.float32)
    rq, rsf = O.silu_mul_quant_nvfp4(g, u, osc)
    qd, sfd = q.cpu().numpy(), sf.cpu().numpy()
    assert np.mean(sfd != rsf) <= 1e-3
    assert np.mean(qd != rq) <= 3e-3
    # coded blobs with their raw scales give the same bytes
    ok1, _, c1 = O.scale_code_table(gs_)
    ok2, _, c2 = O.scale_code_table(us_)
    if ok1 and ok2:
        gc, gr = L.retile_nvfp4_coded(to_dev(gv_), to_dev(gs_), to_dev(c1))
        uc, ur = L.retile_nvfp4_coded(to_dev(uv_), to_dev(us_), to_dev(c2))
        q2, sf2 = L.prefill_swiglu_nvfp4(to_dev(xq), to_dev(xs), gc, ag, uc, au, N, osc, gate_sf=gr, up_sf=ur)
        assert np.array_equal(q2.cpu().numpy(), qd) and np.array_equal(sf2.cpu().numpy(), sfd)


def test_rmsnorm_quant_row_widths(L):
    """Rows of 1024 (one wave), 20480 (two blocks a thread) and 65536 (four) values, and the limit beyond."""
    for H in (1024, 20480, 65536):
        x = O.normal_f32(43, 2.0, (3, H))
        w = O.normal_bf16(44, 0.2, (H,))
        out, q, sf = L.rmsnorm_quant(to_dev(x), to_dev(w.view(np.int16)), 1e-6, True, 0.01)
        ref_out, _, _ = O.rmsnorm_quant(x, w, 1e-6, True, 0.01)
        outd = out.cpu().numpy()
        assert np.max(np.abs(outd - ref_out)) <= 4e-6 * np.max(np.abs(ref_out)), H
        rq, rsf = O.quant_act_nvfp4(outd, 0.01)
        assert np.array_equal(q.cpu().numpy(), rq) and np.array_equal(sf.cpu().numpy(), rsf), H
    w = torch.zeros((66560,), dtype=torch.int16, device=DEV)
    with pytest.raises(L.LingGemmError, match="at most 65536"):
        L.rmsnorm_quant(torch.zeros((1, 66560), dtype=torch.float32, device=DEV), w, 1e-6, True, 1.0)


def test_quant_act_fp8_g128_rounding_boundaries(L):
    """Scaled values x * (1 / s) on and next to E4M3 rounding midpoints, where one FP32 rounding decides the code:
    groups with s = 3 exactly (amax 1344) holding 3 x every midpoint of [2^-9, 448], groups with an inexact s
    (amax 1000) holding the BF16 values nearest to midpoint x s and their BF16 neighbours, and groups of tiny and
    huge magnitudes."""
    codes = np.arange(0, 0x7f, dtype=np.uint8)
    vals = np.array([_e4m3(c) for c in codes], np.float32)
    mids = ((vals[:-1].astype(np.float64) + vals[1:]) / 2)
    rows = []
    for amax, scale in ((1344.0, 3.0), (1000.0, 1000.0 / 448.0)):
        tgt = np.concatenate([mids, -mids]) * scale
        b = O.f32_to_bf16(tgt.astype(np.float32))
        nb = np.concatenate([b, b + 1, b - 1]).astype(np.uint16)
        nb = nb[np.abs(O.bf16_to_f32(nb)) <= amax]
        n = -(-len(nb) // 127) * 127
        nb = np.resize(nb, n).reshape(-1, 127)
        head = np.full((nb.shape[0], 1), O.f32_to_bf16(np.array([amax], np.float32))[0], np.uint16)
        rows.append(np.concatenate([head, nb], axis=1))
    g = np.concatenate(rows).reshape(-1)
    tiny = O.normal_bf16(71, 1e-30, (1, 128)).reshape(-1)
    huge = O.normal_bf16(72, 1e30, (1, 128)).reshape(-1)
    g = np.concatenate([g, tiny, huge])
    x = np.resize(g, -(-g.size // 1024) * 1024).reshape(-1, 1024)
    q, s = L.quant_act_fp8_g128(bf16_dev(x))
    wq, ws = O.quant_act_fp8_g128(x)
    assert np.array_equal(s.cpu().numpy(), ws)
    assert np.array_equal(q.cpu().numpy(), wq)


def _e4m3(c):
    e, m = (int(c) >> 3) & 15, int(c) & 7
    return (m / 8.0) * 2.0 ** -6 if e == 0 else (1 + m / 8.0) * 2.0 ** (e - 7)


def test_quant_act_nvfp4_rounding_boundaries(L):
    """E2M1 codes at their rounding boundaries: with input scale 1 and a block whose largest magnitude is 6, the
    block scale is E4M3(1) and every value is encoded unscaled, so blocks holding each E2M1 midpoint (0.25, 0.75,
    1.25, 1.75, 2.5, 3.5, 5), its BF16 neighbours, both signs, zeros, -0 and small negatives test the
    round-to-nearest-even encoding (ties to the even code) bit for bit against the oracle."""
    mids = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], np.float32)
    b = O.f32_to_bf16(mids)
    vals = np.concatenate([b, b + 1, b - 1]).astype(np.uint16)
    vals = O.bf16_to_f32(vals)
    pool = np.concatenate([vals, -vals, np.array([0.0, -0.0, -0.1, -1e-8, 1e-8, 6.0, -6.0, 0.5, 3.0], np.float32)])
    blocks = []
    for i in range(0, len(pool), 15):
        blk = np.zeros(16, np.float32)
        part = pool[i:i + 15]
        blk[:len(part)] = part
        blk[15] = 6.0  # the block's largest magnitude: scale E4M3(6 / 6) = 1
        blocks.append(blk)
    x = np.concatenate(blocks)
    x = np.resize(x, -(-x.size // 256) * 256).reshape(-1, 256).astype(np.float32)
    q, sf = L.quant_act_nvfp4(to_dev(x), 1.0)
    rq, rsf = O.quant_act_nvfp4(x, 1.0)
    assert np.array_equal(sf.cpu().numpy(), rsf), "scales"
    assert np.array_equal(q.cpu().numpy(), rq), "codes"


def _band_parity(got, ref, v64, input_scale, rel=4e-6):
    """FP8 codes from an FP32 formula with one exp: equal to the oracle's wherever the float64 value's band of
    `rel` fixes the code; elsewhere (a BF16 rounding boundary inside the band, where the device exp and libm expf
    may land on either side) one of the band's two codes. Returns the fraction left to the band."""
    lo, hi = O.fp8_code_band(v64, input_scale, rel)
    fixed = lo == hi
    assert np.array_equal(got[fixed], ref[fixed]), f"{int(np.sum(got[fixed] != ref[fixed]))} fixed codes differ"
    assert np.all((got[~fixed] == lo[~fixed]) | (got[~fixed] == hi[~fixed]))
    return float(np.mean(~fixed))


def _gated_v64(x, z, w, eps):
    x64, z64 = x.astype(np.float64), z.astype(np.float64)
    rstd = 1.0 / np.sqrt((x64 ** 2).sum(axis=1, keepdims=True) / 128 + eps)
    return x64 * rstd * O.bf16_to_f32(w).astype(np.float64) * (z64 / (1 + np.exp(-z64)))


@pytest.mark.parametrize("rows", [1, 13, 4096])
def test_gated_rmsnorm_fp8(L, rows):
    """gated_rmsnorm_fp8 (reference prefill_gemm.cu:461-482, 648-653) against the oracle: the sum of squares,
    rstd and the products are the same FP32 operations in the same order, so the codes are bit-exact except where
    silu's exp may move a value across a BF16 rounding boundary (then one of the two neighbouring codes)."""
    x = O.normal_f32(61 + rows, 1.5, (rows, 128))
    z = O.normal_f32(62 + rows, 2.0, (rows, 128))
    w = O.normal_bf16(63, 0.6, (128,))
    eps, sc = 1e-6, 0.02
    q = L.gated_rmsnorm_fp8(to_dev(x), to_dev(z), to_dev(w.view(np.int16)), eps, sc).cpu().numpy()
    ref = O.gated_rmsnorm_fp8(x, z, w, eps, sc)
    assert _band_parity(q, ref, _gated_v64(x, z, w, eps), sc) < 0.01


def test_gated_rmsnorm_fp8_bf16_inputs(L):
    """gated_rmsnorm_fp8_bf16 (reference prefill_gemm.cu:655-660): BF16 x and z give the bytes the FP32 entry point
    gives for their exact FP32 widening, and match the oracle on that widening."""
    rows = 300
    xb = O.normal_bf16(71, 1.5, (rows, 128))
    zb = O.normal_bf16(72, 2.0, (rows, 128))
    w = O.normal_bf16(73, 0.6, (128,))
    wd = to_dev(w.view(np.int16))
    qb = L.gated_rmsnorm_fp8(bf16_dev(xb), bf16_dev(zb), wd, 1e-6, 0.03).cpu().numpy()
    x, z = O.bf16_to_f32(xb), O.bf16_to_f32(zb)
    qf = L.gated_rmsnorm_fp8(to_dev(x), to_dev(z), wd, 1e-6, 0.03).cpu().numpy()
    assert np.array_equal(qb, qf)
    assert _band_parity(qb, O.gated_rmsnorm_fp8(x, z, w, 1e-6, 0.03), _gated_v64(x, z, w, 1e-6), 0.03) < 0.01


def test_gated_rmsnorm_fp8_edges(L):
    """Known answers on the device (x = 1, w = 1, z = 20: every code E4M3(20); z = 0: zero codes; a huge w
    saturates to 0x7E), rows = 0 does nothing, and D != 128 fails as the reference does."""
    one = torch.ones((8, 128), dtype=torch.float32, device=DEV)
    w1 = torch.full((128,), 0x3F80, dtype=torch.int16, device=DEV)
    q = L.gated_rmsnorm_fp8(one, torch.full_like(one, 20.0), w1, 0.0, 1.0).cpu().numpy()
    assert np.all(q == torch.tensor([20.0]).to(torch.float8_e4m3fn).view(torch.uint8).item())
    assert np.all(L.gated_rmsnorm_fp8(one, torch.zeros_like(one), w1, 0.0, 1.0).cpu().numpy() & 0x7F == 0)
    wbig = torch.full((128,), 0x4780, dtype=torch.int16, device=DEV)
    assert np.all(L.gated_rmsnorm_fp8(one, torch.full_like(one, 20.0), wbig, 0.0, 1.0).cpu().numpy() == 0x7E)
    assert L.gated_rmsnorm_fp8(one[:0], one[:0], w1, 1e-6, 1.0).shape == (0, 128)
    half = torch.ones((4, 64), dtype=torch.float32, device=DEV)
    with pytest.raises(L.LingGemmError, match="D must be 128"):
        L.gated_rmsnorm_fp8(half, half, w1, 1e-6, 1.0)


@pytest.mark.parametrize("shape", [(1, 4), (7, 4096), (4096, 4096)])
def test_sigmoid_mul_fp8(L, shape):
    """sigmoid_mul_fp8 (reference prefill_gemm.cu:484-494, 662-665) against the oracle, bit-exact outside the
    band where the device exp and libm expf may round x / (1 + e^-g) to different BF16 neighbours."""
    x = O.normal_f32(81 + shape[0], 3.0, shape)
    g = O.normal_f32(82 + shape[0], 4.0, shape)
    q = L.sigmoid_mul_fp8(to_dev(x), to_dev(g), 0.05).cpu().numpy()
    ref = O.sigmoid_mul_fp8(x, g, 0.05)
    v64 = x.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))
    assert _band_parity(q, ref, v64, 0.05) < 0.01


def test_sigmoid_mul_fp8_edges(L):
    """gate = 0 halves x, a large gate keeps it, a very negative one gives zero codes; n % 4 != 0 is refused."""
    xs = np.array([[1.0, -3.0, 448.0, 0.5, 900.0, -0.001, 7.0, 2.5]], np.float32)
    got = lambda gv: L.sigmoid_mul_fp8(to_dev(xs), to_dev(np.full_like(xs, gv)), 1.0).cpu().numpy()
    assert np.array_equal(got(0.0), O.quant_act_fp8(xs / 2, 1.0))
    assert np.array_equal(got(40.0), O.quant_act_fp8(xs, 1.0))
    assert np.all(got(-200.0) & 0x7F == 0)
    odd = torch.ones(6, dtype=torch.float32, device=DEV)
    with pytest.raises(L.LingGemmError, match="n % 4"):
        L.sigmoid_mul_fp8(odd, odd, 1.0)
