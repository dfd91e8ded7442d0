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


@pytest.mark.parametrize("M,N,K", [(1, 128, 128), (130, 256, 384), (512, 384, 1024), (257, 128, 2048)])
def test_prefill_small_full(L, M, N, K):
    wq, ws, xq, xs, tw = prefill_case(L, M, N, K, 50 + M)
    y = L.prefill_fp8_block(to_dev(xq), to_dev(xs), tw, to_dev(ws), N)
    ref = O.prefill_fp8_rows(xq, xs, np.arange(M), wq, ws)
    check(bf16_host(y), ref, f"prefill M={M} N={N} K={K}")


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
    """BASELINE config 4 (M = 4096): the full GEMM on the GPU, checked on every 64th token row."""
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
