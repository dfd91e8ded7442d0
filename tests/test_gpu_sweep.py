"""Shape sweeps of the skinny GEMMs on the GPU against the CPU oracle, through the C ABI.

The grids cross the split regimes the launch logic chooses between: one tile or two per wave, tile groups streamed
whole by one workgroup or split over several (last-arriver and finish-workgroup finishes, the early first arrival),
ranges shorter than one tile group and ranges across three, and K from one chunk to 200. Every shape is checked
against the oracle at M = 80 (the bounds of test_gpu_stream: max relative error <= 1e-2 and mean absolute error
<= 1e-3 per row rms, on BF16 outputs) and for row invariance: the first rows of smaller launches equal the M = 80
launch bit for bit (reference tests/stream_tests.cu:206-224).
"""
import numpy as np
import pytest

import oracle as O
from test_gpu_stream import DEV, assert_close_bf16, bf16_dev, bf16_host, fp8_weights, to_dev  # noqa: F401

pytestmark = pytest.mark.gpu

ROW_SETS = (1, 16, 17, 33, 65)


@pytest.fixture(scope="module")
def L():
    import ling_gemm
    ling_gemm.init()
    return ling_gemm


@pytest.mark.parametrize("N", [16, 48, 528, 1040, 2064])
@pytest.mark.parametrize("K", [128, 384, 2048, 8192])
def test_fp8_pc_residual_sweep(L, N, K):
    """FP8 per-channel weights, BF16 activations, residual epilogue (y = x W^T s + r)."""
    q, s = fp8_weights(N * 7 + K, N, K)
    tw, sd = L.retile_fp8(to_dev(q)), to_dev(s)
    x = O.normal_bf16(N + K, 1.0, (80, K))
    r = O.normal_bf16(N + 2 * K, 1.0, (80, N))
    full = bf16_host(L.stream_fp8_pc_residual(bf16_dev(x), tw, sd, bf16_dev(r), N))
    ref = O.epi_residual_bf16(O.gemm_f32(O.bf16_to_f32(x), O.dequant_fp8_pc(q, s)), r)
    assert_close_bf16(full, ref, f"N={N} K={K}", row_scaled=True)
    for M in ROW_SETS:
        got = bf16_host(L.stream_fp8_pc_residual(bf16_dev(x[:M]), tw, sd, bf16_dev(r[:M]), N))
        assert np.array_equal(got, full[:M]), f"row invariance N={N} K={K} M={M}"
    assert L.stream_ffn_deadline_status() == 0


@pytest.mark.parametrize("N,K", [(256, 2560), (1024, 2560), (2048, 2560), (256, 25600), (1024, 25600)])
def test_nvfp4_bf16_sweep(L, N, K):
    """NVFP4 weights (raw blob, and the scale-coded blob where the scales fit the 64-entry table), BF16 activations
    converted in the kernel; the oracle check where it finishes in about a second (K = 2560), row invariance
    everywhere (K = 25600 is config 3's reduction length)."""
    v, sc, g, _ = O.quant_nvfp4(O.normal_bf16(N + K, 0.02, (N, K)))
    ok, table, code_of = O.scale_code_table(sc)
    blobs = [(L.retile_nvfp4(to_dev(v), to_dev(sc)), None)]
    if ok:
        cb, _ = L.retile_nvfp4_coded(to_dev(v), to_dev(sc), to_dev(code_of))
        blobs.append((cb, to_dev(table)))
    x = O.normal_bf16(N * 3 + K, 1.0, (80, K))
    xd = bf16_dev(x)
    ref = None
    if K <= 2560:
        ref = O.f32_to_bf16(O.gemm_f32(O.bf16_to_f32(x), O.dequant_nvfp4(v, sc, g)))
    outs = []
    for w, tab in blobs:
        full = bf16_host(L.stream_nvfp4_bf16(xd, w, tab, g, N))
        if ref is not None:
            assert_close_bf16(full, ref, f"N={N} K={K} coded={tab is not None}", row_scaled=True)
        for M in ROW_SETS + (68,):
            got = bf16_host(L.stream_nvfp4_bf16(bf16_dev(x[:M]), w, tab, g, N))
            assert np.array_equal(got, full[:M]), f"row invariance N={N} K={K} M={M} coded={tab is not None}"
        outs.append(full)
    if len(outs) == 2:
        assert np.array_equal(outs[0], outs[1]), f"coded == raw N={N} K={K}"
