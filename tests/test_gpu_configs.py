"""Every benchmark configuration's exact shapes on the GPU, checked against the CPU oracle through the C ABI
(the reference's own check style: tests/stream_tests.cu:189-225, a double/FP32 product over exactly-decoded
operands).

Bounds (the path's accuracy target): on BF16 outputs max relative error <= 1e-2 and mean |got - ref| <= 1e-3, with
the relative error of an element |got - ref| / max(|ref|, rms(ref row)); dequantized weights bit-exact (tested in
test_gpu_stream.py). Weights ~N(0, 0.02) quantized per the configuration (FP8 per channel; NVFP4 round-to-nearest),
activations ~N(0, 1) in BF16, from the oracle's portable generator. The 151936-row head uses random E4M3 codes with
random per-channel scales (its 778 MB of normal draws would dominate the suite) and is checked on a deterministic
subset of output channels.
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


def to_dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def bf16_dev(bits: np.ndarray) -> torch.Tensor:
    return to_dev(bits.view(np.int16)).view(torch.bfloat16)


def bf16_host(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def assert_close(got_bits, ref_bits, what):
    got = O.bf16_to_f32(got_bits).astype(np.float64)
    ref = O.bf16_to_f32(ref_bits).astype(np.float64)
    assert np.isfinite(got).all(), what
    rms = np.sqrt(np.mean(ref * ref, axis=-1, keepdims=True)) + 1e-30
    rel = np.max(np.abs(got - ref) / np.maximum(np.abs(ref), rms))
    mae = np.mean(np.abs(got - ref))
    print(f"{what}: max rel {rel:.2e} mae {mae:.2e}", flush=True)
    assert rel <= 1e-2, f"{what}: max rel err {rel:.3e}"
    assert mae <= 1e-3, f"{what}: mean abs err {mae:.3e}"


def fp8_pc(seed, N, K):
    return O.quant_fp8_per_channel(O.normal_f32(seed, 0.02, (N, K)))


def random_fp8_pc(seed, N, K):
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 256, (N, K), dtype=np.uint8)
    q[(q & 0x7F) == 0x7F] = 0x30  # no NaN codes
    s = (rng.random(N, dtype=np.float32) * 4e-4 + 2e-5).astype(np.float32)
    return q, s


def test_config1_decode_gemv(L):
    """Config 1: M = 1, K = N = 5120, FP8 per channel, BF16 out."""
    q, s = fp8_pc(0x4C510001, 5120, 5120)
    x = O.normal_bf16(0x4C510101, 1.0, (1, 5120))
    y = L.stream_fp8_pc(bf16_dev(x), L.retile_fp8(to_dev(q)), to_dev(s), 5120)
    assert_close(bf16_host(y), O.stream_fp8_pc_bf16(x, q, s), "config 1")


@pytest.fixture(scope="module")
def config2(L):
    I, H = 17408, 5120
    qg, sg = fp8_pc(0x4C510002, I, H)
    qu, su = fp8_pc(0x4C510012, I, H)
    qd, sd = fp8_pc(0x4C510022, H, I)
    dev = dict(tg=L.retile_fp8(to_dev(qg)), tu=L.retile_fp8(to_dev(qu)), td=L.retile_fp8(to_dev(qd)),
               sg=to_dev(sg), su=to_dev(su), sd=to_dev(sd))
    return (qg, sg, qu, su, qd, sd), dev


@pytest.mark.parametrize("M", [17, 68])
def test_config2_verify_mlp_full_size(L, config2, M):
    """Config 2 at its full size (and the same MLP at config 5's M = 68): gate|up + SiLU*mul into h [M][17408], then
    down + BF16 residual from the GPU's h, each against the oracle (FP32 accumulate, one BF16 rounding)."""
    (qg, sg, qu, su, qd, sd), d = config2
    I, H = 17408, 5120
    x = O.normal_bf16(0x4C510102 + M, 1.0, (M, H))
    r = O.normal_bf16(0x4C510202 + M, 1.0, (M, H))
    h = L.stream_fp8_pc_silu_mul(bf16_dev(x), d["tg"], d["sg"], d["tu"], d["su"], I)
    y = L.stream_fp8_pc_residual(h, d["td"], d["sd"], bf16_dev(r), H)
    hg = bf16_host(h)
    xf = O.bf16_to_f32(x)
    # the oracle on a channel subset of gate|up at M = 68 (its full 12 G multiply-adds are the slow part)
    cols = np.arange(I) if M == 17 else np.concatenate([np.arange(0, 1024), np.arange(9000, 9512), np.arange(I - 512, I)])
    g = O.gemm_f32(xf, O.dequant_fp8_pc(qg[cols], sg[cols]))
    u = O.gemm_f32(xf, O.dequant_fp8_pc(qu[cols], su[cols]))
    assert_close(hg[:, cols], O.epi_silu_mul_bf16(g, u), f"config 2 h M={M}")
    yref = O.epi_residual_bf16(O.gemm_f32(O.bf16_to_f32(hg), O.dequant_fp8_pc(qd, sd)), r)
    assert_close(bf16_host(y), yref, f"config 2 y M={M}")
    if M == 68:
        # rows do not depend on M: down at M = 68 is finished by finish workgroups, at M = 17 by its last arrivals
        y17 = L.stream_fp8_pc_residual(h[:17].contiguous(), d["td"], d["sd"], bf16_dev(r[:17]), H)
        assert np.array_equal(bf16_host(y17), bf16_host(y)[:17])
    # the one-launch FFN gives the same bits
    h2, y2 = L.stream_fp8_pc_ffn(bf16_dev(x), d["tg"], d["sg"], d["tu"], d["su"], d["td"], d["sd"], bf16_dev(r), I)
    assert np.array_equal(bf16_host(h2), hg) and np.array_equal(bf16_host(y2), bf16_host(y))
    assert L.stream_ffn_deadline_status() == 0


@pytest.mark.parametrize("coded", [False, True])
def test_config3_drafter_fc_nvfp4(L, coded):
    """Config 3: NVFP4 drafter fc, M = 16, K = 25600, N = 5120, BF16 activations, raw and scale-coded blobs."""
    N, K, M = 5120, 25600, 16
    v, s, g, _ = L.quantize_nvfp4(O.normal_bf16(0x4C510003, 0.02, (N, K)))
    x = O.normal_bf16(0x4C510103, 1.0, (M, K))
    if coded:
        ok, table, code_of = L.scale_code_table(s)
        assert ok
        tw, _raw = L.retile_nvfp4_coded(to_dev(v), to_dev(s), to_dev(code_of))
        tab = to_dev(table)
    else:
        tw, tab = L.retile_nvfp4(to_dev(v), to_dev(s)), None
    y = L.stream_nvfp4_bf16(bf16_dev(x), tw, tab, g, N)
    ref = O.f32_to_bf16(O.gemm_f32(O.bf16_to_f32(x), O.dequant_nvfp4(v, s, g)))
    assert_close(bf16_host(y), ref, f"config 3 coded={coded}")


@pytest.mark.parametrize("N,K,resid", [(12352, 5120, False), (5120, 6144, True), (7168, 5120, False)])
def test_config5_projections_m68(L, N, K, resid):
    """Config 5's projections at M = 68: DeltaNet in_proj 5120 -> 12352, out_proj / o_proj 6144 -> 5120 with the
    residual, attention QKV 5120 -> 7168."""
    M = 68
    q, s = fp8_pc(0x4C510005 + N + K, N, K)
    x = O.normal_bf16(0x4C510105 + N, 1.0, (M, K))
    tw, sd = L.retile_fp8(to_dev(q)), to_dev(s)
    if resid:
        r = O.normal_bf16(0x4C510205, 1.0, (M, N))
        y = L.stream_fp8_pc_residual(bf16_dev(x), tw, sd, bf16_dev(r), N)
        ref = O.epi_residual_bf16(O.gemm_f32(O.bf16_to_f32(x), O.dequant_fp8_pc(q, s)), r)
    else:
        y = L.stream_fp8_pc(bf16_dev(x), tw, sd, N)
        ref = O.stream_fp8_pc_bf16(x, q, s)
    assert_close(bf16_host(y), ref, f"config 5 {N}x{K} M=68")


def test_config5_lm_head_m68_column_subset(L):
    """Config 5's head, 5120 -> 151936 at M = 68, against the oracle on 6 channel ranges spread over the matrix (the
    first and last tile groups included)."""
    N, K, M = 151936, 5120, 68
    q, s = random_fp8_pc(0x4C510015, N, K)
    x = O.normal_bf16(0x4C510115, 1.0, (M, K))
    y = bf16_host(L.stream_fp8_pc(bf16_dev(x), L.retile_fp8(to_dev(q)), to_dev(s), N))
    for n0 in (0, 4096, 65536 + 48, 100000, 151936 - 1024 - 256, 151936 - 256):
        n1 = n0 + 256
        ref = O.stream_fp8_pc_bf16(x, q, s, n0, n1)
        assert_close(y[:, n0:n1], ref[:, n0:n1], f"config 5 head [{n0}, {n1})")
