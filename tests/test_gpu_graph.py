"""The path under HIP graph capture, as the reference's engine captures its verify (src/core/speculate.cpp:473-494):
the skinny GEMMs (gate|up + SiLU*mul, down + residual, NVFP4 with BF16 activations) and the block-scaled prefill
(quantizer + GEMM, on a shape that uses the tail split) are captured once after an eager warm-up, then replayed
several times with new inputs written eagerly between replays; every replay must equal, bit for bit, eager
launches on the same inputs (split-K counters and partial buffers reset themselves inside the kernels, so no
replay depends on memory a previous one left)."""
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


def bf16(seed, shape, sigma=1.0):
    return to_dev(O.normal_bf16(seed, sigma, shape).view(np.int16)).view(torch.bfloat16)


def test_verify_step_and_nvfp4_under_graph_replay(L):
    M, H, I = 17, 1024, 2048
    qg, sg = O.quant_fp8_per_channel(O.normal_f32(81, 0.02, (I, H)))
    qu, su = O.quant_fp8_per_channel(O.normal_f32(82, 0.02, (I, H)))
    qd, sd = O.quant_fp8_per_channel(O.normal_f32(83, 0.02, (H, I)))
    tg, tu, td = (L.retile_fp8(to_dev(q)) for q in (qg, qu, qd))
    sg, su, sd = (to_dev(s) for s in (sg, su, sd))
    v, s4, g4, _ = O.quant_nvfp4(O.normal_bf16(84, 0.02, (512, H)))
    t4 = L.retile_nvfp4(to_dev(v), to_dev(s4))

    x = torch.empty((M, H), dtype=torch.bfloat16, device=DEV)
    r = torch.empty((M, H), dtype=torch.bfloat16, device=DEV)
    h = torch.empty((M, I), dtype=torch.bfloat16, device=DEV)
    y = torch.empty((M, H), dtype=torch.bfloat16, device=DEV)
    y4 = torch.empty((M, 512), dtype=torch.bfloat16, device=DEV)

    def step(hh, yy, yy4):
        L.stream_fp8_pc_silu_mul(x, tg, sg, tu, su, I, h=hh)
        L.stream_fp8_pc_residual(hh, td, sd, r, H, y=yy)
        L.stream_nvfp4_bf16(x, t4, None, g4, 512, y=yy4)

    x.copy_(bf16(85, (M, H)))
    r.copy_(bf16(86, (M, H)))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(h, y, y4)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(h, y, y4)
    for rep in range(4):
        x.copy_(bf16(90 + rep, (M, H)))
        r.copy_(bf16(100 + rep, (M, H)))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [t.view(torch.int16).clone() for t in (h, y, y4)]
        he, ye, y4e = (torch.empty_like(t) for t in (h, y, y4))
        step(he, ye, y4e)  # eager, same inputs
        torch.cuda.synchronize()
        for a, b, name in zip(got, (he, ye, y4e), ("h", "y", "nvfp4")):
            assert torch.equal(a, b.view(torch.int16)), f"replay {rep}: {name}"


def test_block_prefill_under_graph_replay(L):
    M, N, K = 300, 256, 4096  # a tail-split shape (its partials and arrival counters are in the capture)
    qw, sw = O.quant_fp8_block128(O.normal_f32(111, 0.02, (N, K)))
    tw, ws = L.retile_fp8(to_dev(qw)), to_dev(sw)
    x = torch.empty((M, K), dtype=torch.bfloat16, device=DEV)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)

    def run(yy):
        xq, xs = L.quant_act_fp8_g128(x)
        L.prefill_fp8_block(xq, xs, tw, ws, N, y=yy)

    x.copy_(bf16(112, (M, K)))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run(y)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(y)
    for rep in range(4):
        x.copy_(bf16(120 + rep, (M, K)))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = y.view(torch.int16).clone()
        ye = torch.empty_like(y)
        run(ye)
        torch.cuda.synchronize()
        assert torch.equal(got, ye.view(torch.int16)), f"prefill replay {rep}"


def test_prefill_scratch_is_not_reallocated(L):
    """A graph captured over a tail-split prefill keeps its scratch pointers valid after a larger tail-split shape has
    run eagerly (the library reserves the scratch at its bound once and never reallocates it)."""
    M, N, K = 300, 256, 4096
    qw, sw = O.quant_fp8_block128(O.normal_f32(131, 0.02, (N, K)))
    tw, ws = L.retile_fp8(to_dev(qw)), to_dev(sw)
    x = bf16(132, (M, K))
    y = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)

    def run(yy):
        xq, xs = L.quant_act_fp8_g128(x)
        L.prefill_fp8_block(xq, xs, tw, ws, N, y=yy)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run(y)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(y)
    ref = torch.empty_like(y)
    run(ref)
    # a larger tail split: more rows and weight rows, so more split tiles than the captured shape
    N2, M2 = 1024, 700
    qw2, sw2 = O.quant_fp8_block128(O.normal_f32(133, 0.02, (N2, K)))
    xq2, xs2 = L.quant_act_fp8_g128(bf16(134, (M2, K)))
    L.prefill_fp8_block(xq2, xs2, L.retile_fp8(to_dev(qw2)), to_dev(sw2), N2)
    torch.cuda.synchronize()
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), f"replay {rep} after the larger shape"


def test_finish_workgroups_under_graph_replay(L):
    """A launch whose split-K sums are done by finish workgroups (M = 68, a long K over few tile groups): its
    arrival and finish counters reset themselves, so every replay equals an eager launch on the same inputs."""
    M, N, K = 68, 1024, 8192
    q, s = O.quant_fp8_per_channel(O.normal_f32(121, 0.02, (N, K)))
    tw, sd = L.retile_fp8(to_dev(q)), to_dev(s)
    x = torch.empty((M, K), dtype=torch.bfloat16, device=DEV)
    r = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    x.copy_(bf16(122, (M, K)))
    r.copy_(bf16(123, (M, N)))
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        L.stream_fp8_pc_residual(x, tw, sd, r, N, y=y)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        L.stream_fp8_pc_residual(x, tw, sd, r, N, y=y)
    for rep in range(4):
        x.copy_(bf16(130 + rep, (M, K)))
        r.copy_(bf16(140 + rep, (M, N)))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = y.view(torch.int16).clone()
        ye = L.stream_fp8_pc_residual(x, tw, sd, r, N)
        torch.cuda.synchronize()
        assert torch.equal(got, ye.view(torch.int16)), f"replay {rep}"
    assert L.stream_ffn_deadline_status() == 0
