"""lq_stream_fp8_pc_noalloc (the entry point that allocates nothing; its scratch is a fixed device array of the
library) against lq_stream_fp8_pc through the C ABI: bit for bit on two calls in a row, the second with a smaller
input, then a shape past the fixed scratch is rejected before anything runs."""
import ctypes as C

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
    f = ling_gemm.lib.lq_stream_fp8_pc_noalloc
    f.restype = C.c_int
    f.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p]
    return ling_gemm


def _bf16(seed, shape):
    return torch.from_numpy(O.normal_bf16(seed, 1.0, shape).view(np.int16)).to(DEV).view(torch.bfloat16)


def _noalloc(L, x, tw, s, N, K):
    M = x.shape[0]
    y = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    L._check(L.lib.lq_stream_fp8_pc_noalloc(L._ptr(x), M, L._ptr(tw), L._ptr(s), L._ptr(y), N, K, L._stream()))
    return y


def test_noalloc_equals_workspace_entry_point(L):
    # (68, 5120, 17408): finish workgroups do the split-K sums, with the partials filling 20 of the fixed scratch's 25 MiB
    cases = [(68, 5120, 17408, 500), (68, 17408, 5120, 501), (17, 5120, 17408, 502), (1, 5120, 5120, 503),
             (5, 1024, 1024, 504)]
    for M, N, K, seed in cases:  # each call after the first uses a smaller input than the one before
        q, s = O.quant_fp8_per_channel(O.normal_f32(seed, 0.02, (N, K)))
        tw = L.retile_fp8(torch.from_numpy(q).to(DEV))
        sd = torch.from_numpy(s).to(DEV)
        x = _bf16(seed + 1000, (M, K))
        got = _noalloc(L, x, tw, sd, N, K)
        want = L.stream_fp8_pc(x, tw, sd, N)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"M={M} N={N} K={K}"
        again = _noalloc(L, x, tw, sd, N, K)  # the scratch keeps the last call's contents: results do not change
        torch.cuda.synchronize()
        assert torch.equal(again.view(torch.int16), want.view(torch.int16)), f"repeat M={M} N={N} K={K}"


def test_noalloc_rejects_shapes_past_its_scratch(L):
    x = _bf16(7, (1, 128))
    y = torch.empty((1, 16), dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(16 * 128, dtype=torch.uint8, device=DEV)
    s = torch.ones(16, dtype=torch.float32, device=DEV)
    N = (1 << 16) * 128 + 4096  # more tile groups (128 rows each) than its 65536 counters (nothing is read: rejected first)
    rc = L.lib.lq_stream_fp8_pc_noalloc(L._ptr(x), 1, L._ptr(w), L._ptr(s), L._ptr(y), N, 128, L._stream())
    assert rc == 1 and "fixed scratch" in L.lib.lq_last_error().decode()
