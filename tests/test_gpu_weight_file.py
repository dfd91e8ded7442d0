"""The kernel-order weight file on the GPU: each entry loaded from a compiled file is byte-identical to the device
retile of the same checkpoint tensors (lq_retile_*, the reference's load-time path, src/core/model.cu:131-186),
and the GEMMs fed from the file give bit-identical outputs to the GEMMs fed from the device retile."""
import os

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


def u8(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint8))


@pytest.fixture(scope="module")
def weights(tmp_path_factory):
    import safetensors.torch as st
    import ling_compile as LC
    K = 2560
    v, s, g, _ = O.quant_nvfp4(O.normal_bf16(31, 0.02, (1024, K)))
    qc, sc = O.quant_fp8_per_channel(O.normal_f32(32, 0.02, (512, K)))
    qb, sb = O.quant_fp8_block128(O.normal_f32(33, 0.02, (256, K)))
    d = str(tmp_path_factory.mktemp("ckpt"))
    st.save_file({
        "l.gate.weight": u8(v), "l.gate.weight_scale": u8(s).view(torch.float8_e4m3fn),
        "l.gate.weight_scale_2": torch.tensor(g, dtype=torch.float32),
        "l.up.weight": u8(qc).view(torch.float8_e4m3fn), "l.up.weight_scale": torch.from_numpy(sc).reshape(-1, 1),
        "l.down.weight": u8(qb).view(torch.float8_e4m3fn), "l.down.weight_scale_inv": torch.from_numpy(sb),
    }, os.path.join(d, "model.safetensors"))
    out = os.path.join(d, "model.lqw")
    assert LC.compile_checkpoint(d, out) == 3
    f = LC.WeightFile(out)
    return dict(K=K, v=v, s=s, g=g, qc=qc, sc=sc, qb=qb, sb=sb, f=f)


def test_loaded_nvfp4_coded_matches_device_retile(L, weights):
    W, K = weights, weights["K"]
    lw = W["f"].load("l.gate", DEV)
    ok, table, code_of = O.scale_code_table(W["s"])
    assert ok and lw.kind == L.WENTRY_NVFP4_CODED and (lw.N, lw.K) == (1024, K)
    blob, raw = L.retile_nvfp4_coded(to_dev(W["v"]), to_dev(W["s"]), to_dev(code_of))
    assert torch.equal(lw.w, blob) and torch.equal(lw.raw_scales, raw) and torch.equal(lw.table, to_dev(table))
    x = O.normal_f32(34, 1.0, (17, K))
    xh, xinv = L.to_half_rows(to_dev(x))
    a = L.stream_gemm_nvfp4(xh, xinv, blob, to_dev(table), W["g"], 1024, K)
    b = L.stream_gemm_nvfp4(xh, xinv, lw.w, lw.table, lw.weight_scale, lw.N, lw.K)
    assert torch.equal(a, b)


def test_loaded_fp8_per_channel_matches_device_retile(L, weights):
    W, K = weights, weights["K"]
    lw = W["f"].load("l.up", DEV)
    assert lw.kind == L.WENTRY_FP8 and lw.svec is not None
    tw = L.retile_fp8(to_dev(W["qc"]))
    assert torch.equal(lw.w, tw) and torch.equal(lw.svec, to_dev(W["sc"]))
    x = to_dev(O.f32_to_bf16(O.normal_f32(35, 1.0, (68, K))).view(np.int16)).view(torch.bfloat16)
    assert torch.equal(L.stream_fp8_pc(x, tw, to_dev(W["sc"]), 512), L.stream_fp8_pc(x, lw.w, lw.svec, lw.N))


def test_loaded_fp8_block_matches_device_retile(L, weights):
    W, K = weights, weights["K"]
    lw = W["f"].load("l.down", DEV)
    assert lw.kind == L.WENTRY_FP8 and lw.block_scales is not None and lw.block_scales.shape == (2, K // 128)
    tw = L.retile_fp8(to_dev(W["qb"]))
    assert torch.equal(lw.w, tw) and torch.equal(lw.block_scales, to_dev(W["sb"]))
    xb = O.f32_to_bf16(O.normal_f32(36, 1.0, (300, K)))
    xq, xs = L.quant_act_fp8_g128(to_dev(xb.view(np.int16)).view(torch.bfloat16))
    a = L.prefill_fp8_block(xq, xs, tw, to_dev(W["sb"]), 256)
    b = L.prefill_fp8_block(xq, xs, lw.w, lw.block_scales, lw.N)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
