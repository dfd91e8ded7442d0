"""The HIP path against the committed golden fixtures (tests/golden/vectors.json), read as data: no oracle call
produces the expected values here. Layouts and quantizers are bit-exact; GEMM outputs are held to the same
bounds as the oracle parity tests (BF16 outputs: max relative error <= 1e-2 of max(|ref|, row rms), mean
absolute error <= 1e-3; FP32 products: 1e-5 of the row's largest magnitude)."""
import json
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = json.load(open(os.path.join(HERE, "golden", "vectors.json")))


@pytest.fixture(scope="module")
def L():
    import ling_gemm
    ling_gemm.init()
    return ling_gemm


def arr(key, dtype, shape=None):
    a = np.frombuffer(bytes.fromhex(key), dtype).copy()
    return a.reshape(shape) if shape is not None else a


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def bf16_to_f32(b):
    return (b.astype(np.uint32) << 16).view(np.float32)


def test_golden_stream_fp8_pc(L):
    g = GOLD["stream_fp8_pc"]
    x = arr(g["x_bf16"], np.uint16, (3, 256))
    q = arr(g["q"], np.uint8, (16, 256))
    s = arr(g["s"], np.float32)
    tw = L.retile_fp8(dev(q))
    assert tw.cpu().numpy().tobytes() == bytes.fromhex(g["tiled"])
    y = L.stream_fp8_pc(dev(x.view(np.int16)).view(torch.bfloat16), tw, dev(s), 16)
    got = bf16_to_f32(y.view(torch.int16).cpu().numpy().view(np.uint16)).astype(np.float64)
    ref = bf16_to_f32(arr(g["y_bf16"], np.uint16, (3, 16))).astype(np.float64)
    rms = np.sqrt(np.mean(ref ** 2, axis=1, keepdims=True))
    assert np.max(np.abs(got - ref) / np.maximum(np.abs(ref), rms)) <= 1e-2
    assert np.mean(np.abs(got - ref)) <= 1e-3


def test_golden_nvfp4_layouts(L):
    g, c = GOLD["nvfp4"], GOLD["nvfp4_coded"]
    v = arr(g["values"], np.uint8, (16, 64))
    s = arr(g["scales"], np.uint8, (16, 8))
    assert L.retile_nvfp4(dev(v), dev(s)).cpu().numpy().tobytes() == bytes.fromhex(g["tiled"])
    ok, table, code_of = L.scale_code_table(s)
    assert ok == c["ok"] and table.tobytes() == bytes.fromhex(c["table"])
    blob, raw = L.retile_nvfp4_coded(dev(v), dev(s), dev(code_of))
    assert blob.cpu().numpy().tobytes() == bytes.fromhex(c["blob"])
    assert raw.cpu().numpy().tobytes() == bytes.fromhex(c["raw"])


def test_golden_block_prefill(L):
    g = GOLD["prefill"]
    x = arr(g["x_bf16"], np.uint16, (4, 256))
    xq, xs = L.quant_act_fp8_g128(dev(x.view(np.int16)).view(torch.bfloat16))
    assert xq.cpu().numpy().tobytes() == bytes.fromhex(g["xq"])
    assert xs.cpu().numpy().tobytes() == bytes.fromhex(g["xs"])
    wq = arr(g["wq"], np.uint8, (128, 256))
    ws = arr(g["ws"], np.float32, (1, 2))
    y = L.prefill_fp8_block(xq, xs, L.retile_fp8(dev(wq)), dev(ws), 128)
    got = bf16_to_f32(y.view(torch.int16).cpu().numpy().view(np.uint16)).astype(np.float64)
    ref = arr(g["y_f32"], np.float32, (4, 128)).astype(np.float64)
    rms = np.sqrt(np.mean(ref ** 2, axis=1, keepdims=True))
    assert np.max(np.abs(got - ref) / np.maximum(np.abs(ref), rms)) <= 1e-2


def test_golden_activation_producers(L):
    g = GOLD["act_nvfp4"]
    x = arr(g["x"], np.float32, (2, 64))
    u = arr(g["u"], np.float32, (2, 64))
    q, sf = L.quant_act_nvfp4(dev(x), g["input_scale"])
    assert q.cpu().numpy().tobytes() == bytes.fromhex(g["q"]) and sf.cpu().numpy().tobytes() == bytes.fromhex(g["sf"])
    # silu: the device exp may round differently in the last bit from libm's expf (at most one code of 128 here)
    qs, sfs = L.silu_mul_quant_nvfp4(dev(x), dev(u), g["input_scale"])
    assert np.sum(qs.cpu().numpy() != arr(g["silu_q"], np.uint8, (2, 32))) <= 1
    assert np.sum(sfs.cpu().numpy() != arr(g["silu_sf"], np.uint8, (2, 4))) <= 1
    r = GOLD["rmsnorm_quant"]
    xr = arr(r["x"], np.float32, (2, 1024))
    wr = arr(r["w_bf16"], np.uint16)
    out, q8, _ = L.rmsnorm_quant(dev(xr), dev(wr.view(np.int16)), r["eps"], False, r["fp8_input_scale"])
    ref = arr(r["out"], np.float32, (2, 1024))
    assert np.max(np.abs(out.cpu().numpy() - ref)) <= 4e-6 * np.max(np.abs(ref))  # FP32 rounding of the norm
    # FP8 codes: equal wherever the device's FP32 norm value is the fixture's (a 1-ulp difference may move a code)
    same = out.cpu().numpy() == ref
    assert np.array_equal(q8.cpu().numpy()[same], arr(r["fp8_q"], np.uint8, (2, 1024))[same])
    _, q4, sf4 = L.rmsnorm_quant(dev(xr), dev(wr.view(np.int16)), r["eps"], True, r["nvfp4_input_scale"])
    assert np.mean(q4.cpu().numpy() != arr(r["nvfp4_q"], np.uint8, (2, 512))) <= 1e-2
    assert np.mean(sf4.cpu().numpy() != arr(r["nvfp4_sf"], np.uint8, (2, 64))) <= 1e-2


def test_golden_nvfp4_prefill(L):
    g, w = GOLD["prefill_nvfp4"], GOLD["nvfp4"]
    xq = arr(g["xq"], np.uint8, (2, 64))
    xs = arr(g["xs"], np.uint8, (2, 8))
    v = arr(w["values"], np.uint8, (16, 64))
    s = arr(w["scales"], np.uint8, (16, 8))
    # the prefill GEMM takes N % 128: the 16 golden rows padded with zero rows
    vp = np.zeros((128, 64), np.uint8)
    sp = np.zeros((128, 8), np.uint8)
    vp[:16], sp[:16] = v, s
    y = L.prefill_gemm_nvfp4(dev(xq), dev(xs), L.retile_nvfp4(dev(vp), dev(sp)), g["alpha"], 128)
    got = y.cpu().numpy()[:, :16].astype(np.float64)
    ref = arr(g["y_f64"], np.float64, (2, 16))
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))
    assert not y.cpu().numpy()[:, 16:].any()
