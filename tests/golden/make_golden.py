"""Writes tests/golden/vectors.json: small fixed input/output vectors of the CPU oracle.

They pin the oracle against drift between rounds (tests/test_golden.py recomputes them); the reference-held
known answers (tests/stream_tests.cu:1093-1119 hand-made NVFP4 block, E4M3 0x7e = 448 and 0x01 = 2^-9) are
included literally. Regenerate only when the oracle's arithmetic is meant to change:
    python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle as O  # noqa: E402


def hexa(a: np.ndarray) -> str:
    return np.ascontiguousarray(a).tobytes().hex()


def build() -> dict:
    v = {}
    v["rng_normal_f32_seed_4C510000"] = hexa(O.normal_f32(0x4C510000, 1.0, 16))
    pts = np.array([0.0, -0.0, 1e-4, 0.0019531, 0.015625, 0.1, 1.0, 1.0625, 1.1875, 3.7, 100.0, 447.0, 448.0, 500.0,
                    -2.5, -460.0], np.float32)
    v["e4m3_encode_in"] = hexa(pts)
    v["e4m3_encode_out"] = hexa(np.array([O.lib.or_e4m3_encode(float(p)) for p in pts], np.uint8))
    v["reference_nvfp4_block"] = {
        "row": [2688, 112, 336, 560, 784, 1120, 1568, 2240, 113, -336, -10, 0, -2688, 338, -1568, 448] + [0] * 16,
        "codes": [7, 0, 1, 2, 3, 4, 5, 6, 1, 9, 0, 0, 15, 2, 13, 2],
        "scales": [0x7E, 0x01],
        "scale2": 1.0,
    }
    # FP8 per-channel stream GEMM, M=3, N=16, K=256
    w = O.normal_f32(0x4C51F001, 0.02, (16, 256))
    q, s = O.quant_fp8_per_channel(w)
    x = O.normal_bf16(0x4C51F002, 1.0, (3, 256))
    v["stream_fp8_pc"] = {"x_bf16": hexa(x), "q": hexa(q), "s": hexa(s), "y_bf16": hexa(O.stream_fp8_pc_bf16(x, q, s)),
                          "tiled": hexa(O.retile_fp8(q))}
    # NVFP4 quantizer + tiled blob, N=16, K=128
    wb = O.normal_bf16(0x4C51F003, 0.02, (16, 128))
    vals, sc, g, err = O.quant_nvfp4(wb)
    v["nvfp4"] = {"w_bf16": hexa(wb), "values": hexa(vals), "scales": hexa(sc), "scale2": float(g),
                  "tiled": hexa(O.retile_nvfp4(vals, sc))}
    # block-scaled prefill, M=4, N=128, K=256
    wp = O.normal_f32(0x4C51F004, 0.02, (128, 256))
    wq, ws = O.quant_fp8_block128(wp)
    xp = O.normal_bf16(0x4C51F005, 1.0, (4, 256))
    xq, xs = O.quant_act_fp8_g128(xp)
    y = O.prefill_fp8_rows(xq, xs, np.arange(4), wq, ws)
    v["prefill"] = {"x_bf16": hexa(xp), "w_f32_seed": 0x4C51F004, "xq": hexa(xq), "xs": hexa(xs), "wq": hexa(wq),
                    "ws": hexa(ws), "y_f32": hexa(y)}
    # coded NVFP4 blob (6-bit scale codes) of the same weights
    ok, table, code_of = O.scale_code_table(sc)
    blob, raw = O.retile_nvfp4_coded(vals, sc, code_of)
    v["nvfp4_coded"] = {"ok": ok, "table": hexa(table), "blob": hexa(blob), "raw": hexa(raw)}
    # activation producers: NVFP4 quantizer, silu(g)*u into NVFP4, Gemma RMSNorm into FP8 and NVFP4
    xa = O.normal_f32(0x4C51F006, 1.0, (2, 64))
    xu = O.normal_f32(0x4C51F007, 1.0, (2, 64))
    qa, sfa = O.quant_act_nvfp4(xa, 0.0125)
    qs, sfs = O.silu_mul_quant_nvfp4(xa, xu, 0.0125)
    v["act_nvfp4"] = {"x": hexa(xa), "u": hexa(xu), "input_scale": 0.0125, "q": hexa(qa), "sf": hexa(sfa),
                      "silu_q": hexa(qs), "silu_sf": hexa(sfs)}
    xr = O.normal_f32(0x4C51F008, 1.0, (2, 1024))
    wr = O.normal_bf16(0x4C51F009, 0.1, 1024)
    o8, q8, _ = O.rmsnorm_quant(xr, wr, 1e-6, False, 0.02)
    o4, q4, sf4 = O.rmsnorm_quant(xr, wr, 1e-6, True, 0.005)
    v["rmsnorm_quant"] = {"x": hexa(xr), "w_bf16": hexa(wr), "eps": 1e-6, "out": hexa(o8), "fp8_input_scale": 0.02,
                          "fp8_q": hexa(q8), "nvfp4_input_scale": 0.005, "nvfp4_q": hexa(q4), "nvfp4_sf": hexa(sf4)}
    assert np.array_equal(o4, o8)
    # NVFP4 prefill rows (float64 over exactly dequantized operands), M=2, N=16, K=128
    qx, sfx = O.quant_act_nvfp4(O.normal_f32(0x4C51F00A, 1.0, (2, 128)), 0.0125)
    v["prefill_nvfp4"] = {"xq": hexa(qx), "xs": hexa(sfx), "alpha": 0.0125 * float(g),
                          "y_f64": hexa(O.prefill_nvfp4_rows(qx, sfx, np.arange(2), vals, sc, 0.0125 * float(g)))}
    return v


if __name__ == "__main__":
    with open(os.path.join(HERE, "vectors.json"), "w") as f:
        json.dump(build(), f, indent=1)
    print("wrote", os.path.join(HERE, "vectors.json"))
