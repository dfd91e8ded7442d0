"""ctypes view of the CPU oracle (liboracle.so): TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, as the checker or
as the timed CPU baseline. The product path (ling-engine_amd/) never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")


def build() -> None:
    subprocess.run(["make", "-s", "-B", "-C", _HERE, "liboracle.so"], check=True)


def _load():
    if not os.path.exists(_LIB_PATH):
        build()
    lib = C.CDLL(_LIB_PATH)
    P = C.c_void_p
    i, f, sz, u64 = C.c_int, C.c_float, C.c_size_t, C.c_uint64
    sig = {
        "or_fill_normal": (None, [u64, f, P, sz]),
        "or_fill_normal_bf16": (None, [u64, f, P, sz]),
        "or_e4m3_decode": (f, [C.c_uint8]),
        "or_e4m3_encode": (C.c_uint8, [f]),
        "or_e2m1_decode": (f, [C.c_uint8]),
        "or_e2m1_encode_weight": (C.c_uint8, [f]),
        "or_e2m1_encode_rne": (C.c_uint8, [f]),
        "or_bf16_bits": (C.c_uint16, [f]),
        "or_bf16_float": (f, [C.c_uint16]),
        "or_f16_bits": (C.c_uint16, [f]),
        "or_f16_float": (f, [C.c_uint16]),
        "or_quant_fp8_per_channel": (None, [P, i, i, P, P]),
        "or_quant_nvfp4": (f, [P, i, i, P, P, P]),
        "or_quant_fp8_block128": (None, [P, i, i, P, P]),
        "or_quant_act_fp8_g128": (None, [P, i, i, P, P]),
        "or_tiled_bytes_fp8": (sz, [i, i]),
        "or_tiled_bytes_nvfp4": (sz, [i, i]),
        "or_tiled_bytes_nvfp4_coded": (sz, [i, i]),
        "or_retile_fp8": (None, [P, P, i, i]),
        "or_untile_fp8": (None, [P, P, i, i]),
        "or_retile_nvfp4": (None, [P, P, P, i, i]),
        "or_untile_nvfp4": (None, [P, P, P, i, i]),
        "or_scale_code_table": (i, [P, sz, P, P]),
        "or_retile_nvfp4_coded": (None, [P, P, P, P, P, i, i]),
        "or_dequant_fp8_pc": (None, [P, P, i, i, P]),
        "or_dequant_nvfp4": (None, [P, P, f, i, i, P]),
        "or_dequant_fp8_block128": (None, [P, P, i, i, P]),
        "or_to_half_rows": (None, [P, i, i, P, P]),
        "or_gemm_f32": (None, [P, P, i, i, i, P, i]),
        "or_silu": (f, [f]),
        "or_epi_bf16": (None, [P, sz, P]),
        "or_epi_silu_mul_bf16": (None, [P, P, sz, P]),
        "or_epi_residual_bf16": (None, [P, P, sz, P]),
        "or_stream_fp8_pc_bf16": (None, [P, i, P, P, i, i, i, i, P, i]),
        "or_prefill_fp8_rows": (None, [P, P, P, i, P, P, i, i, P, i]),
        "or_rmsnorm_half": (None, [P, P, i, i, f, i, P, P, P]),
        "or_quant_act_fp8": (None, [P, sz, f, P]),
        "or_quant_act_nvfp4": (None, [P, i, i, f, P, P]),
        "or_silu_mul_quant_nvfp4": (None, [P, P, i, i, f, P, P]),
        "or_rmsnorm_quant": (None, [P, P, P, i, i, f, i, f, P, P]),
        "or_gated_rmsnorm_fp8": (None, [P, P, P, i, f, f, P]),
        "or_sigmoid_mul_fp8": (None, [P, P, sz, f, P]),
        "or_hardware_threads": (i, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.c_void_p)


# ---- generators (seeded, portable) ----
def normal_f32(seed: int, sigma: float, shape) -> np.ndarray:
    out = np.empty(shape, np.float32)
    lib.or_fill_normal(seed, sigma, _p(out), out.size)
    return out


def normal_bf16(seed: int, sigma: float, shape) -> np.ndarray:
    out = np.empty(shape, np.uint16)
    lib.or_fill_normal_bf16(seed, sigma, _p(out), out.size)
    return out


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    flat, o = x.reshape(-1), out.reshape(-1)
    lib.or_epi_bf16(_p(flat), flat.size, _p(o))
    return out


# ---- quantizers ----
def quant_fp8_per_channel(w: np.ndarray):
    N, K = w.shape
    q = np.empty((N, K), np.uint8)
    s = np.empty(N, np.float32)
    lib.or_quant_fp8_per_channel(_p(np.ascontiguousarray(w, np.float32)), N, K, _p(q), _p(s))
    return q, s


def quant_nvfp4(w_bf16: np.ndarray):
    N, K = w_bf16.shape
    v = np.empty((N, K // 2), np.uint8)
    s = np.empty((N, K // 16), np.uint8)
    err = C.c_double(0.0)
    g = lib.or_quant_nvfp4(_p(np.ascontiguousarray(w_bf16, np.uint16)), N, K, _p(v), _p(s), C.byref(err))
    return v, s, float(g), float(err.value)


def quant_fp8_block128(w: np.ndarray):
    N, K = w.shape
    q = np.empty((N, K), np.uint8)
    s = np.empty((N // 128, K // 128), np.float32)
    lib.or_quant_fp8_block128(_p(np.ascontiguousarray(w, np.float32)), N, K, _p(q), _p(s))
    return q, s


def quant_act_fp8_g128(x_bf16: np.ndarray):
    M, K = x_bf16.shape
    q = np.empty((M, K), np.uint8)
    s = np.empty((M, K // 128), np.float32)
    lib.or_quant_act_fp8_g128(_p(np.ascontiguousarray(x_bf16, np.uint16)), M, K, _p(q), _p(s))
    return q, s


# ---- layout ----
def retile_fp8(q: np.ndarray) -> np.ndarray:
    N, K = q.shape
    out = np.empty(lib.or_tiled_bytes_fp8(N, K), np.uint8)
    lib.or_retile_fp8(_p(np.ascontiguousarray(q)), _p(out), N, K)
    return out


def untile_fp8(t: np.ndarray, N: int, K: int) -> np.ndarray:
    out = np.empty((N, K), np.uint8)
    lib.or_untile_fp8(_p(t), _p(out), N, K)
    return out


def retile_nvfp4(v: np.ndarray, s: np.ndarray) -> np.ndarray:
    N = v.shape[0]
    K = v.shape[1] * 2
    out = np.empty(lib.or_tiled_bytes_nvfp4(N, K), np.uint8)
    lib.or_retile_nvfp4(_p(np.ascontiguousarray(v)), _p(np.ascontiguousarray(s)), _p(out), N, K)
    return out


def untile_nvfp4(t: np.ndarray, N: int, K: int):
    v = np.empty((N, K // 2), np.uint8)
    s = np.empty((N, K // 16), np.uint8)
    lib.or_untile_nvfp4(_p(t), _p(v), _p(s), N, K)
    return v, s


def scale_code_table(s: np.ndarray):
    table = np.zeros(64, np.uint8)
    code_of = np.zeros(256, np.uint8)
    flat = np.ascontiguousarray(s).reshape(-1)
    ok = lib.or_scale_code_table(_p(flat), flat.size, _p(table), _p(code_of))
    return bool(ok), table, code_of


def retile_nvfp4_coded(v: np.ndarray, s: np.ndarray, code_of: np.ndarray):
    N = v.shape[0]
    K = v.shape[1] * 2
    out = np.empty(lib.or_tiled_bytes_nvfp4_coded(N, K), np.uint8)
    raw = np.empty(N * K // 16, np.uint8)
    lib.or_retile_nvfp4_coded(_p(np.ascontiguousarray(v)), _p(np.ascontiguousarray(s)), _p(code_of), _p(out),
                              _p(raw), N, K)
    return out, raw


# ---- dequant ----
def dequant_fp8_pc(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    N, K = q.shape
    out = np.empty((N, K), np.float32)
    lib.or_dequant_fp8_pc(_p(np.ascontiguousarray(q)), _p(np.ascontiguousarray(s, np.float32)), N, K, _p(out))
    return out


def dequant_nvfp4(v: np.ndarray, s: np.ndarray, g: float) -> np.ndarray:
    N = v.shape[0]
    K = v.shape[1] * 2
    out = np.empty((N, K), np.float32)
    lib.or_dequant_nvfp4(_p(np.ascontiguousarray(v)), _p(np.ascontiguousarray(s)), g, N, K, _p(out))
    return out


def dequant_fp8_block128(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    N, K = q.shape
    out = np.empty((N, K), np.float32)
    lib.or_dequant_fp8_block128(_p(np.ascontiguousarray(q)), _p(np.ascontiguousarray(s, np.float32)), N, K,
                                _p(out))
    return out


def to_half_rows(x: np.ndarray):
    M, K = x.shape
    xh = np.empty((M, K), np.uint16)
    xinv = np.empty(M, np.float32)
    lib.or_to_half_rows(_p(np.ascontiguousarray(x, np.float32)), M, K, _p(xh), _p(xinv))
    return xh, xinv


# ---- GEMM + epilogues ----
def gemm_f32(x: np.ndarray, wdeq: np.ndarray, threads: int = 0) -> np.ndarray:
    M, K = x.shape
    N = wdeq.shape[0]
    y = np.empty((M, N), np.float32)
    lib.or_gemm_f32(_p(np.ascontiguousarray(x, np.float32)), _p(np.ascontiguousarray(wdeq, np.float32)), M, N, K,
                    _p(y), threads)
    return y


def epi_silu_mul_bf16(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.empty(g.shape, np.uint16)
    lib.or_epi_silu_mul_bf16(_p(g), _p(u), g.size, _p(out))
    return out


def epi_residual_bf16(acc: np.ndarray, resid: np.ndarray) -> np.ndarray:
    acc = np.ascontiguousarray(acc, np.float32)
    resid = np.ascontiguousarray(resid, np.uint16)
    out = np.empty(acc.shape, np.uint16)
    lib.or_epi_residual_bf16(_p(acc), _p(resid), acc.size, _p(out))
    return out


def stream_fp8_pc_bf16(x_bf16: np.ndarray, q: np.ndarray, s: np.ndarray, n0: int = 0, n1: int | None = None,
                       threads: int = 0) -> np.ndarray:
    M, K = x_bf16.shape
    N = q.shape[0]
    n1 = N if n1 is None else n1
    y = np.zeros((M, N), np.uint16)
    lib.or_stream_fp8_pc_bf16(_p(np.ascontiguousarray(x_bf16)), M, _p(np.ascontiguousarray(q)),
                              _p(np.ascontiguousarray(s, np.float32)), N, K, n0, n1, _p(y), threads)
    return y


def prefill_fp8_rows(xq, xs, rows, wq, ws, threads: int = 0) -> np.ndarray:
    rows = np.ascontiguousarray(rows, np.int32)
    R = rows.size
    N, K = wq.shape
    y = np.empty((R, N), np.float32)
    lib.or_prefill_fp8_rows(_p(np.ascontiguousarray(xq)), _p(np.ascontiguousarray(xs, np.float32)), _p(rows), R,
                            _p(np.ascontiguousarray(wq)), _p(np.ascontiguousarray(ws, np.float32)), N, K, _p(y),
                            threads)
    return y


def rmsnorm_half(x: np.ndarray, w_bf16: np.ndarray, eps: float, gemma: bool = True):
    x = np.ascontiguousarray(x, np.float32)
    rows, H = x.shape
    out = np.empty_like(x)
    xh = np.empty((rows, H), np.uint16)
    xinv = np.empty(rows, np.float32)
    lib.or_rmsnorm_half(_p(x), _p(np.ascontiguousarray(w_bf16, np.uint16)), rows, H, eps, int(gemma),
                        _p(out), _p(xh), _p(xinv))
    return out, xh, xinv


def quant_act_fp8(x: np.ndarray, input_scale: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    q = np.empty(x.shape, np.uint8)
    lib.or_quant_act_fp8(_p(x), x.size, input_scale, _p(q))
    return q


def quant_act_nvfp4(x: np.ndarray, input_scale: float):
    """x FP32 [M][K] -> (q [M][K/2] packed E2M1, sf [M][K/16] E4M3) (reference prefill_gemm.cu:382-420)."""
    x = np.ascontiguousarray(x, np.float32)
    M, K = x.shape
    q = np.empty((M, K // 2), np.uint8)
    sf = np.empty((M, K // 16), np.uint8)
    lib.or_quant_act_nvfp4(_p(x), M, K, input_scale, _p(q), _p(sf))
    return q, sf


def silu_mul_quant_nvfp4(g: np.ndarray, u: np.ndarray, input_scale: float):
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    M, K = g.shape
    q = np.empty((M, K // 2), np.uint8)
    sf = np.empty((M, K // 16), np.uint8)
    lib.or_silu_mul_quant_nvfp4(_p(g), _p(u), M, K, input_scale, _p(q), _p(sf))
    return q, sf


def rmsnorm_quant(x: np.ndarray, w_bf16: np.ndarray, eps: float, nvfp4: bool, input_scale: float):
    """-> (out FP32 [M][H], q, sf or None) (reference prefill_gemm.cu:426-459)."""
    x = np.ascontiguousarray(x, np.float32)
    M, H = x.shape
    out = np.empty((M, H), np.float32)
    q = np.empty((M, H // 2) if nvfp4 else (M, H), np.uint8)
    sf = np.empty((M, H // 16), np.uint8) if nvfp4 else None
    lib.or_rmsnorm_quant(_p(x), _p(np.ascontiguousarray(w_bf16, np.uint16)), _p(out), M, H, eps, int(nvfp4),
                         input_scale, _p(q), _p(sf) if sf is not None else None)
    return out, q, sf


def gated_rmsnorm_fp8(x: np.ndarray, z: np.ndarray, w_bf16: np.ndarray, eps: float, input_scale: float):
    """DeltaNet output norm into FP8 (reference prefill_gemm.cu:461-482): x, z FP32 [rows][128] (BF16 inputs are
    widened by the caller, exactly), w BF16 bits [128] -> q uint8 [rows][128]."""
    x = np.ascontiguousarray(x, np.float32)
    z = np.ascontiguousarray(z, np.float32)
    rows, D = x.shape
    assert D == 128 and z.shape == x.shape
    q = np.empty((rows, D), np.uint8)
    lib.or_gated_rmsnorm_fp8(_p(x), _p(z), _p(np.ascontiguousarray(w_bf16, np.uint16)), rows, eps, input_scale, _p(q))
    return q


def sigmoid_mul_fp8(x: np.ndarray, gate: np.ndarray, input_scale: float):
    """x * sigmoid(gate) into FP8 (reference prefill_gemm.cu:484-494), elementwise."""
    x = np.ascontiguousarray(x, np.float32)
    gate = np.ascontiguousarray(gate, np.float32)
    q = np.empty(x.shape, np.uint8)
    lib.or_sigmoid_mul_fp8(_p(x), _p(gate), x.size, input_scale, _p(q))
    return q


def fp8_code_band(v64: np.ndarray, input_scale: float, rel: float):
    """The FP8 codes E4M3_sat(bf16(v) * (1 / input_scale)) can take for every FP32 v within a relative `rel` of
    the float64 value v64: (lo, hi) codes of the band's ends. BF16 rounding is monotone, so where lo == hi the code
    is fixed, and elsewhere (a BF16 rounding boundary inside the band) it is one of the two."""
    v64 = np.asarray(v64, np.float64)
    a = quant_act_fp8((v64 * (1.0 - rel)).astype(np.float32), input_scale)
    b = quant_act_fp8((v64 * (1.0 + rel)).astype(np.float32), input_scale)
    return a, b


def prefill_nvfp4_rows(xq, xs, rows, wv, ws, alpha: float) -> np.ndarray:
    """The NVFP4 prefill GEMM (reference prefill_gemm.cu:344-376, 593-603; y = alpha * xq . W^T over the exactly
    dequantized operands, E2M1 x E4M3 per 16-value block) for the token rows `rows`, in float64."""
    xd = dequant_nvfp4(np.ascontiguousarray(xq[rows]), np.ascontiguousarray(xs[rows]), 1.0).astype(np.float64)
    wd = dequant_nvfp4(wv, ws, 1.0).astype(np.float64)
    return alpha * (xd @ wd.T)


def hardware_threads() -> int:
    return lib.or_hardware_threads()
