"""Python binding of libling_gemm.so (the C ABI in include/ling_gemm.h) over torch device tensors.

torch provides device memory and the stream (plumbing); every computation runs in the library's HIP
kernels. The module fails loudly when the library is missing: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libling_gemm.so")

MAX_STREAM_ROWS = 80

# exported symbols and signatures (argument order of include/ling_gemm.h)
_P, _I, _F, _SZ = C.c_void_p, C.c_int, C.c_float, C.c_size_t
SIGNATURES = {
    "lq_last_error": (C.c_char_p, []),
    "lq_init": (_I, []),
    "lq_version": (C.c_char_p, []),
    "lq_stream_workspace_bytes": (_SZ, [_I]),
    "lq_set_workspace": (_I, [_P, _SZ]),
    "lq_tiled_bytes_fp8": (_SZ, [_I, _I]),
    "lq_tiled_bytes_nvfp4": (_SZ, [_I, _I]),
    "lq_tiled_bytes_nvfp4_coded": (_SZ, [_I, _I]),
    "lq_retile_fp8": (_I, [_P, _P, _I, _I, _P]),
    "lq_retile_nvfp4": (_I, [_P, _P, _P, _I, _I, _P]),
    "lq_scale_code_table": (_I, [_P, _SZ, _P, _P]),
    "lq_retile_nvfp4_coded": (_I, [_P, _P, _P, _P, _P, _I, _I, _P]),
    "lq_dequant_tiled_fp8": (_I, [_P, _F, _P, _I, _I, _P]),
    "lq_dequant_tiled_nvfp4": (_I, [_P, _F, _P, _I, _I, _P, _P]),
    "lq_dequant_tiled_fp8_pc_f32": (_I, [_P, _P, _P, _I, _I, _P]),
    "lq_dequant_tiled_nvfp4_f32": (_I, [_P, _F, _P, _I, _I, _P, _P]),
    "lq_to_half_rows": (_I, [_P, _I, _I, _P, _P, _P]),
    "lq_bf16_to_half_rows": (_I, [_P, _I, _I, _P, _P, _P]),
    "lq_stream_gemm_fp8": (_I, [_P, _P, _I, _P, _F, _P, _I, _I, _P]),
    "lq_stream_gemm_nvfp4": (_I, [_P, _P, _I, _P, _P, _F, _P, _I, _I, _P]),
    "lq_stream_gemm_multi": (_I, [_I, _P, _P, _I, _P, _I, _I, _P]),
    "lq_stream_gemm_gather_nvfp4": (_I, [_P, _P, _I, _P, _P, _F, _P, _P, _I, _P, _I, _I, _P]),
    "lq_l2_prefetch_weights": (_I, [_P, _I, _I, _I, _I, _SZ, _P]),
    "lq_stream_fp8_pc": (_I, [_P, _I, _P, _P, _P, _I, _I, _P]),
    "lq_stream_fp8_pc_noalloc": (_I, [_P, _I, _P, _P, _P, _I, _I, _P]),
    "lq_stream_fp8_pc_silu_mul": (_I, [_P, _I, _P, _P, _P, _P, _P, _I, _I, _P]),
    "lq_stream_fp8_pc_residual": (_I, [_P, _I, _P, _P, _P, _P, _I, _I, _P]),
    "lq_stream_fp8_pc_ffn": (_I, [_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _P]),
    "lq_stream_ffn_deadline_status": (_I, [_P]),
    "lq_stream_nvfp4_bf16": (_I, [_P, _I, _P, _P, _F, _P, _I, _I, _P]),
    "lq_quant_act_fp8_g128": (_I, [_P, _I, _I, _P, _P, _P]),
    "lq_prefill_gemm_nvfp4": (_I, [_P, _P, _I, _P, _F, _P, _I, _I, _I, _I, _P, _P]),
    "lq_prefill_swiglu_nvfp4": (_I, [_P, _P, _I, _P, _F, _P, _F, _I, _I, _F, _P, _P, _P, _P, _P]),
    "lq_quant_act_nvfp4": (_I, [_P, _I, _I, _F, _P, _P, _P]),
    "lq_silu_mul_quant_nvfp4": (_I, [_P, _P, _I, _I, _F, _P, _P, _P]),
    "lq_rmsnorm_quant": (_I, [_P, _P, _P, _I, _I, _F, _I, _F, _P, _P, _P]),
    "lq_prefill_fp8_block": (_I, [_P, _P, _I, _P, _P, _P, _I, _I, _I, _P]),
    "lq_rmsnorm_half": (_I, [_P, _P, _P, _P, _P, _I, _I, _F, _I, _P]),
    "lq_quant_act_fp8": (_I, [_P, _I, _I, _F, _P, _P]),
    "lq_quant_act_fp8_bf16in": (_I, [_P, _I, _I, _F, _P, _P]),
    "lq_rmsnorm_quant_bf16": (_I, [_P, _P, _P, _I, _I, _F, _I, _F, _P, _P, _P]),
    "lq_gated_rmsnorm_fp8": (_I, [_P, _P, _P, _I, _I, _F, _F, _P, _P]),
    "lq_gated_rmsnorm_fp8_bf16": (_I, [_P, _P, _P, _I, _I, _F, _F, _P, _P]),
    "lq_sigmoid_mul_fp8": (_I, [_P, _P, _SZ, _F, _P, _P]),
    "lq_prefill_gemm_fp8": (_I, [_P, _I, _P, _F, _P, _I, _I, _I, _I, _P]),
    "lq_prefill_gemm_fp8_bf16out": (_I, [_P, _I, _P, _F, _P, _I, _I, _I, _P]),
    "lq_wfile_compile": (_I, [C.c_char_p, C.c_char_p, _I, _P]),
    "lq_wfile_open": (_I, [C.c_char_p, _P]),
    "lq_wfile_close": (None, [_P]),
    "lq_wfile_count": (_I, [_P]),
    "lq_wfile_find": (_I, [_P, C.c_char_p]),
    "lq_wfile_entry": (_I, [_P, _I, _P]),
    "lq_wfile_verify": (_I, [_P, _I]),
    "lq_host_retile_fp8": (_I, [_P, _P, _I, _I]),
    "lq_host_retile_nvfp4": (_I, [_P, _P, _P, _I, _I]),
    "lq_host_retile_nvfp4_coded": (_I, [_P, _P, _P, _P, _P, _I, _I]),
    "lq_quantize_nvfp4": (_I, [_P, _I, _I, _P, _P, _P, _P]),
    "lq_quantize_fp8_channel": (_I, [_P, _I, _I, _I, _P, _P]),
    "lq_quantize_fp8_block128": (_I, [_P, _I, _I, _I, _P, _P]),
}

# include/ling_gemm.h lq_wentry / lq_wfile flags and kinds
WFILE_NO_CODES, WFILE_PASSTHROUGH = 1, 2
WFILE_QUANT_FP8, WFILE_QUANT_FP8_BLOCK, WFILE_QUANT_NVFP4 = 4, 8, 16
WENTRY_QUANTIZED = 2
DT_F32, DT_BF16, DT_F16 = 0, 1, 2
WENTRY_FP8, WENTRY_NVFP4, WENTRY_NVFP4_CODED, WENTRY_RAW = 1, 2, 3, 4
WSCALE_NONE, WSCALE_TENSOR, WSCALE_CHANNEL, WSCALE_BLOCK128 = 0, 1, 2, 3
WENTRY_HAS_INPUT_SCALE = 1


class WEntry(C.Structure):
    _fields_ = [("name", C.c_char_p), ("kind", C.c_int), ("scale_kind", C.c_int), ("N", C.c_int), ("K", C.c_int),
                ("weight_scale", C.c_float), ("input_scale", C.c_float), ("flags", C.c_int),
                ("dtype", C.c_char * 16), ("ndim", C.c_int), ("shape", C.c_int64 * 4),
                ("blob", C.c_void_p), ("blob_bytes", C.c_size_t), ("aux", C.c_void_p), ("aux_bytes", C.c_size_t),
                ("table", C.c_void_p), ("table_bytes", C.c_size_t)]


class StreamTarget(C.Structure):
    _fields_ = [("w", C.c_void_p), ("wscale", C.c_void_p), ("scale", C.c_float), ("y", C.c_void_p), ("N", C.c_int)]


class LingGemmError(RuntimeError):
    pass


def load_library(path: str = LIB_PATH) -> C.CDLL:
    if not os.path.exists(path):
        raise ImportError(f"{path} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                          "(or make -C ling-engine_amd/csrc)")
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = load_library()


def _ptr(t):
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return C.c_void_p(t.data_ptr())


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _check(rc: int) -> None:
    if rc != 0:
        raise LingGemmError(lib.lq_last_error().decode())


def _dev(t: torch.Tensor, dtype=None) -> torch.Tensor:
    if not t.is_cuda:
        raise ValueError("expected a device tensor")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"expected {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError("expected a contiguous tensor")
    return t


def init() -> None:
    _check(lib.lq_init())


def stream_workspace_bytes(max_rows: int = MAX_STREAM_ROWS) -> int:
    return lib.lq_stream_workspace_bytes(max_rows)


def set_workspace(buf) -> None:
    """buf: a uint8 device tensor that stays alive while set (None: back to the library's own workspace)."""
    if buf is None:
        _check(lib.lq_set_workspace(None, 0))
    else:
        _check(lib.lq_set_workspace(_ptr(_dev(buf, torch.uint8)), buf.numel()))


# ---------------- layout ----------------
def tiled_bytes_fp8(N: int, K: int) -> int:
    return lib.lq_tiled_bytes_fp8(N, K)


def tiled_bytes_nvfp4(N: int, K: int) -> int:
    return lib.lq_tiled_bytes_nvfp4(N, K)


def tiled_bytes_nvfp4_coded(N: int, K: int) -> int:
    return lib.lq_tiled_bytes_nvfp4_coded(N, K)


def retile_fp8(w: torch.Tensor) -> torch.Tensor:
    """Row-major FP8 codes [N][K] (uint8) -> the tiled blob (uint8)."""
    N, K = w.shape
    out = torch.empty(tiled_bytes_fp8(N, K), dtype=torch.uint8, device=w.device)
    _check(lib.lq_retile_fp8(_ptr(_dev(w, torch.uint8)), _ptr(out), N, K, _stream()))
    return out


def retile_nvfp4(values: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    N = values.shape[0]
    K = values.shape[1] * 2
    out = torch.empty(tiled_bytes_nvfp4(N, K), dtype=torch.uint8, device=values.device)
    _check(lib.lq_retile_nvfp4(_ptr(_dev(values, torch.uint8)), _ptr(_dev(scales, torch.uint8)), _ptr(out), N, K,
                               _stream()))
    return out


def scale_code_table(scales_host) -> tuple[bool, bytes, bytes]:
    import numpy as np
    s = np.ascontiguousarray(scales_host, dtype=np.uint8).reshape(-1)
    table = np.zeros(64, np.uint8)
    code_of = np.zeros(256, np.uint8)
    ok = lib.lq_scale_code_table(s.ctypes.data_as(C.c_void_p), s.size, table.ctypes.data_as(C.c_void_p),
                                 code_of.ctypes.data_as(C.c_void_p))
    return bool(ok), table, code_of


def _np_ptr(a):
    return a.ctypes.data_as(C.c_void_p)


def host_retile_fp8(w_host):
    """Row-major FP8 codes [N][K] (numpy uint8) -> the tiled blob, on CPU threads (bytes of retile_fp8)."""
    import numpy as np
    w = np.ascontiguousarray(w_host, dtype=np.uint8)
    N, K = w.shape
    out = np.empty(tiled_bytes_fp8(N, K), np.uint8)
    _check(lib.lq_host_retile_fp8(_np_ptr(w), _np_ptr(out), N, K))
    return out


def host_retile_nvfp4(values_host, scales_host):
    import numpy as np
    v = np.ascontiguousarray(values_host, dtype=np.uint8)
    sc = np.ascontiguousarray(scales_host, dtype=np.uint8)
    N, K = v.shape[0], v.shape[1] * 2
    out = np.empty(tiled_bytes_nvfp4(N, K), np.uint8)
    _check(lib.lq_host_retile_nvfp4(_np_ptr(v), _np_ptr(sc), _np_ptr(out), N, K))
    return out


def host_retile_nvfp4_coded(values_host, scales_host, code_of):
    """-> (coded blob, raw scale copy), the bytes of retile_nvfp4_coded."""
    import numpy as np
    v = np.ascontiguousarray(values_host, dtype=np.uint8)
    sc = np.ascontiguousarray(scales_host, dtype=np.uint8)
    cm = np.ascontiguousarray(code_of, dtype=np.uint8)
    N, K = v.shape[0], v.shape[1] * 2
    out = np.empty(tiled_bytes_nvfp4_coded(N, K), np.uint8)
    raw = np.empty(N * K // 16, np.uint8)
    _check(lib.lq_host_retile_nvfp4_coded(_np_ptr(v), _np_ptr(sc), _np_ptr(cm), _np_ptr(out), _np_ptr(raw), N, K))
    return out, raw


def retile_nvfp4_coded(values: torch.Tensor, scales: torch.Tensor, code_of: torch.Tensor):
    N = values.shape[0]
    K = values.shape[1] * 2
    out = torch.empty(tiled_bytes_nvfp4_coded(N, K), dtype=torch.uint8, device=values.device)
    raw = torch.empty(N * K // 16, dtype=torch.uint8, device=values.device)
    _check(lib.lq_retile_nvfp4_coded(_ptr(_dev(values, torch.uint8)), _ptr(_dev(scales, torch.uint8)),
                                     _ptr(_dev(code_of, torch.uint8)), _ptr(out), _ptr(raw), N, K, _stream()))
    return out, raw


def dequant_tiled_fp8(tw: torch.Tensor, wscale: float, N: int, K: int) -> torch.Tensor:
    out = torch.empty((N, K), dtype=torch.bfloat16, device=tw.device)
    _check(lib.lq_dequant_tiled_fp8(_ptr(tw), wscale, _ptr(out), N, K, _stream()))
    return out


def dequant_tiled_fp8_pc_f32(tw: torch.Tensor, wscale_n: torch.Tensor, N: int, K: int) -> torch.Tensor:
    out = torch.empty((N, K), dtype=torch.float32, device=tw.device)
    _check(lib.lq_dequant_tiled_fp8_pc_f32(_ptr(tw), _ptr(_dev(wscale_n, torch.float32)), _ptr(out), N, K, _stream()))
    return out


def dequant_tiled_nvfp4(tw: torch.Tensor, scale2: float, N: int, K: int, raw_scales=None) -> torch.Tensor:
    out = torch.empty((N, K), dtype=torch.bfloat16, device=tw.device)
    _check(lib.lq_dequant_tiled_nvfp4(_ptr(tw), scale2, _ptr(out), N, K, _stream(), _ptr(raw_scales)))
    return out


def dequant_tiled_nvfp4_f32(tw: torch.Tensor, scale2: float, N: int, K: int, raw_scales=None) -> torch.Tensor:
    out = torch.empty((N, K), dtype=torch.float32, device=tw.device)
    _check(lib.lq_dequant_tiled_nvfp4_f32(_ptr(tw), scale2, _ptr(out), N, K, _stream(), _ptr(raw_scales)))
    return out


# ---------------- rows path, reference-compatible ----------------
def to_half_rows(x: torch.Tensor):
    M, K = x.shape
    xh = torch.empty((M, K), dtype=torch.float16, device=x.device)
    xinv = torch.empty(M, dtype=torch.float32, device=x.device)
    _check(lib.lq_to_half_rows(_ptr(_dev(x, torch.float32)), M, K, _ptr(xh), _ptr(xinv), _stream()))
    return xh, xinv


def bf16_to_half_rows(x: torch.Tensor):
    M, K = x.shape
    xh = torch.empty((M, K), dtype=torch.float16, device=x.device)
    xinv = torch.empty(M, dtype=torch.float32, device=x.device)
    _check(lib.lq_bf16_to_half_rows(_ptr(_dev(x, torch.bfloat16)), M, K, _ptr(xh), _ptr(xinv), _stream()))
    return xh, xinv


def rmsnorm_half(x, w, eps: float, gemma: bool = True):
    """x FP32 [rows][H], w BF16 [H] -> (out FP32, xh FP16, xinv FP32 [rows])."""
    rows, H = x.shape
    out = torch.empty_like(x, dtype=torch.float32)
    xh = torch.empty((rows, H), dtype=torch.float16, device=x.device)
    xinv = torch.empty(rows, dtype=torch.float32, device=x.device)
    _check(lib.lq_rmsnorm_half(_ptr(_dev(x, torch.float32)), _ptr(_dev(w, torch.bfloat16)), _ptr(out), _ptr(xh),
                               _ptr(xinv), rows, H, eps, int(gemma), _stream()))
    return out, xh, xinv


def stream_gemm_fp8(xh, xinv, w, wscale: float, N: int, K: int, y=None):
    M = xh.shape[0]
    y = torch.empty((M, N), dtype=torch.float32, device=xh.device) if y is None else y
    _check(lib.lq_stream_gemm_fp8(_ptr(_dev(xh, torch.float16)), _ptr(xinv), M, _ptr(w), wscale, _ptr(y), N, K,
                                  _stream()))
    return y


def stream_gemm_nvfp4(xh, xinv, w, table, scale2: float, N: int, K: int, y=None):
    M = xh.shape[0]
    y = torch.empty((M, N), dtype=torch.float32, device=xh.device) if y is None else y
    _check(lib.lq_stream_gemm_nvfp4(_ptr(_dev(xh, torch.float16)), _ptr(xinv), M, _ptr(w), _ptr(table), scale2,
                                    _ptr(y), N, K, _stream()))
    return y


def stream_gemm_gather_nvfp4(xh, xinv, w, raw_scales, scale2: float, rows, nrows, cap: int, N: int, K: int, y=None):
    """rows: int32 device [>= count]; nrows: int32 device [1]. Returns y [M][cap] FP32."""
    M = xh.shape[0]
    y = torch.empty((M, cap), dtype=torch.float32, device=xh.device) if y is None else y
    _check(lib.lq_stream_gemm_gather_nvfp4(_ptr(_dev(xh, torch.float16)), _ptr(xinv), M, _ptr(w), _ptr(raw_scales),
                                           scale2, _ptr(_dev(rows, torch.int32)), _ptr(_dev(nrows, torch.int32)), cap,
                                           _ptr(y), K, N, _stream()))
    return y


def l2_prefetch_weights(w, fp4: bool, coded: bool, N: int, K: int, nbytes: int):
    """Warms the caches with about nbytes of what a stream GEMM over (w, N, K) reads first; writes nothing."""
    _check(lib.lq_l2_prefetch_weights(_ptr(w), int(fp4), int(coded), N, K, int(nbytes),
                                      _stream()))


def stream_gemm_multi(nvfp4: bool, xh, xinv, targets, K: int):
    """targets: list of (w, table_or_None, scale, y, N)."""
    M = xh.shape[0]
    arr = (StreamTarget * len(targets))()
    for i, (w, tab, sc, y, N) in enumerate(targets):
        arr[i] = StreamTarget(w.data_ptr(), tab.data_ptr() if tab is not None else None, sc, y.data_ptr(), N)
    _check(lib.lq_stream_gemm_multi(int(nvfp4), _ptr(_dev(xh, torch.float16)), _ptr(xinv), M, arr, len(targets), K,
                                    _stream()))


# ---------------- rows path, BF16 formats ----------------
def stream_fp8_pc(x, w, wscale_n, N: int, y=None):
    M, K = x.shape
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device) if y is None else y
    _check(lib.lq_stream_fp8_pc(_ptr(_dev(x, torch.bfloat16)), M, _ptr(w), _ptr(_dev(wscale_n, torch.float32)),
                                _ptr(y), N, K, _stream()))
    return y


def stream_fp8_pc_noalloc(x, w, wscale_n, N: int, y=None):
    """stream_fp8_pc with the library's fixed scratch instead of its workspace (allocates nothing; y is the caller's)."""
    M, K = x.shape
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device) if y is None else y
    _check(lib.lq_stream_fp8_pc_noalloc(_ptr(_dev(x, torch.bfloat16)), M, _ptr(w), _ptr(wscale_n), _ptr(y), N, K,
                                        _stream()))
    return y


def stream_fp8_pc_silu_mul(x, w_gate, s_gate, w_up, s_up, N: int, h=None):
    M, K = x.shape
    h = torch.empty((M, N), dtype=torch.bfloat16, device=x.device) if h is None else h
    _check(lib.lq_stream_fp8_pc_silu_mul(_ptr(_dev(x, torch.bfloat16)), M, _ptr(w_gate), _ptr(s_gate), _ptr(w_up),
                                         _ptr(s_up), _ptr(h), N, K, _stream()))
    return h


def stream_fp8_pc_residual(x, w, wscale_n, resid, N: int, y=None):
    M, K = x.shape
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device) if y is None else y
    _check(lib.lq_stream_fp8_pc_residual(_ptr(_dev(x, torch.bfloat16)), M, _ptr(w), _ptr(wscale_n),
                                         _ptr(_dev(resid, torch.bfloat16)), _ptr(y), N, K, _stream()))
    return y


def stream_fp8_pc_ffn(x, w_gate, s_gate, w_up, s_up, w_down, s_down, resid, I: int, h=None, y=None):
    """One launch: h = silu(gate) * up (BF16 [M][I]), y = down(h) + resid (BF16 [M][H]); returns (h, y)."""
    M, H = x.shape
    h = torch.empty((M, I), dtype=torch.bfloat16, device=x.device) if h is None else h
    y = torch.empty((M, H), dtype=torch.bfloat16, device=x.device) if y is None else y
    _check(lib.lq_stream_fp8_pc_ffn(_ptr(_dev(x, torch.bfloat16)), M, _ptr(w_gate), _ptr(s_gate), _ptr(w_up),
                                    _ptr(s_up), _ptr(w_down), _ptr(s_down), _ptr(_dev(resid, torch.bfloat16)),
                                    _ptr(_dev(h, torch.bfloat16)), _ptr(_dev(y, torch.bfloat16)), I, H, _stream()))
    return h, y


def stream_ffn_deadline_status() -> int:
    hit = C.c_int(0)
    _check(lib.lq_stream_ffn_deadline_status(C.byref(hit)))
    return hit.value


def stream_nvfp4_bf16(x, w, table, scale2: float, N: int, y=None):
    M, K = x.shape
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device) if y is None else y
    _check(lib.lq_stream_nvfp4_bf16(_ptr(_dev(x, torch.bfloat16)), M, _ptr(w), _ptr(table), scale2, _ptr(y), N, K,
                                    _stream()))
    return y


# ---------------- prefill, NVFP4 ----------------
def prefill_gemm_nvfp4(xq, xs, w, alpha: float, N: int, y=None, ldy: int | None = None, accumulate: bool = False,
                       wsf=None):
    M, K2 = xq.shape
    K = K2 * 2
    ldy = N if ldy is None else ldy
    y = torch.empty((M, ldy), dtype=torch.float32, device=xq.device) if y is None else y
    _check(lib.lq_prefill_gemm_nvfp4(_ptr(_dev(xq, torch.uint8)), _ptr(_dev(xs, torch.uint8)), M, _ptr(w), alpha,
                                     _ptr(_dev(y, torch.float32)), ldy, N, K, int(accumulate), _stream(), _ptr(wsf)))
    return y


def prefill_swiglu_nvfp4(xq, xs, gate, alpha_gate: float, up, alpha_up: float, N: int, out_input_scale: float,
                         gate_sf=None, up_sf=None):
    M, K2 = xq.shape
    K = K2 * 2
    q = torch.empty((M, N // 2), dtype=torch.uint8, device=xq.device)
    sf = torch.empty((M, N // 16), dtype=torch.uint8, device=xq.device)
    _check(lib.lq_prefill_swiglu_nvfp4(_ptr(_dev(xq, torch.uint8)), _ptr(_dev(xs, torch.uint8)), M, _ptr(gate),
                                       alpha_gate, _ptr(up), alpha_up, N, K, out_input_scale, _ptr(q), _ptr(sf),
                                       _stream(), _ptr(gate_sf), _ptr(up_sf)))
    return q, sf


# ---------------- prefill activation producers ----------------
def quant_act_nvfp4(x, input_scale: float):
    M, K = x.shape
    q = torch.empty((M, K // 2), dtype=torch.uint8, device=x.device)
    sf = torch.empty((M, K // 16), dtype=torch.uint8, device=x.device)
    _check(lib.lq_quant_act_nvfp4(_ptr(_dev(x, torch.float32)), M, K, input_scale, _ptr(q), _ptr(sf), _stream()))
    return q, sf


def silu_mul_quant_nvfp4(g, u, input_scale: float):
    M, K = g.shape
    q = torch.empty((M, K // 2), dtype=torch.uint8, device=g.device)
    sf = torch.empty((M, K // 16), dtype=torch.uint8, device=g.device)
    _check(lib.lq_silu_mul_quant_nvfp4(_ptr(_dev(g, torch.float32)), _ptr(_dev(u, torch.float32)), M, K, input_scale,
                                       _ptr(q), _ptr(sf), _stream()))
    return q, sf


def rmsnorm_quant(x, w_bf16, eps: float, nvfp4: bool, input_scale: float, with_out: bool = True):
    """-> (out FP32 or None, q, sf or None)."""
    M, H = x.shape
    out = torch.empty((M, H), dtype=torch.float32, device=x.device) if with_out else None
    q = torch.empty((M, H // 2) if nvfp4 else (M, H), dtype=torch.uint8, device=x.device)
    sf = torch.empty((M, H // 16), dtype=torch.uint8, device=x.device) if nvfp4 else None
    _check(lib.lq_rmsnorm_quant(_ptr(_dev(x, torch.float32)), _ptr(_dev(w_bf16)), _ptr(out), M, H, eps, int(nvfp4),
                                input_scale, _ptr(q), _ptr(sf), _stream()))
    return out, q, sf


def rmsnorm_quant_bf16(x, w_bf16, eps: float, nvfp4: bool, input_scale: float, with_out: bool = True):
    """-> (out BF16 or None, q, sf or None)."""
    M, H = x.shape
    out = torch.empty((M, H), dtype=torch.bfloat16, device=x.device) if with_out else None
    q = torch.empty((M, H // 2) if nvfp4 else (M, H), dtype=torch.uint8, device=x.device)
    sf = torch.empty((M, H // 16), dtype=torch.uint8, device=x.device) if nvfp4 else None
    _check(lib.lq_rmsnorm_quant_bf16(_ptr(_dev(x, torch.float32)), _ptr(_dev(w_bf16)), _ptr(out), M, H, eps,
                                     int(nvfp4), input_scale, _ptr(q), _ptr(sf), _stream()))
    return out, q, sf


# ---------------- prefill ----------------
def quant_act_fp8_g128(x):
    M, K = x.shape
    q = torch.empty((M, K), dtype=torch.uint8, device=x.device)
    s = torch.empty((M, K // 128), dtype=torch.float32, device=x.device)
    _check(lib.lq_quant_act_fp8_g128(_ptr(_dev(x, torch.bfloat16)), M, K, _ptr(q), _ptr(s), _stream()))
    return q, s


def prefill_fp8_block(xq, xs, w, ws, N: int, y=None, ldy: int | None = None):
    M, K = xq.shape
    ldy = N if ldy is None else ldy
    y = torch.empty((M, ldy), dtype=torch.bfloat16, device=xq.device) if y is None else y
    _check(lib.lq_prefill_fp8_block(_ptr(_dev(xq, torch.uint8)), _ptr(_dev(xs, torch.float32)), M, _ptr(w),
                                    _ptr(_dev(ws, torch.float32)), _ptr(y), ldy, N, K, _stream()))
    return y


def quant_act_fp8(x, input_scale: float):
    M, K = x.shape
    q = torch.empty((M, K), dtype=torch.uint8, device=x.device)
    _check(lib.lq_quant_act_fp8(_ptr(_dev(x, torch.float32)), M, K, input_scale, _ptr(q), _stream()))
    return q


def quant_act_fp8_bf16in(x, input_scale: float):
    M, K = x.shape
    q = torch.empty((M, K), dtype=torch.uint8, device=x.device)
    _check(lib.lq_quant_act_fp8_bf16in(_ptr(_dev(x, torch.bfloat16)), M, K, input_scale, _ptr(q), _stream()))
    return q


def gated_rmsnorm_fp8(x, z, w_bf16, eps: float, input_scale: float):
    """DeltaNet output norm into FP8 (reference src/core/prefill_gemm.cu:648-660): x, z [rows][128], FP32 or both
    BF16 (the _bf16 entry point); w BF16 [128] as int16 bits or bfloat16."""
    rows, D = x.shape
    if z.shape != x.shape:
        raise ValueError("gated_rmsnorm_fp8: x and z must have the same shape")
    q = torch.empty((rows, D), dtype=torch.uint8, device=x.device)
    fn, dt = ((lib.lq_gated_rmsnorm_fp8_bf16, torch.bfloat16) if x.dtype == torch.bfloat16
              else (lib.lq_gated_rmsnorm_fp8, torch.float32))
    _check(fn(_ptr(_dev(x, dt)), _ptr(_dev(z, dt)), _ptr(_dev(w_bf16)), rows, D, eps, input_scale, _ptr(q), _stream()))
    return q


def sigmoid_mul_fp8(x, gate, input_scale: float):
    """x * sigmoid(gate) into FP8 (reference src/core/prefill_gemm.cu:662-665), elementwise over x's shape."""
    if gate.shape != x.shape:
        raise ValueError("sigmoid_mul_fp8: x and gate must have the same shape")
    q = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    _check(lib.lq_sigmoid_mul_fp8(_ptr(_dev(x, torch.float32)), _ptr(_dev(gate, torch.float32)), x.numel(),
                                  input_scale, _ptr(q), _stream()))
    return q


def prefill_gemm_fp8(xq, w, alpha: float, N: int, y=None, ldy: int | None = None, accumulate: bool = False):
    M, K = xq.shape
    ldy = N if ldy is None else ldy
    y = torch.empty((M, ldy), dtype=torch.float32, device=xq.device) if y is None else y
    _check(lib.lq_prefill_gemm_fp8(_ptr(_dev(xq, torch.uint8)), M, _ptr(w), alpha, _ptr(_dev(y, torch.float32)), ldy, N,
                                   K, int(accumulate), _stream()))
    return y


def prefill_gemm_fp8_bf16out(xq, w, alpha: float, N: int, y=None, ldy: int | None = None):
    M, K = xq.shape
    ldy = N if ldy is None else ldy
    y = torch.empty((M, ldy), dtype=torch.bfloat16, device=xq.device) if y is None else y
    _check(lib.lq_prefill_gemm_fp8_bf16out(_ptr(_dev(xq, torch.uint8)), M, _ptr(w), alpha,
                                           _ptr(_dev(y, torch.bfloat16)), ldy, N, K, _stream()))
    return y


# ---------------- host weight quantizers (numpy arrays on the host) ----------------
def _host_w(w):
    import numpy as np
    w = np.ascontiguousarray(w)
    if w.dtype == np.float32:
        return w, DT_F32
    if w.dtype == np.float16:
        return w, DT_F16
    if w.dtype == np.uint16:  # BF16 bit patterns
        return w, DT_BF16
    raise TypeError("weights must be float32, float16 or uint16 (BF16 bits)")


def quantize_nvfp4(w_bf16):
    """BF16 bits [N][K] -> (values [N][K/2], scales [N][K/16], scale2, rel_sq_err) (reference model.cu:188-249)."""
    import numpy as np
    w = np.ascontiguousarray(w_bf16, np.uint16)
    N, K = w.shape
    v = np.empty((N, K // 2), np.uint8)
    s = np.empty((N, K // 16), np.uint8)
    g = C.c_float()
    e = C.c_double()
    _check(lib.lq_quantize_nvfp4(_np_ptr(w), N, K, _np_ptr(v), _np_ptr(s), C.byref(g), C.byref(e)))
    return v, s, g.value, e.value


def quantize_fp8_channel(w):
    """[N][K] float32 / float16 / BF16 bits -> (q [N][K] E4M3, scale [N]) (drafter_variants.py:77-81)."""
    import numpy as np
    w, dt = _host_w(w)
    N, K = w.shape
    q = np.empty((N, K), np.uint8)
    s = np.empty(N, np.float32)
    _check(lib.lq_quantize_fp8_channel(_np_ptr(w), dt, N, K, _np_ptr(q), _np_ptr(s)))
    return q, s


def quantize_fp8_block128(w):
    """[N][K] -> (q [N][K] E4M3, scale [ceil(N/128)][ceil(K/128)])."""
    import numpy as np
    w, dt = _host_w(w)
    N, K = w.shape
    q = np.empty((N, K), np.uint8)
    s = np.empty(((N + 127) // 128, (K + 127) // 128), np.float32)
    _check(lib.lq_quantize_fp8_block128(_np_ptr(w), dt, N, K, _np_ptr(q), _np_ptr(s)))
    return q, s
