"""The on-disk kernel-order weight file: compile a safetensors checkpoint once, load its tiled blobs by copy.

The reference's README names an offline compiler (ling-compile) that was never built; its load path maps
the checkpoint (reference src/core/safetensors.hpp:14-52) and retiles each quantized linear on the GPU at
every load (src/core/model.cu:131-186). Here `compile_checkpoint` runs the library's host compiler
(lq_wfile_compile: CPU threads, no GPU) and `WeightFile` maps the result; `WeightFile.load` copies an
entry's sections to device memory, ready for the GEMM entry points of ling_gemm.

    python ling-engine_amd/ling_compile.py CHECKPOINT_DIR OUT.lqw [--no-codes] [--passthrough]
        [--quantize {fp8,fp8-block,nvfp4}] [--list]

--quantize also turns high-precision (BF16 / F16 / F32) linear weights into FP8 per-channel, FP8 128x128-block or
NVFP4 entries with the library's host quantizers, as the reference's loader does for its NVFP4 copies
(src/core/model.cu:188-249).
"""
from __future__ import annotations

import argparse
import ctypes as C
import dataclasses
import sys

import numpy as np
import torch

import ling_gemm as L


QUANTIZE = {None: 0, "fp8": L.WFILE_QUANT_FP8, "fp8-block": L.WFILE_QUANT_FP8_BLOCK, "nvfp4": L.WFILE_QUANT_NVFP4}


def compile_checkpoint(checkpoint_dir: str, out_path: str, codes: bool = True, passthrough: bool = False,
                       quantize: str | None = None) -> int:
    """Compile checkpoint_dir into out_path; returns the number of entries written."""
    flags = (0 if codes else L.WFILE_NO_CODES) | (L.WFILE_PASSTHROUGH if passthrough else 0) | QUANTIZE[quantize]
    n = C.c_int(0)
    L._check(L.lib.lq_wfile_compile(checkpoint_dir.encode(), out_path.encode(), flags, C.byref(n)))
    return n.value


@dataclasses.dataclass
class Entry:
    """One entry of a weight file; blob / aux / table are numpy views of the mapped file (no copy)."""
    name: str
    kind: int
    scale_kind: int
    N: int
    K: int
    weight_scale: float
    input_scale: float | None
    dtype: str
    shape: tuple
    quantized: bool
    blob: np.ndarray
    aux: np.ndarray | None
    table: np.ndarray | None


@dataclasses.dataclass
class DeviceWeight:
    """An entry on the device. w: the tiled blob (raw entries: the tensor's bytes); table: coded NVFP4's code
    table; raw_scales: coded NVFP4's raw scale copy; svec: FP8 per-channel scales [N]; block_scales: FP8
    [ceil(N/128)][ceil(K/128)]."""
    name: str
    kind: int
    N: int
    K: int
    w: torch.Tensor
    weight_scale: float
    input_scale: float | None
    table: torch.Tensor | None = None
    raw_scales: torch.Tensor | None = None
    svec: torch.Tensor | None = None
    block_scales: torch.Tensor | None = None


def _view(ptr, n):
    if not ptr or not n:
        return None
    return np.ctypeslib.as_array((C.c_uint8 * n).from_address(ptr))


class WeightFile:
    def __init__(self, path: str):
        self._h = C.c_void_p()
        L._check(L.lib.lq_wfile_open(path.encode(), C.byref(self._h)))
        self.path = path

    def close(self) -> None:
        if self._h:
            L.lib.lq_wfile_close(self._h)
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        self.close()

    def __len__(self) -> int:
        return L.lib.lq_wfile_count(self._h)

    def names(self) -> list[str]:
        return [self.entry(i).name for i in range(len(self))]

    def index(self, name: str) -> int:
        i = L.lib.lq_wfile_find(self._h, name.encode())
        if i < 0:
            raise KeyError(name)
        return i

    def entry(self, key) -> Entry:
        i = self.index(key) if isinstance(key, str) else int(key)
        e = L.WEntry()
        L._check(L.lib.lq_wfile_entry(self._h, i, C.byref(e)))
        aux = _view(e.aux, e.aux_bytes)
        return Entry(name=e.name.decode(), kind=e.kind, scale_kind=e.scale_kind, N=e.N, K=e.K,
                     weight_scale=e.weight_scale,
                     input_scale=e.input_scale if e.flags & L.WENTRY_HAS_INPUT_SCALE else None,
                     dtype=e.dtype.decode(), shape=tuple(e.shape[d] for d in range(e.ndim)),
                     quantized=bool(e.flags & L.WENTRY_QUANTIZED), blob=_view(e.blob, e.blob_bytes), aux=aux, table=_view(e.table, e.table_bytes))

    def verify(self, key) -> None:
        i = self.index(key) if isinstance(key, str) else int(key)
        L._check(L.lib.lq_wfile_verify(self._h, i))

    def load(self, key, device="cuda") -> DeviceWeight:
        """Copy an entry's sections to `device` (host -> HBM; the file's pages are read on first touch)."""
        e = self.entry(key)
        dev = lambda a: torch.from_numpy(a).to(device) if a is not None else None
        out = DeviceWeight(name=e.name, kind=e.kind, N=e.N, K=e.K, w=dev(e.blob), weight_scale=e.weight_scale,
                           input_scale=e.input_scale)
        if e.kind == L.WENTRY_NVFP4_CODED:
            out.table, out.raw_scales = dev(e.table), dev(e.aux)
        elif e.kind == L.WENTRY_FP8 and e.scale_kind == L.WSCALE_CHANNEL:
            out.svec = dev(e.aux.view(np.float32))
        elif e.kind == L.WENTRY_FP8 and e.scale_kind == L.WSCALE_BLOCK128:
            out.block_scales = dev(e.aux.view(np.float32).reshape((e.N + 127) // 128, (e.K + 127) // 128))
        return out


_KINDS = {L.WENTRY_FP8: "fp8", L.WENTRY_NVFP4: "nvfp4", L.WENTRY_NVFP4_CODED: "nvfp4-coded", L.WENTRY_RAW: "raw"}
_SCALES = {L.WSCALE_NONE: "", L.WSCALE_TENSOR: "per-tensor", L.WSCALE_CHANNEL: "per-channel",
           L.WSCALE_BLOCK128: "block128"}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="compile a safetensors checkpoint into a kernel-order weight file")
    ap.add_argument("checkpoint")
    ap.add_argument("out")
    ap.add_argument("--no-codes", action="store_true", help="write NVFP4 weights raw, never scale-coded")
    ap.add_argument("--passthrough", action="store_true", help="copy every non-quantized tensor too")
    ap.add_argument("--quantize", choices=["fp8", "fp8-block", "nvfp4"],
                    help="quantize high-precision linear weights into this format")
    ap.add_argument("--list", action="store_true", help="print the entries written")
    a = ap.parse_args(argv)
    n = compile_checkpoint(a.checkpoint, a.out, codes=not a.no_codes, passthrough=a.passthrough, quantize=a.quantize)
    print(f"{a.out}: {n} entries")
    if a.list:
        with WeightFile(a.out) as f:
            for i in range(len(f)):
                e = f.entry(i)
                print(f"  {e.name}: {_KINDS[e.kind]} {_SCALES.get(e.scale_kind, '')} N={e.N} K={e.K} "
                      f"blob={e.blob.nbytes}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
