"""CPU-side checks of the C ABI library: it loads, exports every entry point include/ling_gemm.h declares, and
its host-only functions behave (no device work is started here)."""
import ctypes as C
import os
import re

import numpy as np

import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ling_gemm.h")
LIB = os.path.join(ROOT, "ling-engine_amd", "libling_gemm.so")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lq_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(LIB)
    names = declared_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_the_header():
    import ling_gemm
    assert set(declared_functions()) == set(ling_gemm.SIGNATURES)


def test_tiled_sizes_match_oracle():
    import ling_gemm as L
    for N, K in [(16, 128), (5120, 5120), (34816, 5120), (5120, 17408), (5120, 25600)]:
        assert L.tiled_bytes_fp8(N, K) == O.lib.or_tiled_bytes_fp8(N, K)
        assert L.tiled_bytes_nvfp4(N, K) == O.lib.or_tiled_bytes_nvfp4(N, K)
        assert L.tiled_bytes_nvfp4_coded(N, K) == O.lib.or_tiled_bytes_nvfp4_coded(N, K)


def test_scale_code_table_matches_oracle():
    import ling_gemm as L
    w = O.normal_bf16(12, 0.02, (64, 512))
    _, s, _, _ = O.quant_nvfp4(w)
    ok, table, code_of = L.scale_code_table(s)
    ok2, table2, code_of2 = O.scale_code_table(s)
    assert ok and ok2
    assert np.array_equal(table, table2) and np.array_equal(code_of, code_of2)
    assert not L.scale_code_table(np.arange(100, dtype=np.uint8))[0]


def test_errors_are_reported_before_any_launch():
    import ling_gemm as L
    lib = L.lib
    # shape errors come back as status codes with the reference's message texts, no device touched
    assert lib.lq_stream_fp8_pc(None, 1, None, None, None, 16, 100, None) == 1
    assert b"K must be a multiple of 128" in lib.lq_last_error()
    assert lib.lq_stream_fp8_pc(None, 1, None, None, None, 16, 128, None) == 2  # then null pointers
    assert lib.lq_stream_gemm_fp8(None, None, 81, None, 1.0, None, 16, 128, None) == 1
    assert b"M must be in [1, 80]" in lib.lq_last_error()
    assert lib.lq_stream_gemm_multi(0, None, None, 1, None, 5, 128, None) == 1
    assert b"1 to 4 matrices per launch" in lib.lq_last_error()
    assert lib.lq_retile_fp8(None, None, 17, 128, None) == 1
    assert b"N % 16 and K % 128 must be 0" in lib.lq_last_error()
    # prefill with no rows returns silently, as the reference's does (prefill_gemm.cu:596): no launch, no error
    assert lib.lq_prefill_fp8_block(None, None, 0, None, None, None, 128, 128, 128, None) == 0
    assert lib.lq_prefill_gemm_fp8(None, 0, None, 1.0, None, 128, 128, 128, 0, None) == 0
    assert lib.lq_prefill_gemm_fp8_bf16out(None, 0, None, 1.0, None, 128, 128, 128, None) == 0
    assert lib.lq_prefill_gemm_nvfp4(None, None, 0, None, 1.0, None, 128, 128, 128, 0, None, None) == 0
    # but the shape rules still hold for it
    assert lib.lq_prefill_fp8_block(None, None, 0, None, None, None, 64, 64, 128, None) == 1


CPP = r"""
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include "ling_gemm.hpp"
namespace K = ling::kernels;
int main() {
  int fails = 0;
  if (K::tiled_bytes_fp8(5120, 5120) != size_t(5120) * 5120) ++fails;
  if (K::tiled_bytes_nvfp4(16, 128) != 16 * 64 + 16 * 8) ++fails;
  uint8_t scales[4] = {0x38, 0x40, 0x38, 0x41}, table[64], code_of[256];
  if (!K::scale_code_table(scales, 4, table, code_of) || table[0] != 0x38 || code_of[0x41] != 2) ++fails;
  // the reference's error texts, thrown before any device work
  const char* want[] = {"stream_gemm: K must be a multiple of 128", "stream_gemm: M must be in [1, 80]",
                        "stream_gemm: 1 to 4 matrices per launch", "retile_fp8: N % 16 and K % 128 must be 0",
                        "prefill_gemm: N % 128 and K % 128 must be 0"};
  for (int c = 0; c < 5; ++c) {
    try {
      if (c == 0) K::stream_gemm_fp8(nullptr, nullptr, 1, nullptr, 1.f, nullptr, 16, 100, nullptr);
      if (c == 1) K::stream_gemm_fp8(nullptr, nullptr, 81, nullptr, 1.f, nullptr, 16, 128, nullptr);
      if (c == 2) K::stream_gemm_multi(false, nullptr, nullptr, 1, nullptr, 5, 128, nullptr);
      if (c == 3) K::retile_fp8(nullptr, nullptr, 17, 128, nullptr);
      if (c == 4) K::prefill_gemm_fp8_block(nullptr, nullptr, 4, nullptr, nullptr, nullptr, 64, 64, 128, nullptr);
      ++fails;
    } catch (const std::runtime_error& e) {
      if (std::strcmp(e.what(), want[c]) != 0) { std::printf("got '%s'\n", e.what()); ++fails; }
    }
  }
  // host quantizers (CPU only): an all-zero matrix has g = 1 and zero codes; 448 and -224 on one channel of
  // scale 1 encode as 0x7e and 0xf6 (E4M3 1.75 x 2^8, -1.75 x 2^7)
  uint16_t wz[16 * 16] = {};
  uint8_t v[16 * 8], sc[16];
  if (K::quantize_nvfp4(wz, 16, 16, v, sc) != 1.f) ++fails;
  for (int i = 0; i < 16 * 8; ++i) if (v[i]) ++fails;
  float w1[2] = {448.f, -224.f};
  uint8_t q1[2];
  float s1 = 0.f;
  K::quantize_fp8_channel(w1, LQ_DT_F32, 1, 2, q1, &s1);
  if (s1 != 1.f || q1[0] != 0x7e || q1[1] != 0xf6) ++fails;
  try {
    K::quantize_nvfp4(wz, 16, 8, v, sc);
    ++fails;
  } catch (const std::runtime_error& e) {
    if (std::strcmp(e.what(), "quantize_nvfp4: K must be a positive multiple of 16") != 0) ++fails;
  }
  std::printf("fails=%d\n", fails);
  return fails;
}
"""


def test_cpp_wrapper_compiles_and_throws_reference_messages(tmp_path):
    import subprocess
    src = tmp_path / "w.cpp"
    src.write_text(CPP)
    exe = tmp_path / "w"
    libdir = os.path.dirname(LIB)
    cmd = ["/opt/rocm/bin/hipcc", "-std=c++17", "-O1", str(src), "-o", str(exe), f"-I{ROOT}/include", f"-L{libdir}",
           "-lling_gemm", f"-Wl,-rpath,{libdir}", "--offload-arch=gfx950"]
    subprocess.run(cmd, check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "fails=0" in r.stdout
