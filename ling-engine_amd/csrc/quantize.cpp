// Host weight quantizers: the formats the GEMMs read, made from high-precision (BF16 / F16 / F32) weights on CPU
// threads. They are the library's own (the oracle holds an independent restatement the tests compare against):
//
//  * NVFP4 round-to-nearest (reference src/core/model.cu:188-249, quantize_nvfp4): global scale g = amax / (448 * 6)
//    (1 for an all-zero matrix); per 16-value block the E4M3 scale sc = E4M3(max(amax16 / 6 / g, 2^-9)); each value
//    x / (e4m3(sc) * g) takes the E2M1 code of the nearest magnitude, ties to the smaller magnitude (the reference's
//    walk over the bounds {0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5}), with the sign only on a non-zero code.
//  * FP8 per output channel (reference bench/quant/drafter_variants.py:77-81, fake_fp8): s_n = max(amax_n / 448,
//    1e-12), q = E4M3(w / s_n).
//  * FP8 in 128 x 128 blocks (the prefill's weight format): s = amax_block / 448 (1 for an all-zero block),
//    q = E4M3(w / s).
// E4M3 is the OCP E4M3FN format, encoded with round-to-nearest-even and saturation to +-448 (NaN -> 0x7f).
#include "lq_quantize.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <string>
#include <thread>
#include <vector>

#include "lq_common.hpp"

namespace lq {
namespace hostq {

uint8_t e4m3_encode(float x) {
  if (std::isnan(x)) return 0x7f;
  const uint8_t sign = std::signbit(x) ? 0x80 : 0x00;
  const float a = std::fabs(x);
  if (a >= 448.f) return sign | 0x7e;  // satfinite (also every value that would round above 448)
  if (a < 0x1p-6f) {
    // subnormal: a / 2^-9 in [0, 8), rounded to nearest even; 8 is the smallest normal's code
    const float m = std::nearbyint(a * 0x1p9f);
    return sign | static_cast<uint8_t>(m);
  }
  int e2 = 0;
  (void)std::frexp(a, &e2);  // a = f * 2^e2, f in [0.5, 1)
  int e = e2 - 1;            // a in [2^e, 2^(e+1))
  float m = std::nearbyint(std::ldexp(a, 3 - e));  // in [8, 16], exact scaling then RNE
  if (m == 16.f) {
    m = 8.f;
    ++e;
  }
  const int code = ((e + 7) << 3) | (static_cast<int>(m) - 8);
  return sign | static_cast<uint8_t>(std::min(code, 0x7e));
}

float e4m3_decode(uint8_t c) {
  const int e = (c >> 3) & 15, m = c & 7;
  if (e == 15 && m == 7) return NAN;
  const float v = e == 0 ? std::ldexp(static_cast<float>(m), -9) : std::ldexp(static_cast<float>(8 + m), e - 10);
  return (c & 0x80) ? -v : v;
}

float bf16_to_f32(uint16_t b) {
  const uint32_t u = static_cast<uint32_t>(b) << 16;
  float v;
  std::memcpy(&v, &u, 4);
  return v;
}

uint16_t f32_to_bf16(float x) {
  uint32_t u;
  std::memcpy(&u, &x, 4);
  if (std::isnan(x)) return static_cast<uint16_t>((u >> 16) | 0x40);
  u += 0x7fff + ((u >> 16) & 1);
  return static_cast<uint16_t>(u >> 16);
}

float f16_to_f32(uint16_t h) {
  const uint32_t s = (h >> 15) & 1, e = (h >> 10) & 31, m = h & 1023;
  float v;
  if (e == 0) v = std::ldexp(static_cast<float>(m), -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = std::ldexp(static_cast<float>(m | 1024), static_cast<int>(e) - 25);
  return s ? -v : v;
}

float element(const void* w, int dtype, size_t i) {
  if (dtype & kRoundBf16) return bf16_to_f32(f32_to_bf16(element(w, dtype & ~kRoundBf16, i)));
  switch (dtype) {
    case LQ_DT_BF16: return bf16_to_f32(static_cast<const uint16_t*>(w)[i]);
    case LQ_DT_F16: return f16_to_f32(static_cast<const uint16_t*>(w)[i]);
    default: return static_cast<const float*>(w)[i];
  }
}

namespace {

// fn(lo, hi) over [0, n) on up to 16 threads
void parallel_rows(int n, const std::function<void(int, int)>& fn) {
  const int hw = static_cast<int>(std::max(1u, std::thread::hardware_concurrency()));
  const int nt = std::max(1, std::min({hw, 16, n}));
  if (nt == 1) {
    fn(0, n);
    return;
  }
  std::vector<std::thread> ts;
  for (int t = 0; t < nt; ++t) {
    const int lo = static_cast<int>(int64_t(n) * t / nt), hi = static_cast<int>(int64_t(n) * (t + 1) / nt);
    ts.emplace_back([&fn, lo, hi] { fn(lo, hi); });
  }
  for (auto& th : ts) th.join();
}

constexpr float kE2M1[8] = {0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};
constexpr float kBounds[7] = {0.25f, 0.75f, 1.25f, 1.75f, 2.5f, 3.5f, 5.f};

}  // namespace

float nvfp4_scales(const void* w, int dtype, int N, int K, uint8_t* scales) {
  std::vector<float> amax(N, 0.f);
  parallel_rows(N, [&](int r0, int r1) {
    for (int r = r0; r < r1; ++r) {
      float m = 0.f;
      for (size_t i = size_t(r) * K; i < size_t(r + 1) * K; ++i) m = std::max(m, std::fabs(element(w, dtype, i)));
      amax[r] = m;
    }
  });
  const float mx = N ? *std::max_element(amax.begin(), amax.end()) : 0.f;
  const float g = mx > 0.f ? mx / (448.f * 6.f) : 1.f;
  parallel_rows(N, [&](int r0, int r1) {
    for (int r = r0; r < r1; ++r)
      for (int b = 0; b < K / 16; ++b) {
        const size_t base = size_t(r) * K + size_t(b) * 16;
        float bm = 0.f;
        for (int j = 0; j < 16; ++j) bm = std::max(bm, std::fabs(element(w, dtype, base + j)));
        scales[size_t(r) * (K / 16) + b] = e4m3_encode(std::max(bm / 6.f / g, 0x1p-9f));
      }
  });
  return g;
}

double nvfp4_values(const void* w, int dtype, int N, int K, float g, const uint8_t* scales, uint8_t* values) {
  std::vector<double> err(N, 0.0), ref(N, 0.0);
  parallel_rows(N, [&](int r0, int r1) {
    for (int r = r0; r < r1; ++r) {
      double e = 0, s2 = 0;
      for (int b = 0; b < K / 16; ++b) {
        const size_t base = size_t(r) * K + size_t(b) * 16;
        const float s = e4m3_decode(scales[size_t(r) * (K / 16) + b]) * g;
        for (int j = 0; j < 16; j += 2) {
          uint8_t pair = 0;
          for (int h = 0; h < 2; ++h) {
            const float x = element(w, dtype, base + j + h), a = std::fabs(x / s);
            uint8_t c = 0;
            while (c < 7 && kBounds[c] < a) ++c;
            const float dq = (x < 0.f ? -kE2M1[c] : kE2M1[c]) * s;
            if (x < 0.f && c > 0) c |= 8;
            pair |= static_cast<uint8_t>(c << (4 * h));
            e += double(dq - x) * double(dq - x);
            s2 += double(x) * double(x);
          }
          values[(base + j) / 2] = pair;
        }
      }
      err[r] = e;
      ref[r] = s2;
    }
  });
  double e = 0, s2 = 0;
  for (int r = 0; r < N; ++r) e += err[r], s2 += ref[r];
  return s2 > 0 ? e / s2 : 0.0;
}

void fp8_channel(const void* w, int dtype, int N, int K, uint8_t* q, float* scale) {
  parallel_rows(N, [&](int r0, int r1) {
    for (int r = r0; r < r1; ++r) {
      float m = 0.f;
      for (size_t i = size_t(r) * K; i < size_t(r + 1) * K; ++i) m = std::max(m, std::fabs(element(w, dtype, i)));
      const float s = std::max(m / 448.f, 1e-12f);
      scale[r] = s;
      for (size_t i = size_t(r) * K; i < size_t(r + 1) * K; ++i) q[i] = e4m3_encode(element(w, dtype, i) / s);
    }
  });
}

void fp8_block128(const void* w, int dtype, int N, int K, uint8_t* q, float* scale) {
  const int NB = (N + 127) / 128, KB = (K + 127) / 128;
  parallel_rows(NB, [&](int b0, int b1) {
    for (int nb = b0; nb < b1; ++nb)
      for (int kb = 0; kb < KB; ++kb) {
        const int n0 = nb * 128, n1 = std::min(N, n0 + 128), k0 = kb * 128, k1 = std::min(K, k0 + 128);
        float m = 0.f;
        for (int n = n0; n < n1; ++n)
          for (int k = k0; k < k1; ++k) m = std::max(m, std::fabs(element(w, dtype, size_t(n) * K + k)));
        const float s = m > 0.f ? m / 448.f : 1.f;
        scale[size_t(nb) * KB + kb] = s;
        for (int n = n0; n < n1; ++n)
          for (int k = k0; k < k1; ++k) q[size_t(n) * K + k] = e4m3_encode(element(w, dtype, size_t(n) * K + k) / s);
      }
  });
}

}  // namespace hostq
}  // namespace lq

extern "C" {

static int check_q(const char* name, const void* w, const void* a, const void* b, int dtype, int N, int K, int kmul) {
  if (!w || !a || !b) return lq::fail(LQ_ERR_ARG, std::string(name) + ": null pointer");
  if (dtype != LQ_DT_F32 && dtype != LQ_DT_BF16 && dtype != LQ_DT_F16)
    return lq::fail(LQ_ERR_ARG, std::string(name) + ": dtype must be LQ_DT_F32, LQ_DT_BF16 or LQ_DT_F16");
  if (N <= 0 || K <= 0 || K % kmul != 0)
    return lq::fail(LQ_ERR_SHAPE, std::string(name) + ": K must be a positive multiple of " + std::to_string(kmul));
  return LQ_OK;
}

int lq_quantize_nvfp4(const uint16_t* w_bf16, int N, int K, uint8_t* values, uint8_t* scales, float* scale2,
                      double* rel_sq_err) {
  if (int rc = check_q("quantize_nvfp4", w_bf16, values, scales, LQ_DT_BF16, N, K, 16)) return rc;
  if (!scale2) return lq::fail(LQ_ERR_ARG, "quantize_nvfp4: null pointer");
  const float g = lq::hostq::nvfp4_scales(w_bf16, LQ_DT_BF16, N, K, scales);
  const double e = lq::hostq::nvfp4_values(w_bf16, LQ_DT_BF16, N, K, g, scales, values);
  *scale2 = g;
  if (rel_sq_err) *rel_sq_err = e;
  return LQ_OK;
}

int lq_quantize_fp8_channel(const void* w, int dtype, int N, int K, uint8_t* q, float* scale) {
  if (int rc = check_q("quantize_fp8_channel", w, q, scale, dtype, N, K, 1)) return rc;
  lq::hostq::fp8_channel(w, dtype, N, K, q, scale);
  return LQ_OK;
}

int lq_quantize_fp8_block128(const void* w, int dtype, int N, int K, uint8_t* q, float* scale) {
  if (int rc = check_q("quantize_fp8_block128", w, q, scale, dtype, N, K, 1)) return rc;
  lq::hostq::fp8_block128(w, dtype, N, K, q, scale);
  return LQ_OK;
}

}  // extern "C"
