/*
 * CPU oracle for the fused quantized GEMM path: TEST INFRASTRUCTURE ONLY (see oracle.h).
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it, as the checker or as the
 * timed CPU baseline; the product never calls it.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------------------------------------ */
/* generator                                                                                          */
/* ------------------------------------------------------------------------------------------------ */

void or_rng_init(or_rng* r, uint64_t seed) {
  r->s = seed;
  r->have = 0;
  r->spare = 0.0;
}

/* splitmix64 (Steele, Lea, Flood 2014) */
uint64_t or_rng_next(or_rng* r) {
  uint64_t z = (r->s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static double uniform_open(or_rng* r) { /* (0, 1]: 53 random bits */
  return ((double)(or_rng_next(r) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

/* Box-Muller in double; the second value of each pair is kept for the next call. */
double or_rng_normal(or_rng* r) {
  if (r->have) {
    r->have = 0;
    return r->spare;
  }
  const double u1 = uniform_open(r), u2 = uniform_open(r);
  const double rad = sqrt(-2.0 * log(u1)), th = 6.283185307179586 * u2;
  r->spare = rad * sin(th);
  r->have = 1;
  return rad * cos(th);
}

void or_fill_normal(uint64_t seed, float sigma, float* out, size_t n) {
  or_rng r;
  or_rng_init(&r, seed);
  for (size_t i = 0; i < n; ++i) out[i] = (float)(or_rng_normal(&r) * (double)sigma);
}

void or_fill_normal_bf16(uint64_t seed, float sigma, uint16_t* out, size_t n) {
  or_rng r;
  or_rng_init(&r, seed);
  for (size_t i = 0; i < n; ++i) out[i] = or_bf16_bits((float)(or_rng_normal(&r) * (double)sigma));
}

/* ------------------------------------------------------------------------------------------------ */
/* codecs                                                                                             */
/* ------------------------------------------------------------------------------------------------ */

static uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* OCP 8-bit floating point spec (2023), E4M3: exponent bias 7, 3 mantissa bits, no infinities,
 * S.1111.111 is NaN, so the largest finite magnitude is 1.75 * 2^8 = 448; subnormals m * 2^-9. */
float or_e4m3_decode(uint8_t c) {
  const int e = (c >> 3) & 15, m = c & 7;
  float v;
  if (e == 15 && m == 7) return NAN;
  if (e == 0) v = ldexpf((float)m, -9);
  else v = ldexpf((float)(8 + m), e - 10);
  return (c & 0x80) ? -v : v;
}

/* Round to nearest, ties to even, on the E4M3 grid; magnitudes past 448 saturate to 448. */
uint8_t or_e4m3_encode(float x) {
  if (isnan(x)) return 0x7f;
  const uint8_t sign = signbit(x) ? 0x80 : 0;
  const double a = fabs((double)x);
  if (a >= 448.0) return sign | 0x7e;
  if (a < 0.015625) { /* below 2^-6: subnormal grid of 2^-9 */
    const double m = nearbyint(a * 512.0); /* 0 .. 8; 8 is the smallest normal, code 0x08 */
    return sign | (uint8_t)m;
  }
  int e;
  const double fr = frexp(a, &e); /* a = fr * 2^e, fr in [0.5, 1) */
  e -= 1;                         /* a = (2 fr) * 2^e, 2 fr in [1, 2) */
  double m = nearbyint((2.0 * fr - 1.0) * 8.0);
  if (m == 8.0) {
    m = 0.0;
    e += 1;
  }
  /* e <= 8 here; 1.875 * 2^8 (=480) cannot occur since a < 448 rounds at most to 448 */
  return sign | (uint8_t)(((e + 7) << 3) | (int)m);
}

static const float kE2M1[8] = {0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};

float or_e2m1_decode(uint8_t nib) {
  const float v = kE2M1[nib & 7];
  return (nib & 8) ? -v : v;
}

/* model.cu:223-229: the first code whose upper bound is >= |y|, so a value halfway between two codes
 * takes the smaller magnitude; the sign bit only on a non-zero code. */
uint8_t or_e2m1_encode_weight(float y) {
  static const float kBounds[7] = {0.25f, 0.75f, 1.25f, 1.75f, 2.5f, 3.5f, 5.f};
  const float a = fabsf(y);
  uint8_t c = 0;
  while (c < 7 && kBounds[c] < a) ++c;
  if (y < 0.f && c > 0) c |= 8;
  return c;
}

/* Textbook round to nearest on the E2M1 grid with ties to the even code (even mantissa bit), saturating
 * at 6, sign kept (the activation quantizer's rule, tests/prefill_tests.cu:44-54 restated). */
uint8_t or_e2m1_encode_rne(float y) {
  const float a = fabsf(y);
  int best = 0;
  if (a >= 6.f || isnan(a)) best = 7;
  else {
    for (int i = 1; i < 8; ++i) {
      const float d = fabsf(kE2M1[i] - a), db = fabsf(kE2M1[best] - a);
      if (d < db || (d == db && (i & 1) == 0)) best = i;
    }
  }
  return (uint8_t)(best | (signbit(y) ? 8 : 0));
}

uint16_t or_bf16_bits(float x) {
  const uint32_t u = f2u(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40); /* quiet NaN */
  const uint32_t r = u + 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(r >> 16);
}

float or_bf16_float(uint16_t b) { return u2f((uint32_t)b << 16); }

uint16_t or_f16_bits(float x) {
  const uint16_t sign = signbit(x) ? 0x8000 : 0;
  if (isnan(x)) return 0x7e00;
  const double a = fabs((double)x);
  if (a >= 65520.0) return sign | 0x7c00; /* halfway to 2^16 and above round to inf */
  if (a < 6.103515625e-05) {              /* below 2^-14: subnormal grid of 2^-24 */
    const double m = nearbyint(a * 16777216.0);
    return sign | (uint16_t)m; /* m == 1024 is the smallest normal's bit pattern */
  }
  int e;
  const double fr = frexp(a, &e);
  e -= 1;
  double m = nearbyint((2.0 * fr - 1.0) * 1024.0);
  if (m == 1024.0) {
    m = 0.0;
    e += 1;
  }
  if (e > 15) return sign | 0x7c00;
  return sign | (uint16_t)(((e + 15) << 10) | (int)m);
}

float or_f16_float(uint16_t h) {
  const int e = (h >> 10) & 31, m = h & 1023;
  float v;
  if (e == 31) v = m ? NAN : INFINITY;
  else if (e == 0) v = ldexpf((float)m, -24);
  else v = ldexpf((float)(1024 + m), e - 25);
  return (h & 0x8000) ? -v : v;
}

/* ------------------------------------------------------------------------------------------------ */
/* weight and activation quantizers                                                                   */
/* ------------------------------------------------------------------------------------------------ */

void or_quant_fp8_per_channel(const float* w, int N, int K, uint8_t* q, float* scale) {
  for (int n = 0; n < N; ++n) {
    const float* row = w + (size_t)n * K;
    float amax = 0.f;
    for (int k = 0; k < K; ++k) amax = fmaxf(amax, fabsf(row[k]));
    float s = amax / 448.f;
    if (s < 1e-12f) s = 1e-12f;
    scale[n] = s;
    for (int k = 0; k < K; ++k) q[(size_t)n * K + k] = or_e4m3_encode(row[k] / s);
  }
}

float or_quant_nvfp4(const uint16_t* w, int N, int K, uint8_t* values, uint8_t* scales, double* rel_sq_err) {
  float mx = 0.f;
  for (size_t i = 0; i < (size_t)N * K; ++i) mx = fmaxf(mx, fabsf(or_bf16_float(w[i])));
  const float g = mx > 0.f ? mx / (448.f * 6.f) : 1.f;
  memset(values, 0, (size_t)N * K / 2);
  double err = 0.0, ref = 0.0;
  for (int r = 0; r < N; ++r)
    for (int b = 0; b < K / 16; ++b) {
      const size_t base = (size_t)r * K + (size_t)b * 16;
      float bm = 0.f;
      for (int j = 0; j < 16; ++j) bm = fmaxf(bm, fabsf(or_bf16_float(w[base + j])));
      float sv = bm / 6.f / g;
      if (sv < 0x1p-9f) sv = 0x1p-9f;
      const uint8_t sc = or_e4m3_encode(sv);
      scales[(size_t)r * (K / 16) + b] = sc;
      const float s = or_e4m3_decode(sc) * g;
      for (int j = 0; j < 16; ++j) {
        const float x = or_bf16_float(w[base + j]);
        const uint8_t c = or_e2m1_encode_weight(x / s);
        const float dq = or_e2m1_decode(c) * s;
        values[(base + j) / 2] |= (uint8_t)((j & 1) ? (c << 4) : c);
        err += ((double)dq - x) * ((double)dq - x);
        ref += (double)x * x;
      }
    }
  if (rel_sq_err) *rel_sq_err = ref > 0 ? err / ref : 0.0;
  return g;
}

void or_quant_fp8_block128(const float* w, int N, int K, uint8_t* q, float* scale) {
  const int KB = K / 128;
  for (int nb = 0; nb < N / 128; ++nb)
    for (int kb = 0; kb < KB; ++kb) {
      float amax = 0.f;
      for (int r = 0; r < 128; ++r)
        for (int c = 0; c < 128; ++c) amax = fmaxf(amax, fabsf(w[(size_t)(nb * 128 + r) * K + kb * 128 + c]));
      const float s = amax > 0.f ? amax / 448.f : 1.f;
      scale[(size_t)nb * KB + kb] = s;
      for (int r = 0; r < 128; ++r)
        for (int c = 0; c < 128; ++c) {
          const size_t i = (size_t)(nb * 128 + r) * K + kb * 128 + c;
          q[i] = or_e4m3_encode(w[i] / s);
        }
    }
}

void or_quant_act_fp8_g128(const uint16_t* x, int M, int K, uint8_t* q, float* scale) {
  const int KB = K / 128;
  for (int m = 0; m < M; ++m)
    for (int kb = 0; kb < KB; ++kb) {
      const size_t base = (size_t)m * K + (size_t)kb * 128;
      float amax = 0.f;
      for (int c = 0; c < 128; ++c) amax = fmaxf(amax, fabsf(or_bf16_float(x[base + c])));
      const float s = amax > 0.f ? amax / 448.f : 1.f;
      scale[(size_t)m * KB + kb] = s;
      const float r = 1.f / s;  /* x times the reciprocal, each rounded to FP32 (the library's definition) */
      for (int c = 0; c < 128; ++c) {
        const float v = or_bf16_float(x[base + c]) * r;
        q[base + c] = or_e4m3_encode(v);
      }
    }
}

/* ------------------------------------------------------------------------------------------------ */
/* tiled layout                                                                                       */
/* ------------------------------------------------------------------------------------------------ */

enum { kChunk = 128, kTileFp8 = 2048, kTileFp4 = 1152, kValFp4 = 1024, kCodeFp4 = 96 };

size_t or_tiled_bytes_fp8(int N, int K) { return (size_t)N * K; }
size_t or_tiled_bytes_nvfp4(int N, int K) { return (size_t)N * K / 2 + (size_t)N * K / 16; }
size_t or_tiled_bytes_nvfp4_coded(int N, int K) { return (size_t)(N / 16) * (K / kChunk) * (kValFp4 + kCodeFp4); }

/* FP8 block (tile, chunk), 16-byte piece p = ((h*2 + q)*8 + g)*4 + t holds row 16*tile + g + 8h,
 * values [128*chunk + 32t + 16q, +16) (stream_gemm.cu:725-738). */
static void fp8_piece(int p, int* row_in_tile, int* k_in_chunk) {
  const int t = p & 3, g = (p >> 2) & 7, q = (p >> 5) & 1, h = p >> 6;
  *row_in_tile = g + 8 * h;
  *k_in_chunk = 32 * t + 16 * q;
}

void or_retile_fp8(const uint8_t* w, uint8_t* out, int N, int K) {
  const int C = K / kChunk;
  for (int tile = 0; tile < N / 16; ++tile)
    for (int c = 0; c < C; ++c)
      for (int p = 0; p < 128; ++p) {
        int r, kk;
        fp8_piece(p, &r, &kk);
        memcpy(out + ((size_t)tile * C + c) * kTileFp8 + p * 16, w + (size_t)(tile * 16 + r) * K + c * kChunk + kk, 16);
      }
}

void or_untile_fp8(const uint8_t* tiled, uint8_t* w, int N, int K) {
  const int C = K / kChunk;
  for (int tile = 0; tile < N / 16; ++tile)
    for (int c = 0; c < C; ++c)
      for (int p = 0; p < 128; ++p) {
        int r, kk;
        fp8_piece(p, &r, &kk);
        memcpy(w + (size_t)(tile * 16 + r) * K + c * kChunk + kk, tiled + ((size_t)tile * C + c) * kTileFp8 + p * 16, 16);
      }
}

/* NVFP4 block: slot s = r*4 + t (r the row in the tile) holds 16 bytes = values [32t, +32) of the chunk,
 * and 2 scale bytes at 1024 + 2s (stream_gemm.cu:705-723). */
void or_retile_nvfp4(const uint8_t* values, const uint8_t* scales, uint8_t* out, int N, int K) {
  const int C = K / kChunk;
  for (int tile = 0; tile < N / 16; ++tile)
    for (int c = 0; c < C; ++c) {
      uint8_t* blk = out + ((size_t)tile * C + c) * kTileFp4;
      for (int s = 0; s < 64; ++s) {
        const int r = s >> 2, t = s & 3;
        const size_t n = (size_t)tile * 16 + r;
        memcpy(blk + s * 16, values + n * (K / 2) + c * 64 + t * 16, 16);
        memcpy(blk + 1024 + s * 2, scales + n * (K / 16) + c * 8 + t * 2, 2);
      }
    }
}

void or_untile_nvfp4(const uint8_t* tiled, uint8_t* values, uint8_t* scales, int N, int K) {
  const int C = K / kChunk;
  for (int tile = 0; tile < N / 16; ++tile)
    for (int c = 0; c < C; ++c) {
      const uint8_t* blk = tiled + ((size_t)tile * C + c) * kTileFp4;
      for (int s = 0; s < 64; ++s) {
        const int r = s >> 2, t = s & 3;
        const size_t n = (size_t)tile * 16 + r;
        memcpy(values + n * (K / 2) + c * 64 + t * 16, blk + s * 16, 16);
        memcpy(scales + n * (K / 16) + c * 8 + t * 2, blk + 1024 + s * 2, 2);
      }
    }
}

int or_scale_code_table(const uint8_t* scales, size_t n, uint8_t* table, uint8_t* code_of) {
  size_t count[256] = {0};
  for (size_t i = 0; i < n; ++i) ++count[scales[i]];
  int distinct = 0;
  for (int v = 0; v < 256; ++v) distinct += count[v] > 0;
  if (distinct > 64) return 0;
  memset(table, 0, 64);
  memset(code_of, 0xff, 256);
  int next = 0;
  for (int v = 0; v < 256; ++v)
    if (count[v]) {
      code_of[v] = (uint8_t)next;
      table[next++] = (uint8_t)v;
    }
  return 1;
}

/* The coded blob (stream_gemm.cu:740-780): every block's 1024 value bytes, then every block's 96 code
 * bytes. A slot's two 6-bit codes form 12 bits (first scale low); lane L's slots L and L+32 keep their low
 * bytes at 2L, 2L+1 and their high nibbles in byte 64+L. raw_scales: 128 bytes per block, slot order. */
void or_retile_nvfp4_coded(const uint8_t* values, const uint8_t* scales, const uint8_t* code_of, uint8_t* out,
                           uint8_t* raw, int N, int K) {
  const int C = K / kChunk;
  const size_t blocks = (size_t)(N / 16) * C;
  memset(out, 0, or_tiled_bytes_nvfp4_coded(N, K));
  for (size_t blk = 0; blk < blocks; ++blk) {
    const int tile = (int)(blk / C), c = (int)(blk % C);
    uint32_t f[64];
    for (int s = 0; s < 64; ++s) {
      const int r = s >> 2, t = s & 3;
      const size_t n = (size_t)tile * 16 + r;
      memcpy(out + blk * kValFp4 + s * 16, values + n * (K / 2) + c * 64 + t * 16, 16);
      const uint8_t s0 = scales[n * (K / 16) + c * 8 + t * 2], s1 = scales[n * (K / 16) + c * 8 + t * 2 + 1];
      raw[blk * 128 + s * 2] = s0;
      raw[blk * 128 + s * 2 + 1] = s1;
      f[s] = (uint32_t)code_of[s0] | ((uint32_t)code_of[s1] << 6);
    }
    uint8_t* dst = out + blocks * kValFp4 + blk * kCodeFp4;
    for (int L = 0; L < 32; ++L) {
      dst[2 * L] = (uint8_t)(f[L] & 0xff);
      dst[2 * L + 1] = (uint8_t)(f[L + 32] & 0xff);
      dst[64 + L] = (uint8_t)((f[L] >> 8) | ((f[L + 32] >> 8) << 4));
    }
  }
}

/* ------------------------------------------------------------------------------------------------ */
/* dequantization                                                                                     */
/* ------------------------------------------------------------------------------------------------ */

void or_dequant_fp8_pc(const uint8_t* q, const float* scale, int N, int K, float* out) {
  for (int n = 0; n < N; ++n)
    for (int k = 0; k < K; ++k) out[(size_t)n * K + k] = or_e4m3_decode(q[(size_t)n * K + k]) * scale[n];
}

void or_dequant_nvfp4(const uint8_t* values, const uint8_t* scales, float scale2, int N, int K, float* out) {
  for (int n = 0; n < N; ++n)
    for (int k = 0; k < K; ++k) {
      const float s = or_e4m3_decode(scales[(size_t)n * (K / 16) + k / 16]) * scale2;
      const uint8_t b = values[((size_t)n * K + k) / 2];
      out[(size_t)n * K + k] = or_e2m1_decode((k & 1) ? (b >> 4) : (b & 15)) * s;
    }
}

void or_dequant_fp8_block128(const uint8_t* q, const float* scale, int N, int K, float* out) {
  const int KB = K / 128;
  for (int n = 0; n < N; ++n)
    for (int k = 0; k < K; ++k)
      out[(size_t)n * K + k] = or_e4m3_decode(q[(size_t)n * K + k]) * scale[(size_t)(n / 128) * KB + k / 128];
}

void or_to_half_rows(const float* x, int M, int K, uint16_t* xh, float* xinv) {
  for (int m = 0; m < M; ++m) {
    const float* row = x + (size_t)m * K;
    float mx = 0.f;
    for (int k = 0; k < K; ++k) mx = fmaxf(mx, fabsf(row[k]));
    int e = 0;
    if (mx > 0.f && isfinite(mx)) frexpf(mx, &e);
    const float s = ldexpf(1.f, 15 - e);
    for (int k = 0; k < K; ++k) xh[(size_t)m * K + k] = or_f16_bits(row[k] * s);
    xinv[m] = ldexpf(1.f, e - 15);
  }
}

/* RMSNorm + FP16 row copy (stream_gemm.cu:380-418): the sum of squares in double (any FP32 order of the
 * device is within its rounding of this), rstd = 1 / sqrtf(float(sum / H) + eps), v = x * rstd * w' in FP32
 * (w' = 1 + w for Gemma), then the to_half_rows conversion of v. */
void or_rmsnorm_half(const float* x, const uint16_t* w, int rows, int H, float eps, int gemma, float* out,
                     uint16_t* xh, float* xinv) {
  for (int r = 0; r < rows; ++r) {
    const float* row = x + (size_t)r * H;
    double ss = 0.0;
    for (int h = 0; h < H; ++h) ss += (double)row[h] * row[h];
    const float rstd = 1.f / sqrtf((float)(ss / H) + eps);
    for (int h = 0; h < H; ++h) {
      const float wf = or_bf16_float(w[h]);
      out[(size_t)r * H + h] = row[h] * rstd * (gemma ? 1.f + wf : wf);
    }
  }
  or_to_half_rows(out, rows, H, xh, xinv);
}

/* Per-tensor FP8 activation quantizer (prefill_gemm.cu:496-511): E4M3_satfinite(bf16(x) * (1 / input_scale)). */
void or_quant_act_fp8(const float* x, size_t n, float input_scale, uint8_t* q) {
  const float inv = 1.f / input_scale;
  for (size_t i = 0; i < n; ++i) q[i] = or_e4m3_encode(or_bf16_float(or_bf16_bits(x[i])) * inv);
}

/* NVFP4 activation block (reference put_nvfp4, src/core/prefill_gemm.cu:382-394; the host restatement the
 * reference's own test checks the device against, tests/prefill_tests.cu:71-80): 16 values already rounded to
 * BF16, g = 1 / input_scale; sc = E4M3(g * (amax * (1/6))), os = sv != 0 ? 1 / (sv * (1/g)) : 0, codes =
 * E2M1 RNE (ties to the even code, saturating, sign kept) of v * os, low nibble first. */
static void nvfp4_act_block(const float* v, float g, uint8_t* q8, uint8_t* sfb) {
  float amax = 0.f;
  for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
  const uint8_t sc = or_e4m3_encode(g * (amax * (1.f / 6.f)));
  const float sv = or_e4m3_decode(sc);
  const float os = sv != 0.f ? 1.f / (sv * (1.f / g)) : 0.f;
  for (int i = 0; i < 16; i += 2)
    q8[i / 2] = (uint8_t)(or_e2m1_encode_rne(v[i] * os) | (or_e2m1_encode_rne(v[i + 1] * os) << 4));
  *sfb = sc;
}

/* quant_act_nvfp4 (reference src/core/prefill_gemm.cu:404-420, 607-611): x [M][K] FP32 -> q [M][K/2], sf [M][K/16]. */
void or_quant_act_nvfp4(const float* x, int M, int K, float input_scale, uint8_t* q, uint8_t* sf) {
  const float g = 1.f / input_scale;
  const size_t blocks = (size_t)M * K / 16;
  for (size_t b = 0; b < blocks; ++b) {
    float v[16];
    for (int i = 0; i < 16; ++i) v[i] = or_bf16_float(or_bf16_bits(x[b * 16 + i]));
    nvfp4_act_block(v, g, q + b * 8, sf + b);
  }
}

/* silu_mul_quant_nvfp4 (reference prefill_gemm.cu:404-420 with SILU, 613-618): the values are silu(g) * u. */
void or_silu_mul_quant_nvfp4(const float* gt, const float* u, int M, int K, float input_scale, uint8_t* q, uint8_t* sf) {
  const float g = 1.f / input_scale;
  const size_t blocks = (size_t)M * K / 16;
  for (size_t b = 0; b < blocks; ++b) {
    float v[16];
    for (int i = 0; i < 16; ++i) v[i] = or_bf16_float(or_bf16_bits(or_silu(gt[b * 16 + i]) * u[b * 16 + i]));
    nvfp4_act_block(v, g, q + b * 8, sf + b);
  }
}

/* rmsnorm_quant (reference norm_quant_kernel, prefill_gemm.cu:426-459, 632-637): Gemma RMSNorm of each row,
 * v = x * rstd * (1 + w), rstd = 1 / sqrt(sum(x^2) / H + eps) (the sum in double here), into `out` when given,
 * then BF16(v) into NVFP4 or FP8 E4M3(BF16(v) * (1 / input_scale)) saturated. */
void or_rmsnorm_quant(const float* x, const uint16_t* w, float* out, int M, int H, float eps, int nvfp4,
                      float input_scale, uint8_t* q, uint8_t* sf) {
  const float g = 1.f / input_scale;
  float* v = (float*)malloc(sizeof(float) * (size_t)H);
  for (int r = 0; r < M; ++r) {
    const float* row = x + (size_t)r * H;
    double ss = 0.0;
    for (int h = 0; h < H; ++h) ss += (double)row[h] * row[h];
    const float rstd = 1.f / sqrtf((float)(ss / H) + eps);
    for (int h = 0; h < H; ++h) {
      v[h] = row[h] * rstd * (1.f + or_bf16_float(w[h]));
      if (out) out[(size_t)r * H + h] = v[h];
      v[h] = or_bf16_float(or_bf16_bits(v[h]));
    }
    if (nvfp4) {
      for (int b = 0; b < H / 16; ++b)
        nvfp4_act_block(v + b * 16, g, q + ((size_t)r * H / 16 + b) * 8, sf + (size_t)r * H / 16 + b);
    } else {
      for (int h = 0; h < H; ++h) q[(size_t)r * H + h] = or_e4m3_encode(v[h] * g);
    }
  }
  free(v);
}

/* gated_rmsnorm_fp8 (reference gated_norm_fp8_kernel, prefill_gemm.cu:461-482, 648-653): per row of 128,
 * lane l of 32 holds x[4l..4l+3] and forms fma(x3, x3, fma(x2, x2, fma(x1, x1, x0 * x0))); the 32 partial sums are
 * combined by the xor butterfly (distances 16, 8, 4, 2, 1: after the step at distance o, s[l] = s[l] + s[l ^ o],
 * the same FP32 value in both lanes); rstd = 1 / sqrtf(ss / 128 + eps); v = bf16(x * rstd * w * silu(z)) (products
 * left to right); q = E4M3_satfinite(v * (1 / input_scale)). The BF16-input form widens x and z exactly first. */
void or_gated_rmsnorm_fp8(const float* x, const float* z, const uint16_t* w, int rows, float eps, float input_scale,
                          uint8_t* q) {
  const float g = 1.f / input_scale;
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + (size_t)r * 128;
    const float* zr = z + (size_t)r * 128;
    float s[32];
    for (int l = 0; l < 32; ++l) {
      float t = xr[4 * l] * xr[4 * l];
      t = fmaf(xr[4 * l + 1], xr[4 * l + 1], t);
      t = fmaf(xr[4 * l + 2], xr[4 * l + 2], t);
      s[l] = fmaf(xr[4 * l + 3], xr[4 * l + 3], t);
    }
    for (int o = 16; o > 0; o >>= 1) {
      float t[32];
      for (int l = 0; l < 32; ++l) t[l] = s[l] + s[l ^ o];
      memcpy(s, t, sizeof t);
    }
    const float rstd = 1.f / sqrtf(s[0] / 128.f + eps);
    for (int h = 0; h < 128; ++h) {
      const float v = or_bf16_float(or_bf16_bits(xr[h] * rstd * or_bf16_float(w[h]) * or_silu(zr[h])));
      q[(size_t)r * 128 + h] = or_e4m3_encode(v * g);
    }
  }
}

/* sigmoid_mul_fp8 (reference sigmoid_mul_fp8_kernel, prefill_gemm.cu:484-494, 662-665):
 * q[i] = E4M3_satfinite(bf16(x[i] / (1 + expf(-gate[i]))) * (1 / input_scale)). */
void or_sigmoid_mul_fp8(const float* x, const float* gate, size_t n, float input_scale, uint8_t* q) {
  const float g = 1.f / input_scale;
  for (size_t i = 0; i < n; ++i) q[i] = or_e4m3_encode(or_bf16_float(or_bf16_bits(x[i] / (1.f + expf(-gate[i])))) * g);
}

/* ------------------------------------------------------------------------------------------------ */
/* reference GEMM                                                                                     */
/* ------------------------------------------------------------------------------------------------ */

int or_hardware_threads(void) {
  const long n = sysconf(_SC_NPROCESSORS_ONLN);
  return n > 0 ? (int)n : 1;
}

typedef void (*range_fn)(void* ctx, int lo, int hi);
typedef struct { range_fn fn; void* ctx; int lo, hi; } range_job;

static void* range_thread(void* p) {
  range_job* j = (range_job*)p;
  j->fn(j->ctx, j->lo, j->hi);
  return NULL;
}

/* Runs fn over [0, n) split in contiguous ranges across `threads` threads (0: all cores). */
static void parallel_for(int n, int threads, range_fn fn, void* ctx) {
  if (threads <= 0) threads = or_hardware_threads();
  if (threads > n) threads = n > 0 ? n : 1;
  if (threads > 256) threads = 256;
  pthread_t tid[256];
  range_job job[256];
  for (int t = 0; t < threads; ++t) {
    job[t].fn = fn;
    job[t].ctx = ctx;
    job[t].lo = (int)((long long)n * t / threads);
    job[t].hi = (int)((long long)n * (t + 1) / threads);
  }
  for (int t = 1; t < threads; ++t) pthread_create(&tid[t], NULL, range_thread, &job[t]);
  range_thread(&job[0]);
  for (int t = 1; t < threads; ++t) pthread_join(tid[t], NULL);
}

typedef struct { const float* x; const float* w; int M, N, K; float* y; } gemm_ctx;

static void gemm_range(void* p, int n0, int n1) {
  const gemm_ctx* c = (const gemm_ctx*)p;
  for (int n = n0; n < n1; ++n) {
    const float* wr = c->w + (size_t)n * c->K;
    for (int m = 0; m < c->M; ++m) {
      const float* xr = c->x + (size_t)m * c->K;
      float acc = 0.f;
      for (int k = 0; k < c->K; ++k) acc += xr[k] * wr[k];
      c->y[(size_t)m * c->N + n] = acc;
    }
  }
}

void or_gemm_f32(const float* x, const float* wdeq, int M, int N, int K, float* y, int threads) {
  gemm_ctx c = {x, wdeq, M, N, K, y};
  parallel_for(N, threads, gemm_range, &c);
}

float or_silu(float v) { return v / (1.f + expf(-v)); }

void or_epi_bf16(const float* acc, size_t n, uint16_t* out) {
  for (size_t i = 0; i < n; ++i) out[i] = or_bf16_bits(acc[i]);
}

void or_epi_silu_mul_bf16(const float* g, const float* u, size_t n, uint16_t* out) {
  for (size_t i = 0; i < n; ++i) out[i] = or_bf16_bits(or_silu(g[i]) * u[i]);
}

void or_epi_residual_bf16(const float* acc, const uint16_t* resid, size_t n, uint16_t* out) {
  for (size_t i = 0; i < n; ++i) out[i] = or_bf16_bits(acc[i] + or_bf16_float(resid[i]));
}

/* The whole CPU path for FP8 per-channel weights: each thread dequantizes its output channels' rows to FP32
 * (e4m3 * s_n) and accumulates x . w in FP32, k ascending; the result is rounded to BF16. */
typedef struct {
  const uint16_t* x;
  const float* xf; /* x in FP32 [M][K] */
  int M;
  const uint8_t* q;
  const float* scale;
  int N, K, n0;
  uint16_t* y;
} stream_ctx;

static void stream_range(void* p, int lo, int hi) {
  const stream_ctx* c = (const stream_ctx*)p;
  float* wr = (float*)malloc(sizeof(float) * (size_t)c->K);
  for (int i = lo; i < hi; ++i) {
    const int n = c->n0 + i;
    for (int k = 0; k < c->K; ++k) wr[k] = or_e4m3_decode(c->q[(size_t)n * c->K + k]) * c->scale[n];
    for (int m = 0; m < c->M; ++m) {
      const float* xr = c->xf + (size_t)m * c->K;
      float acc = 0.f;
      for (int k = 0; k < c->K; ++k) acc += xr[k] * wr[k];
      c->y[(size_t)m * c->N + n] = or_bf16_bits(acc);
    }
  }
  free(wr);
}

void or_stream_fp8_pc_bf16(const uint16_t* x, int M, const uint8_t* q, const float* scale, int N, int K, int n0,
                           int n1, uint16_t* y, int threads) {
  float* xf = (float*)malloc(sizeof(float) * (size_t)M * K);
  for (size_t i = 0; i < (size_t)M * K; ++i) xf[i] = or_bf16_float(x[i]);
  stream_ctx c = {x, xf, M, q, scale, N, K, n0, y};
  parallel_for(n1 - n0, threads, stream_range, &c);
  free(xf);
}

typedef struct {
  const uint8_t* xq;
  const float* xs;
  const int* rows;
  int R;
  const uint8_t* wq;
  const float* ws;
  int N, K;
  float* y;
} prefill_ctx;

/* Dequantize to FP32 on both sides (e4m3 * block scale) and accumulate in FP32, k ascending. */
static void prefill_range(void* p, int lo, int hi) {
  const prefill_ctx* c = (const prefill_ctx*)p;
  const int K = c->K, KB = K / 128;
  float* wr = (float*)malloc(sizeof(float) * (size_t)K);
  float* xr = (float*)malloc(sizeof(float) * (size_t)K * c->R);
  for (int r = 0; r < c->R; ++r) {
    const int m = c->rows[r];
    for (int k = 0; k < K; ++k)
      xr[(size_t)r * K + k] = or_e4m3_decode(c->xq[(size_t)m * K + k]) * c->xs[(size_t)m * KB + k / 128];
  }
  for (int n = lo; n < hi; ++n) {
    for (int k = 0; k < K; ++k) wr[k] = or_e4m3_decode(c->wq[(size_t)n * K + k]) * c->ws[(size_t)(n / 128) * KB + k / 128];
    for (int r = 0; r < c->R; ++r) {
      const float* x = xr + (size_t)r * K;
      float acc = 0.f;
      for (int k = 0; k < K; ++k) acc += x[k] * wr[k];
      c->y[(size_t)r * c->N + n] = acc;
    }
  }
  free(wr);
  free(xr);
}

void or_prefill_fp8_rows(const uint8_t* xq, const float* xs, const int* rows, int R, const uint8_t* wq,
                         const float* ws, int N, int K, float* y, int threads) {
  prefill_ctx c = {xq, xs, rows, R, wq, ws, N, K, y};
  parallel_for(N, threads, prefill_range, &c);
}
