// Exact small integer division by a float reciprocal, for code on both sides (device kernels, host tests).
#pragma once

#if defined(__HIPCC__)
#define LQ_HOST_DEVICE __host__ __device__
#else
#define LQ_HOST_DEVICE
#endif

namespace lq {

// floor(n / d) for n >= 0, d > 0, n + d < 2^31 and a quotient below 2^21, from rd = 1.f / d: the float
// estimate n * rd is within 3 * 2^-24 relative of n / d, so within 0.4 of it, and its truncation is the quotient
// or one off; one step each way corrects it. Eight instructions where an integer division takes about 35.
LQ_HOST_DEVICE inline int div_by_rcp(int n, int d, float rd) {
  int q = static_cast<int>(static_cast<float>(n) * rd);
  if (q * d > n)
    --q;
  else if ((q + 1) * d <= n)
    ++q;
  return q;
}

}  // namespace lq
