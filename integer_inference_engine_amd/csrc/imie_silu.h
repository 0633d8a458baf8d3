// Fixed-point SiLU pieces shared by the element-wise kernels and the matvec prologue (reference semantics:
// fixedpoint.py:143-174 over reference_bonsai.py:245-264): exp2(-u) by the cubic on the fraction and a shift by the
// integer part, sigmoid as e1 / (e0 + e1) with both arguments clipped at dclip.
#pragma once
#include "imie_common.h"

namespace imie_silu {

__host__ __device__ inline int64_t rshift_np(int64_t a, int64_t s) {   // numpy int64 `a >> s` incl. out-of-range counts
  if (s < 0 || s >= 64) return a < 0 ? -1 : 0;
  return a >> s;
}

__host__ __device__ inline int64_t exp2_neg_fixed(int64_t u, int frac) {
  const int64_t fp = (int64_t)1 << frac;
  const int64_t k = u >> frac, f = u & (fp - 1);
  const int sh = 16 - frac;
  int64_t c0, c1, c2, c3;
  if (sh >= 0) { c0 = 65536 >> sh; c1 = 45426 >> sh; c2 = 15743 >> sh; c3 = 3638 >> sh; }
  else { c0 = (int64_t)65536 << -sh; c1 = (int64_t)45426 << -sh; c2 = (int64_t)15743 << -sh; c3 = (int64_t)3638 << -sh; }
  const int64_t f2 = (int64_t)((uint64_t)f * (uint64_t)f) >> frac;
  const int64_t f3 = (int64_t)((uint64_t)f2 * (uint64_t)f) >> frac;
  int64_t poly = c0 - ((int64_t)((uint64_t)c1 * (uint64_t)f) >> frac) + ((int64_t)((uint64_t)c2 * (uint64_t)f2) >> frac) -
                 ((int64_t)((uint64_t)c3 * (uint64_t)f3) >> frac);
  if (poly < 0) poly = 0;
  return rshift_np(poly, k < 63 ? k : 63);
}

__host__ __device__ inline int64_t sigmoid_fixed(int64_t x, int frac, int64_t log2e, int64_t dclip) {
  const int64_t m = x > 0 ? x : 0;
  int64_t d0 = m, d1 = (int64_t)((uint64_t)m - (uint64_t)x);
  if (d0 > dclip) d0 = dclip;
  if (d1 > dclip) d1 = dclip;
  const int64_t e0 = exp2_neg_fixed((int64_t)((uint64_t)d0 * (uint64_t)log2e) >> frac, frac);
  const int64_t e1 = exp2_neg_fixed((int64_t)((uint64_t)d1 * (uint64_t)log2e) >> frac, frac);
  const int64_t z = e0 + e1;
  if (z == 0) return 0;
  const uint64_t num = (uint64_t)e1 << frac;               // e1 << frac >= 0 and fits (e1 <= c0 + c2)
  if (num < ((uint64_t)1 << 52)) {                         // exact double quotient estimate, +-1 integer fix
    uint64_t q = (uint64_t)((double)num / (double)z);
    if (q * (uint64_t)z > num) --q;
    else if (num - q * (uint64_t)z >= (uint64_t)z) ++q;
    return (int64_t)q;
  }
  return (int64_t)(num / (uint64_t)z);
}

// exp2_neg_fixed for frac <= 29 and 0 <= u: every product of the cubic is below 2^58 with both factors below
// 2^32 (f, f2, f3 < 2^frac, the coefficients < 2^29), so each is one 32 x 32 -> 64 multiply
__host__ __device__ inline int64_t exp2_neg_fixed32(int64_t u, int frac) {
  const int64_t fp = (int64_t)1 << frac;
  const int64_t k = u >> frac;
  const uint32_t f = (uint32_t)(u & (fp - 1));
  const int sh = 16 - frac;
  uint32_t c0, c1, c2, c3;
  if (sh >= 0) { c0 = 65536u >> sh; c1 = 45426u >> sh; c2 = 15743u >> sh; c3 = 3638u >> sh; }
  else { c0 = 65536u << -sh; c1 = 45426u << -sh; c2 = 15743u << -sh; c3 = 3638u << -sh; }
  const uint32_t f2 = (uint32_t)(((uint64_t)f * f) >> frac);
  const uint32_t f3 = (uint32_t)(((uint64_t)f2 * f) >> frac);
  int64_t poly = (int64_t)c0 - (int64_t)(((uint64_t)c1 * f) >> frac) + (int64_t)(((uint64_t)c2 * f2) >> frac) -
                 (int64_t)(((uint64_t)c3 * f3) >> frac);
  if (poly < 0) poly = 0;
  return rshift_np(poly, k < 63 ? k : 63);
}

// sigmoid_fixed with one exponential: of the two clipped exponents one is 0 (x > 0: (min(x, dclip), 0); x <= 0:
// (0, min(-x, dclip))) and exp2(-0) = c0 = 2^frac. Taken when frac <= 29, dclip and log2e are below 2^32 (so
// d * log2e is one 32 x 32 product, below 2^62 by the clip) and x != INT64_MIN (whose negation wraps);
// otherwise the two-exponential form.
__host__ __device__ inline int64_t sigmoid_fixed_fast(int64_t x, int frac, int64_t log2e, int64_t dclip) {
  if (frac > 29 || (dclip >> 32) != 0 || (log2e >> 32) != 0 || x == INT64_MIN)
    return sigmoid_fixed(x, frac, log2e, dclip);
  int64_t d = x > 0 ? x : -x;
  if (d > dclip) d = dclip;
  const int64_t e = exp2_neg_fixed32((int64_t)(((uint64_t)(uint32_t)d * (uint32_t)log2e) >> frac), frac);
  const int64_t c0 = (int64_t)1 << frac;
  const int64_t e0 = x > 0 ? e : c0, e1 = x > 0 ? c0 : e;
  const int64_t z = e0 + e1;
  if (z == 0) return 0;
  const uint64_t num = (uint64_t)e1 << frac;
  if (num < ((uint64_t)1 << 52)) {
    uint64_t q = (uint64_t)((double)num / (double)z);
    if (q * (uint64_t)z > num) --q;
    else if (num - q * (uint64_t)z >= (uint64_t)z) ++q;
    return (int64_t)q;
  }
  return (int64_t)(num / (uint64_t)z);
}

// silu_mul through sigmoid_fixed_fast (the same values)
__host__ __device__ inline int64_t silu_mul_fast(int64_t g, int64_t u, int frac, int64_t log2e, int64_t dclip) {
  const int64_t silu = (int64_t)((uint64_t)g * (uint64_t)sigmoid_fixed_fast(g, frac, log2e, dclip)) >> frac;
  return (int64_t)((uint64_t)silu * (uint64_t)u) >> frac;
}

// exp2_neg_fixed((d * log2e) >> frac) of a clipped softmax difference d (0 <= d <= dclip): one 32 x 32 product and
// the 32-bit cubic when dclip and log2e are below 2^32 (fast, decided once per launch; frac <= 29), else the
// general form. Same values.
__host__ __device__ inline int64_t exp_clipped(int64_t d, int frac, int64_t log2e, bool fast) {
  if (fast && d >= 0)
    return exp2_neg_fixed32((int64_t)(((uint64_t)(uint32_t)d * (uint32_t)log2e) >> frac), frac);
  return exp2_neg_fixed((int64_t)((uint64_t)d * (uint64_t)log2e) >> frac, frac);
}

// p = floor((e << frac) / z) for 0 <= e, 0 < z: below 2^52 (numerator and z) the double quotient num * (1 / z)
// is within one of the answer and the exact remainder settles it; otherwise the integer division.
__host__ __device__ inline int64_t prob_div(int64_t e, int frac, uint64_t z, double rz) {
  const uint64_t num = (uint64_t)e << frac;
  if ((num >> 52) == 0 && (z >> 52) == 0) {
    uint64_t q = (uint64_t)((double)num * rz);
    const int64_t r = (int64_t)(num - q * z);
    if (r < 0) --q;
    else if ((uint64_t)r >= z) ++q;
    return (int64_t)q;
  }
  return (int64_t)(num / z);
}

// (silu(g) * u) >> frac with silu(g) = (g * sigmoid(g)) >> frac (wrapping int64 products, as the reference)
__host__ __device__ inline int64_t silu_mul(int64_t g, int64_t u, int frac, int64_t log2e, int64_t dclip) {
  const int64_t silu = (int64_t)((uint64_t)g * (uint64_t)sigmoid_fixed(g, frac, log2e, dclip)) >> frac;
  return (int64_t)((uint64_t)silu * (uint64_t)u) >> frac;
}

}  // namespace imie_silu
