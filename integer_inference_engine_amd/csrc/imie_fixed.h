// Exact fixed-point helpers shared by the RMSNorm kernels (whole-row and per-head fused forms).
// Semantics: bonsai/src/trinote/determinism/fixedpoint.py:31-71 (128-bit sum of squares, isqrt of the floor mean,
// floor division of x << frac by the rms).
#pragma once
#include "imie_common.h"

namespace imie_fx {

typedef unsigned __int128 u128;

__host__ __device__ inline u128 div_u128_u32(u128 v, uint32_t d) {
  const uint64_t hi = (uint64_t)(v >> 64), lo = (uint64_t)v;
  const uint64_t qh = hi / d, r0 = hi % d;
  const uint64_t mid = (r0 << 32) | (lo >> 32);
  const uint64_t qm = mid / d, r1 = mid % d;
  const uint64_t low = (r1 << 32) | (lo & 0xFFFFFFFFu);
  const uint64_t ql = low / d;
  return ((u128)qh << 64) | ((u128)qm << 32) | (u128)ql;
}

// floor(v / d) for a power-of-two d takes a shift; otherwise the three-step 64/32 long division
__host__ __device__ inline u128 div_u128_cols(u128 v, uint32_t d) {
  if ((d & (d - 1)) == 0) return v >> (31 - __builtin_clz(d));
  return div_u128_u32(v, d);
}

// floor(sqrt(v)) for v < 2^128. Below 2^100 the double-precision root is within 1 of the answer and two exact
// integer steps finish it; above, the estimate (within ~2^-52 * 2^64 of the root) is narrowed by an exact
// binary search over [est - 2^12, est + 2^12], with a full 64-step search as the fallback.
__host__ __device__ inline uint64_t isqrt_u128(u128 v) {
  const double fv = (double)(uint64_t)(v >> 64) * 18446744073709551616.0 + (double)(uint64_t)v;
  double fe = sqrt(fv);
  uint64_t est = fe >= 18446744073709549568.0 ? ~(uint64_t)0 : (uint64_t)fe;
  if ((v >> 100) == 0) {
    while (est > 0 && (u128)est * est > v) --est;
    while ((u128)(est + 1) * (est + 1) <= v) ++est;
    return est;
  }
  uint64_t lo = est > 4096 ? est - 4096 : 0;
  uint64_t hi = est < ~(uint64_t)0 - 4096 ? est + 4096 : ~(uint64_t)0;
  auto sq_le = [&](uint64_t c) { return (u128)c * c <= v; };
  if (!sq_le(lo) || (hi != ~(uint64_t)0 && sq_le(hi + 1))) { lo = 0; hi = ~(uint64_t)0; }
  while (lo < hi) {                                 // invariant: lo^2 <= v, answer in [lo, hi]
    const uint64_t mid = lo + (hi - lo + 1) / 2;
    if (sq_le(mid)) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// floor(sqrt(v)) with a short path below 2^52: v converts exactly, the double root is within one of the answer,
// and one integer check each way settles it (k <= 2^26, so the squares are 32 x 32 -> 64-bit products).
__host__ __device__ inline uint64_t isqrt_u128_fast(u128 v) {
  if ((v >> 52) == 0) {
    const uint64_t u = (uint64_t)v;
    uint64_t k = (uint64_t)sqrt((double)u);
    if ((uint64_t)(uint32_t)k * (uint32_t)k > u) --k;
    else if ((uint64_t)(uint32_t)(k + 1) * (uint32_t)(k + 1) <= u) ++k;
    return k;
  }
  return isqrt_u128(v);
}

// n = floor((x << frac) / rms) in double precision where that is exact to settle: |x| << frac below 2^53 and rms
// below 2^51. The quotient estimate num * (1 / rms) is within 2 of the answer; the remainder num - q * rms comes
// exactly from one fma (|r| < 4 rms < 2^53) and steers the correction. Returns false where the bounds do not hold
// (the caller takes the integer routine).
__host__ __device__ inline bool norm_elem_f64(int64_t x, int frac, uint64_t rms, double rms_d, double rinv_d,
                                              int64_t* out) {
  const uint64_t ax = imie_absu64(x);
  if (frac < 1 || frac > 52 || (ax >> (53 - frac)) != 0 || (rms >> 51) != 0) return false;
  const double num = (double)(ax << frac);
  double q = floor(num * rinv_d);
  double r = fma(-q, rms_d, num);
  while (r < 0) { q -= 1.0; r += rms_d; }
  while (r >= rms_d) { q += 1.0; r -= rms_d; }
  const uint64_t qi = (uint64_t)q;
  *out = x < 0 ? -(int64_t)(qi + (r != 0 ? 1 : 0)) : (int64_t)qi;
  return true;
}

// norm_elem_f64 without the bounds test, for callers that have established them (|x| << frac < 2^53, rms < 2^51,
// 1 <= frac <= 52): the quotient estimate is within 2, so two select-based steps each way settle it (no loop)
__device__ inline int64_t norm_elem_f64_fast(int64_t x, int frac, double rms_d, double rinv_d) {
  const uint64_t ax = imie_absu64(x);
  const double num = (double)(ax << frac);
  double q = floor(num * rinv_d);
  double r = fma(-q, rms_d, num);
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const bool lo = r < 0.0, hi = r >= rms_d;
    q += lo ? -1.0 : (hi ? 1.0 : 0.0);
    r += lo ? rms_d : (hi ? -rms_d : 0.0);
  }
  const uint64_t qi = (uint64_t)q;
  return x < 0 ? -(int64_t)(qi + (r != 0.0 ? 1 : 0)) : (int64_t)qi;
}

// floor(num / d) for |num| < 2^127 given as sign + 128-bit magnitude, d > 0 (bitwise long division; rare path)
__device__ inline int64_t floor_div_mag128(bool neg, u128 mag, uint64_t d, bool* fits) {
  u128 q = 0, r = 0;
  for (int b = 127; b >= 0; --b) {
    r = (r << 1) | ((mag >> b) & 1);
    if (r >= d) { r -= d; q |= (u128)1 << b; }
  }
  if (neg && r != 0) q += 1;
  if (!neg) { *fits = q <= (u128)INT64_MAX; return (int64_t)(uint64_t)q; }
  *fits = q <= ((u128)1 << 63);
  return (int64_t)(0 - (uint64_t)q);
}

// floor((2^64 - 1) / d) for d >= 1: a double estimate (within ~2^11), one exact remainder step, then +-1 fixes
__host__ __device__ inline uint64_t recip_u64(uint64_t d) {
  if (d <= 1) return ~(uint64_t)0;
  const u128 full = (u128)(~(uint64_t)0);
  uint64_t e = (uint64_t)(18446744073709551616.0 / (double)d);      // d >= 2: the quotient is below 2^64
  const __int128 rem = (__int128)full - (__int128)((u128)e * d);
  e = (uint64_t)((__int128)e + (__int128)((double)rem / (double)d));
  while ((u128)e * d > full) --e;
  while ((u128)(e + 1) * d <= full) ++e;
  return e;
}

// n = floor((x << frac) / rms); *fits false if the quotient leaves int64. rinv = floor((2^64 - 1) / rms): for
// num < 2^64, umulhi(num, rinv) is at most 2 below floor(num / rms), fixed by the correction loop.
__device__ inline int64_t norm_elem(int64_t x, int frac, uint64_t rms, uint64_t rinv, bool* fits) {
  const uint64_t ax = imie_absu64(x);
  const bool neg = x < 0;
  *fits = true;
  if (frac < 63 && ax < ((uint64_t)1 << (63 - frac))) {
    const uint64_t num = ax << frac;
    uint64_t q = __umul64hi(num, rinv);
    uint64_t r = num - q * rms;
    while (r >= rms) { ++q; r -= rms; }
    if (neg) return -(int64_t)(q + (r != 0));
    return (int64_t)q;
  }
  return floor_div_mag128(neg, (u128)ax << frac, rms, fits);
}

// 128-bit sums across a wave: (hi, lo) limbs with the carry folded into hi
__device__ inline void wave_sum_u128(uint64_t& hi, uint64_t& lo, int& bad) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint64_t l2 = __shfl_xor(lo, o, 64), h2 = __shfl_xor(hi, o, 64);
    const int b2 = __shfl_xor(bad, o, 64);
    const uint64_t nl = lo + l2;
    const uint64_t c = nl < lo ? 1 : 0;
    const uint64_t nh = hi + h2;
    bad |= b2 | (nh < hi ? 1 : 0) | (nh + c < nh ? 1 : 0);
    hi = nh + c;
    lo = nl;
  }
}

// 128-bit sums as four 32-bit limb sums: per lane (hi, lo) splits into limbs a[0..3] (a lane-level overflow
// adds 2^33 to a[3], which survives into the fold as an overflow); limb sums over up to 2^31 lanes stay below
// 2^64, so lanes combine without carries. fold carries the limbs back into (hi, lo) and flags sums >= 2^128.
__device__ inline void u128_limbs(uint64_t hi, uint64_t lo, int bad, uint64_t a[4]) {
  a[0] = lo & 0xFFFFFFFFull;
  a[1] = lo >> 32;
  a[2] = hi & 0xFFFFFFFFull;
  a[3] = (hi >> 32) + (bad ? (1ull << 33) : 0);
}
__device__ inline void u128_fold(const uint64_t a[4], uint64_t& hi, uint64_t& lo, int& bad) {
  const uint64_t c0 = a[0], c1 = a[1] + (c0 >> 32), c2 = a[2] + (c1 >> 32), c3 = a[3] + (c2 >> 32);
  lo = (c0 & 0xFFFFFFFFull) | (c1 << 32);
  hi = (c2 & 0xFFFFFFFFull) | (c3 << 32);
  bad = (c3 >> 32) != 0 ? 1 : 0;
}
// wave_sum_u128 over DPP moves; every lane of the wave must be active. Result is wave-uniform.
__device__ inline void wave_sum_u128_full(uint64_t& hi, uint64_t& lo, int& bad) {
  uint64_t a[4];
  u128_limbs(hi, lo, bad, a);
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = imie_wave_sum_u64_full(a[i]);
  u128_fold(a, hi, lo, bad);
}

}  // namespace imie_fx
