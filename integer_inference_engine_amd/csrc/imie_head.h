// Per-head stage arithmetic shared by the head kernel and the single-token decode attention (reference semantics:
// reference_bonsai.py:286-297 head RMSNorm over fixedpoint.py:31-71, then the NeoX RoPE of rope_v2.py:92-117).
#pragma once
#include "imie_common.h"
#include "imie_fixed.h"

namespace imie_head {

// One head on one full wave: lane j holds the rotation pair (x0, x1) = (x[j], x[j + hd/2]) with gains (g0, g1)
// and the position's (c, s) (act: j < hd/2; idle lanes hold zeros). On success o0, o1 are the rotated values and
// mx_y / mx_cs the wave's max|y| and max|cos, sin| for the RoPE envelope; false = refused (rms == 0, an n
// outside int64, or max|n| * max|gain| beyond int64), where the head stage raises the RMSNorm status bit.
__device__ inline bool head_norm_rope(int64_t x0, int64_t x1, int64_t g0, int64_t g1, int64_t c, int64_t s, bool act,
                                      int64_t hd, int frac, int64_t eps, int64_t& o0, int64_t& o1, uint64_t& mx_y,
                                      uint64_t& mx_cs) {
  using namespace imie_fx;
  // 128-bit sum of squares (two squares per lane cannot overflow 128 bits); every |x| of the head below 2^26:
  // 52-bit squares, the wave's sum in one 64-bit word (one reduction instead of four limb sums)
  uint64_t hi = 0, lo = 0;
  int bad = 0;
  const uint64_t a0 = imie_absu64(x0), a1 = imie_absu64(x1);
  if (!__any(((a0 | a1) >> 26) ? 1 : 0)) {
    lo = imie_wave_sum_u64_full((uint64_t)(uint32_t)a0 * (uint32_t)a0 + (uint64_t)(uint32_t)a1 * (uint32_t)a1);
  } else {
    const u128 sq = (u128)a0 * a0 + (u128)a1 * a1;
    hi = (uint64_t)(sq >> 64);
    lo = (uint64_t)sq;
    wave_sum_u128_full(hi, lo, bad);
  }
  uint64_t rms = 0;
  if (!bad) {
    const u128 mean = div_u128_cols(((u128)hi << 64) | lo, (uint32_t)hd);
    if (mean <= ~(u128)0 - (u128)(uint64_t)eps) rms = isqrt_u128_fast(mean + (u128)(uint64_t)eps);
  }
  o0 = o1 = 0;
  mx_y = mx_cs = 0;
  if (rms == 0) return false;
  // n in double precision where exact; the integer routine (and its reciprocal) only if some lane needs it
  const double rd = (double)rms, rid = 1.0 / rd;
  int64_t n0 = 0, n1 = 0;
  const bool q0 = !act || norm_elem_f64(x0, frac, rms, rd, rid, &n0);
  const bool q1 = !act || norm_elem_f64(x1, frac, rms, rd, rid, &n1);
  bool f0 = true, f1 = true;
  if (__any((q0 && q1) ? 0 : 1)) {
    const uint64_t rinv = recip_u64(rms);
    if (!q0) n0 = norm_elem(x0, frac, rms, rinv, &f0);
    if (!q1) n1 = norm_elem(x1, frac, rms, rinv, &f1);
  }
  const bool ok = __all((f0 && f1) ? 1 : 0) != 0;
  uint64_t mxn = imie_absu64(n0) > imie_absu64(n1) ? imie_absu64(n0) : imie_absu64(n1);
  uint64_t mxg = imie_absu64(g0) > imie_absu64(g1) ? imie_absu64(g0) : imie_absu64(g1);
  mxn = imie_wave_max_u64_full(mxn);
  mxg = imie_wave_max_u64_full(mxg);
  if (!ok || (mxn != 0 && mxg > (uint64_t)INT64_MAX / mxn)) return false;
  const int64_t y0 = imie_floor_shift((int64_t)((uint64_t)n0 * (uint64_t)g0), frac);
  const int64_t y1 = imie_floor_shift((int64_t)((uint64_t)n1 * (uint64_t)g1), frac);
  o0 = (int64_t)((uint64_t)y0 * (uint64_t)c - (uint64_t)y1 * (uint64_t)s) >> frac;
  o1 = (int64_t)((uint64_t)y0 * (uint64_t)s + (uint64_t)y1 * (uint64_t)c) >> frac;
  const uint64_t my = imie_absu64(y0) > imie_absu64(y1) ? imie_absu64(y0) : imie_absu64(y1);
  const uint64_t mc = imie_absu64(c) > imie_absu64(s) ? imie_absu64(c) : imie_absu64(s);
  mx_y = imie_wave_max_u64_full(my);
  mx_cs = imie_wave_max_u64_full(mc);
  return true;
}

}  // namespace imie_head
