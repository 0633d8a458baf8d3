// Fused per-head stage of the Bonsai layer, between the q/k/v projections and the attention:
//   q, k <- head RMSNorm (gain qng / kng)              reference_bonsai.py:286-297 (_head_rmsnorm)
//   q, k <- NeoX RoPE at the row's position            rope_v2.py:92-117, guard rope.py:26-39
//   cache <- (k, v) at that position (int32 storage guarded)
// One 64-lane workgroup per (row, head); lane j owns the rotation pair (j, j + hd/2). The per-head RMSNorm
// follows the whole-row kernel's exact arithmetic (shared helpers); the RoPE envelope
// 2 * max|x| * max|cos, sin| <= INT64_MAX is evaluated over the whole q (and k) tensor through atomic maxima in
// `guard` (q: [0], [1]; k: [2], [3]) and checked by the attention's final kernel.
#include "imie_common.h"
#include "imie_kernels.h"
#include "imie_fixed.h"

namespace {

using namespace imie_fx;

__device__ inline void amax_u64(uint64_t* p, uint64_t v) { atomicMax((unsigned long long*)p, (unsigned long long)v); }

template <typename KT>
__global__ __launch_bounds__(64) void qk_head_kernel(QkHeadArgs a) {
  const int64_t r = blockIdx.x, h = blockIdx.y;
  const bool isq = h < a.H;
  const int64_t half = a.hd / 2;
  const int j = threadIdx.x;
  const bool act = j < half;
  const int64_t* src = isq ? a.q + (r * a.H + h) * a.hd : a.k + (r * a.Hkv + (h - a.H)) * a.hd;
  const int64_t* gain = isq ? a.qng : a.kng;
  const int64_t x0 = act ? src[j] : 0, x1 = act ? src[j + half] : 0;
  const int64_t g0 = act ? gain[j] : 0, g1 = act ? gain[j + half] : 0;
  // 128-bit sum of squares (two squares per lane cannot overflow 128 bits)
  uint64_t hi, lo;
  {
    const uint64_t a0 = imie_absu64(x0), a1 = imie_absu64(x1);
    const u128 sq = (u128)a0 * a0 + (u128)a1 * a1;
    hi = (uint64_t)(sq >> 64);
    lo = (uint64_t)sq;
  }
  int bad = 0;
  wave_sum_u128(hi, lo, bad);
  uint64_t rms = 0;
  if (!bad) {
    const u128 mean = div_u128_cols(((u128)hi << 64) | lo, (uint32_t)a.hd);
    if (mean <= ~(u128)0 - (u128)(uint64_t)a.eps) rms = isqrt_u128(mean + (u128)(uint64_t)a.eps);
  }
  if (rms == 0) {
    if (j == 0) atomicOr(a.status, IMIE_ERMS);
    return;
  }
  const uint64_t rinv = recip_u64(rms);
  bool f0 = true, f1 = true;
  const int64_t n0 = act ? norm_elem(x0, a.frac, rms, rinv, &f0) : 0;
  const int64_t n1 = act ? norm_elem(x1, a.frac, rms, rinv, &f1) : 0;
  int ok = (f0 && f1) ? 1 : 0;
  uint64_t mxn = imie_absu64(n0) > imie_absu64(n1) ? imie_absu64(n0) : imie_absu64(n1);
  uint64_t mxg = imie_absu64(g0) > imie_absu64(g1) ? imie_absu64(g0) : imie_absu64(g1);
  mxn = imie_wave_max_u64(mxn);
  mxg = imie_wave_max_u64(mxg);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ok &= __shfl_xor(ok, o, 64);
  if (!ok || (mxn != 0 && mxg > (uint64_t)INT64_MAX / mxn)) {
    if (j == 0) atomicOr(a.status, IMIE_ERMS);
    return;
  }
  const int64_t y0 = imie_floor_shift((int64_t)((uint64_t)n0 * (uint64_t)g0), a.frac);
  const int64_t y1 = imie_floor_shift((int64_t)((uint64_t)n1 * (uint64_t)g1), a.frac);
  const int64_t p = a.pos[r];
  const int64_t c = act ? a.cos[p * half + j] : 0, s = act ? a.sin[p * half + j] : 0;
  const int64_t o0 = (int64_t)((uint64_t)y0 * (uint64_t)c - (uint64_t)y1 * (uint64_t)s) >> a.frac;
  const int64_t o1 = (int64_t)((uint64_t)y0 * (uint64_t)s + (uint64_t)y1 * (uint64_t)c) >> a.frac;
  {
    uint64_t mx = imie_absu64(y0) > imie_absu64(y1) ? imie_absu64(y0) : imie_absu64(y1);
    uint64_t mc = imie_absu64(c) > imie_absu64(s) ? imie_absu64(c) : imie_absu64(s);
    mx = imie_wave_max_u64(mx);
    mc = imie_wave_max_u64(mc);
    if (j == 0) {
      amax_u64(&a.guard[isq ? 0 : 2], mx);
      amax_u64(&a.guard[isq ? 1 : 3], mc);
    }
  }
  if (isq) {
    if (act) {
      a.qo[(r * a.H + h) * a.hd + j] = o0;
      a.qo[(r * a.H + h) * a.hd + j + half] = o1;
    }
    return;
  }
  const int64_t kvh = h - a.H, b = r / a.M;
  const uint32_t pq = (uint32_t)p / (uint32_t)a.P;              // positions are below 2^31
  const int64_t off = a.pt[b * a.mp + pq] * (a.Hkv * a.P * a.hd) + kvh * a.P * a.hd + ((uint32_t)p - pq * (uint32_t)a.P) * a.hd;
  const int64_t* vr = a.v + (r * a.Hkv + kvh) * a.hd;
  const int64_t v0 = act ? vr[j] : 0, v1 = act ? vr[j + half] : 0;
  if (!act) return;
  if (sizeof(KT) == 4) {
    if (o0 != (int64_t)(int32_t)o0 || o1 != (int64_t)(int32_t)o1 || v0 != (int64_t)(int32_t)v0 ||
        v1 != (int64_t)(int32_t)v1)
      atomicOr(a.status, IMIE_EOVF);
  }
  KT* kp = (KT*)a.kpool + off;
  KT* vp = (KT*)a.vpool + off;
  kp[j] = (KT)o0;
  kp[j + half] = (KT)o1;
  vp[j] = (KT)v0;
  vp[j + half] = (KT)v1;
}

}  // namespace

int imie_qk_head_launch(const QkHeadArgs& a, int kv32, hipStream_t st) {
  const int64_t rows = a.rows;
  if (rows <= 0) return IMIE_OK;
  if (a.hd > 128 || (a.hd & 1) || a.hd <= 0) return IMIE_EARG;
  const dim3 grid((unsigned)rows, (unsigned)(a.H + a.Hkv));
  if (kv32) hipLaunchKernelGGL(qk_head_kernel<int32_t>, grid, dim3(64), 0, st, a);
  else hipLaunchKernelGGL(qk_head_kernel<int64_t>, grid, dim3(64), 0, st, a);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}
