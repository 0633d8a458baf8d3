// Integer RMSNorm for gfx950 (reference semantics: bonsai/src/trinote/determinism/fixedpoint.py:31-71 and the
// C producer bonsai/tools/bonsai_q1_kernel.c:238-323):
//   ssq = sum x^2 (exact, 128-bit), rms = isqrt(ssq // cols + eps), n = floor((x << frac) / rms),
//   y = (n * gain) >> frac, refused (status bit 4) when ssq needs more than 128 bits, rms == 0, or
//   max|n| * max|gain| > INT64_MAX (the oracle's fail-loud gain envelope, checked per row = globally).
// One workgroup per row; the 128-bit sum is reduced by wave shuffles and LDS, the isqrt / mean run on one lane.
#include "imie_common.h"
#include "imie_kernels.h"

namespace {

typedef unsigned __int128 u128;

__device__ inline u128 div_u128_u32(u128 v, uint32_t d) {
  const uint64_t hi = (uint64_t)(v >> 64), lo = (uint64_t)v;
  const uint64_t qh = hi / d, r0 = hi % d;
  const uint64_t mid = (r0 << 32) | (lo >> 32);
  const uint64_t qm = mid / d, r1 = mid % d;
  const uint64_t low = (r1 << 32) | (lo & 0xFFFFFFFFu);
  const uint64_t ql = low / d;
  return ((u128)qh << 64) | ((u128)qm << 32) | (u128)ql;
}

// floor(sqrt(v)) for v < 2^128: a double-precision estimate narrowed by an exact integer binary search over
// [est - 2^12, est + 2^12] (the estimate is within ~2^-52 * 2^64 of the root); full 64-step search otherwise.
__device__ inline uint64_t isqrt_u128(u128 v) {
  const double fv = (double)(uint64_t)(v >> 64) * 18446744073709551616.0 + (double)(uint64_t)v;
  double fe = sqrt(fv);
  uint64_t est = fe >= 18446744073709549568.0 ? ~(uint64_t)0 : (uint64_t)fe;
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

// One workgroup (nt threads, 64..1024) per row; per-thread partials reduced by wave shuffles, then across the
// waves through LDS. Rows of up to 4 * nt columns are loaded once and kept in registers (x and gain); longer rows
// are re-read. Steps: (1) 128-bit sum of squares; (2) n = floor((x << f) / rms) with max|n| and max|gain| for
// the envelope; (3) y = (n * gain) >> f.
constexpr int kNormPer = 4;

__global__ __launch_bounds__(1024) void rmsnorm_kernel(const int64_t* __restrict__ x, int64_t cols, int frac,
                                                        int64_t eps, const int64_t* __restrict__ gain,
                                                        int64_t* __restrict__ out, int* __restrict__ status) {
  __shared__ uint64_t s_hi[16], s_lo[16], s_mn[16], s_mg[16];
  __shared__ int s_bad[16];
  __shared__ uint64_t s_rms, s_rinv;
  __shared__ int s_ok;
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, nt = blockDim.x, lane = tid & 63, wave = tid >> 6, nw = nt >> 6;
  const int64_t* xr = x + row * cols;
  const bool cached = cols <= (int64_t)kNormPer * nt;
  int64_t xv[kNormPer], gv[kNormPer];
  if (cached) {
#pragma unroll
    for (int k = 0; k < kNormPer; ++k) {
      const int64_t c = tid + (int64_t)k * nt;
      xv[k] = c < cols ? xr[c] : 0;
      gv[k] = (gain && c < cols) ? gain[c] : 0;
    }
  }
  uint64_t hi = 0, lo = 0;
  int bad = 0;
  auto add_sq = [&](int64_t v) {
    const uint64_t a = imie_absu64(v);
    const u128 sq = (u128)a * a;
    const uint64_t sl = (uint64_t)sq, sh = (uint64_t)(sq >> 64);
    const uint64_t nl = lo + sl;
    const uint64_t cy = nl < lo ? 1 : 0;
    const uint64_t nh = hi + sh;
    bad |= (nh < hi ? 1 : 0) | (nh + cy < nh ? 1 : 0);
    hi = nh + cy;
    lo = nl;
  };
  if (cached) {
#pragma unroll
    for (int k = 0; k < kNormPer; ++k) add_sq(xv[k]);
  } else {
    for (int64_t c = tid; c < cols; c += nt) add_sq(xr[c]);
  }
  wave_sum_u128(hi, lo, bad);
  if (lane == 0) { s_hi[wave] = hi; s_lo[wave] = lo; s_bad[wave] = bad; }
  __syncthreads();
  if (tid == 0) {
    uint64_t H = 0, Lo = 0;
    int B = 0;
    for (int w = 0; w < nw; ++w) {
      const uint64_t nl = Lo + s_lo[w];
      const uint64_t cy = nl < Lo ? 1 : 0;
      const uint64_t nh = H + s_hi[w];
      B |= s_bad[w] | (nh < H ? 1 : 0) | (nh + cy < nh ? 1 : 0);
      H = nh + cy;
      Lo = nl;
    }
    uint64_t rms = 0;
    if (!B) {
      const u128 mean = div_u128_u32(((u128)H << 64) | Lo, (uint32_t)cols);
      if (mean <= ~(u128)0 - (u128)(uint64_t)eps) rms = isqrt_u128(mean + (u128)(uint64_t)eps);
    }
    s_rms = rms;
    s_rinv = rms ? (~(uint64_t)0) / rms : 0;
    if (rms == 0) atomicOr(status, IMIE_ERMS);
  }
  __syncthreads();
  const uint64_t rms = s_rms, rinv = s_rinv;
  if (rms == 0) return;
  uint64_t mxn = 0, mxg = 0;
  int nfit = 1;
  int64_t nvk[kNormPer];
  auto norm1 = [&](int64_t v, int64_t g, int64_t c, int64_t* keep) {
    bool fits;
    const int64_t nv = norm_elem(v, frac, rms, rinv, &fits);
    nfit &= fits ? 1 : 0;
    const uint64_t an = imie_absu64(nv);
    mxn = an > mxn ? an : mxn;
    if (gain) {
      const uint64_t ag = imie_absu64(g);
      mxg = ag > mxg ? ag : mxg;
    } else {
      out[row * cols + c] = nv;
    }
    if (keep) *keep = nv;
  };
  if (cached) {
#pragma unroll
    for (int k = 0; k < kNormPer; ++k) {
      const int64_t c = tid + (int64_t)k * nt;
      if (c < cols) norm1(xv[k], gv[k], c, &nvk[k]);
    }
  } else {
    for (int64_t c = tid; c < cols; c += nt) norm1(xr[c], gain ? gain[c] : 0, c, nullptr);
  }
  if (!gain) {
    if (!nfit) atomicOr(status, IMIE_ERMS);
    return;
  }
  mxn = imie_wave_max_u64(mxn);
  mxg = imie_wave_max_u64(mxg);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) nfit &= __shfl_xor(nfit, o, 64);
  if (lane == 0) { s_mn[wave] = mxn; s_mg[wave] = mxg; s_bad[wave] = nfit; }
  __syncthreads();
  if (tid == 0) {
    uint64_t mn = 0, mg = 0;
    int ok = 1;
    for (int w = 0; w < nw; ++w) {
      mn = s_mn[w] > mn ? s_mn[w] : mn;
      mg = s_mg[w] > mg ? s_mg[w] : mg;
      ok &= s_bad[w];
    }
    if (ok && mn != 0 && mg > (uint64_t)INT64_MAX / mn) ok = 0;
    if (!ok) atomicOr(status, IMIE_ERMS);
    s_ok = ok;
  }
  __syncthreads();
  if (!s_ok) return;
  if (cached) {
#pragma unroll
    for (int k = 0; k < kNormPer; ++k) {
      const int64_t c = tid + (int64_t)k * nt;
      if (c < cols) out[row * cols + c] = imie_floor_shift((int64_t)((uint64_t)nvk[k] * (uint64_t)gv[k]), frac);
    }
  } else {
    for (int64_t c = tid; c < cols; c += nt) {
      bool fits;
      const int64_t nv = norm_elem(xr[c], frac, rms, rinv, &fits);
      out[row * cols + c] = imie_floor_shift((int64_t)((uint64_t)nv * (uint64_t)gain[c]), frac);
    }
  }
}

}  // namespace

int imie_rmsnorm_launch(const int64_t* x, int64_t rows, int64_t cols, int64_t frac, int64_t eps,
                        const int64_t* gain, int64_t* out, int* status, hipStream_t st) {
  if (rows <= 0) return IMIE_OK;
  // one thread per 4 columns up to 1024 threads; at least one wave
  int nt = (int)((cols + 3) / 4);
  nt = nt < 64 ? 64 : (nt > 1024 ? 1024 : ((nt + 63) / 64) * 64);
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(nt), 0, st, x, cols, (int)frac, eps, gain, out,
                     status);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

namespace {
struct NormWs {
  DevBuf x, out, gain, status;
} g_nws;
}  // namespace

extern "C" {

// bonsai_q1_gpu.cu:625-670 / gpu_native.py:390-415 `bonsai_rmsnorm_gpu`: host in/out, synchronous, rc 4 on the
// 128-bit or gain envelope.
int bonsai_rmsnorm_gpu(const int64_t* x, int64_t rows, int64_t cols, int64_t frac, int64_t eps, const int64_t* gain,
                       int64_t* out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!x || !out || rows < 0 || cols <= 0 || cols > 0xFFFFFFFFll || frac < 0 || frac > 62 || eps < 0) return IMIE_EARG;
  if (rows == 0) return IMIE_OK;
  if (imie_device_ready() != 0) return IMIE_EARG;
  hipStream_t st = imie_stream();
  const size_t xb = (size_t)(rows * cols) * 8;
  if (g_nws.x.ensure(xb) || g_nws.out.ensure(xb) || g_nws.gain.ensure((size_t)cols * 8) || g_nws.status.ensure(64))
    return IMIE_EARG;
  IMIE_HIP(hipMemcpyAsync(g_nws.x.p, x, xb, hipMemcpyHostToDevice, st));
  if (gain) IMIE_HIP(hipMemcpyAsync(g_nws.gain.p, gain, (size_t)cols * 8, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemsetAsync(g_nws.status.p, 0, 4, st));
  int rc = imie_rmsnorm_launch((const int64_t*)g_nws.x.p, rows, cols, frac, eps,
                               gain ? (const int64_t*)g_nws.gain.p : nullptr, (int64_t*)g_nws.out.p,
                               (int*)g_nws.status.p, st);
  if (rc) return rc;
  int stat = 0;
  IMIE_HIP(hipMemcpyAsync(&stat, g_nws.status.p, 4, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipMemcpyAsync(out, g_nws.out.p, xb, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipStreamSynchronize(st));
  return stat ? IMIE_ERMS : IMIE_OK;
}

// Device-pointer RMSNorm; status (device int) receives bit 4 on refusal. Asynchronous on `stream`.
int imie_rmsnorm_dev(const int64_t* x, int64_t rows, int64_t cols, int64_t frac, int64_t eps, const int64_t* gain,
                     int64_t* out, int* status, void* stream) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!x || !out || !status || rows < 0 || cols <= 0 || cols > 0xFFFFFFFFll || frac < 0 || frac > 62 || eps < 0)
    return IMIE_EARG;
  return imie_rmsnorm_launch(x, rows, cols, frac, eps, gain, out, status, (hipStream_t)stream);
}

}  // extern "C"
