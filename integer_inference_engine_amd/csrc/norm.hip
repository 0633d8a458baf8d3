// Integer RMSNorm for gfx950 (reference semantics: bonsai/src/trinote/determinism/fixedpoint.py:31-71 and the
// C producer bonsai/tools/bonsai_q1_kernel.c:238-323):
//   ssq = sum x^2 (exact, 128-bit), rms = isqrt(ssq // cols + eps), n = floor((x << frac) / rms),
//   y = (n * gain) >> frac, refused (status bit 4) when ssq needs more than 128 bits, rms == 0, or
//   max|n| * max|gain| > INT64_MAX (the oracle's fail-loud gain envelope, checked per row = globally).
// One workgroup per row; the 128-bit sum is reduced through LDS, the isqrt / mean run on one lane.
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

__device__ inline uint64_t isqrt_u128(u128 v) {
  uint64_t r = 0;
  for (int b = 63; b >= 0; --b) {
    const uint64_t c = r | ((uint64_t)1 << b);
    if ((u128)c * c <= v) r = c;
  }
  return r;
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

// n = floor((x << frac) / rms); *fits false if the quotient leaves int64
__device__ inline int64_t norm_elem(int64_t x, int frac, uint64_t rms, bool* fits) {
  const uint64_t ax = imie_absu64(x);
  const bool neg = x < 0;
  *fits = true;
  if (frac < 63 && ax < ((uint64_t)1 << (63 - frac))) {
    const uint64_t num = ax << frac;
    uint64_t q = num / rms;
    const uint64_t r = num - q * rms;
    if (neg) return -(int64_t)(q + (r != 0));
    return (int64_t)q;
  }
  return floor_div_mag128(neg, (u128)ax << frac, rms, fits);
}

__global__ __launch_bounds__(256) void rmsnorm_kernel(const int64_t* __restrict__ x, int64_t cols, int frac,
                                                       int64_t eps, const int64_t* __restrict__ gain,
                                                       int64_t* __restrict__ out, int* __restrict__ status) {
  __shared__ u128 s_ssq[256];
  __shared__ int s_bad[256];
  __shared__ uint64_t s_mx[256];
  __shared__ uint64_t s_rms;
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, nt = blockDim.x;
  const int64_t* xr = x + row * cols;
  u128 ssq = 0;
  int bad = 0;
  for (int64_t c = tid; c < cols; c += nt) {
    const uint64_t a = imie_absu64(xr[c]);
    const u128 sq = (u128)a * a;
    if (ssq > ~(u128)0 - sq) bad = 1;
    ssq += sq;
  }
  s_ssq[tid] = ssq;
  s_bad[tid] = bad;
  __syncthreads();
  for (int o = nt / 2; o > 0; o >>= 1) {
    if (tid < o) {
      const u128 b = s_ssq[tid + o];
      if (s_ssq[tid] > ~(u128)0 - b) s_bad[tid] = 1;
      s_ssq[tid] += b;
      s_bad[tid] |= s_bad[tid + o];
    }
    __syncthreads();
  }
  if (tid == 0) {
    uint64_t rms = 0;
    if (!s_bad[0]) {
      u128 mean = div_u128_u32(s_ssq[0], (uint32_t)cols);
      if (mean <= ~(u128)0 - (u128)(uint64_t)eps) rms = isqrt_u128(mean + (u128)(uint64_t)eps);
    }
    s_rms = rms;
    if (rms == 0) atomicOr(status, IMIE_ERMS);
  }
  __syncthreads();
  const uint64_t rms = s_rms;
  if (rms == 0) return;
  // normalized values (kept in registers for the gain pass when cols <= 16 * blockDim)
  uint64_t mxn = 0, mxg = 0;
  int nfit = 1;
  for (int64_t c = tid; c < cols; c += nt) {
    bool fits;
    const int64_t nv = norm_elem(xr[c], frac, rms, &fits);
    nfit &= fits ? 1 : 0;
    const uint64_t an = imie_absu64(nv);
    mxn = an > mxn ? an : mxn;
    if (gain) {
      const uint64_t ag = imie_absu64(gain[c]);
      mxg = ag > mxg ? ag : mxg;
    }
    out[row * cols + c] = nv;
  }
  if (!nfit) atomicOr(status, IMIE_ERMS);
  if (!gain) return;
  s_mx[tid] = mxn;
  __syncthreads();
  for (int o = nt / 2; o > 0; o >>= 1) {
    if (tid < o) s_mx[tid] = s_mx[tid] > s_mx[tid + o] ? s_mx[tid] : s_mx[tid + o];
    __syncthreads();
  }
  const uint64_t mn = s_mx[0];
  __syncthreads();
  s_mx[tid] = mxg;
  __syncthreads();
  for (int o = nt / 2; o > 0; o >>= 1) {
    if (tid < o) s_mx[tid] = s_mx[tid] > s_mx[tid + o] ? s_mx[tid] : s_mx[tid + o];
    __syncthreads();
  }
  const uint64_t mg = s_mx[0];
  if (mn != 0 && mg > (uint64_t)INT64_MAX / mn) {
    if (tid == 0) atomicOr(status, IMIE_ERMS);
    return;
  }
  for (int64_t c = tid; c < cols; c += nt) {
    const int64_t nv = out[row * cols + c];
    out[row * cols + c] = imie_floor_shift((int64_t)((uint64_t)nv * (uint64_t)gain[c]), frac);
  }
}

}  // namespace

int imie_rmsnorm_launch(const int64_t* x, int64_t rows, int64_t cols, int64_t frac, int64_t eps,
                        const int64_t* gain, int64_t* out, int* status, hipStream_t st) {
  if (rows <= 0) return IMIE_OK;
  const int nt = cols >= 2048 ? 256 : (cols >= 512 ? 128 : 64);
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
