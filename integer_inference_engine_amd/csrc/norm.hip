// Integer RMSNorm for gfx950 (reference semantics: bonsai/src/trinote/determinism/fixedpoint.py:31-71 and the
// C producer bonsai/tools/bonsai_q1_kernel.c:238-323):
//   ssq = sum x^2 (exact, 128-bit), rms = isqrt(ssq // cols + eps), n = floor((x << frac) / rms),
//   y = (n * gain) >> frac, refused (status bit 4) when ssq needs more than 128 bits, rms == 0, or
//   max|n| * max|gain| > INT64_MAX (the oracle's fail-loud gain envelope, checked per row = globally).
// One workgroup per row; the 128-bit sum is reduced by wave shuffles and LDS, the isqrt / mean run on one lane.
#include "imie_common.h"
#include "imie_kernels.h"
#include "imie_fixed.h"
#include "imie_silu.h"
#include <stdlib.h>

namespace {

using namespace imie_fx;
typedef unsigned __int128 u128;

// One workgroup (nt = 64..256 threads) per row. Rows of up to kNormPer * nt columns are loaded once and kept in
// registers (x and gain); longer rows are re-read. Each wave reduces its partials by shuffles; after one barrier
// every wave combines the per-wave partials from LDS itself (no single-lane serial phase). Steps: (1) 128-bit sum
// of squares -> rms, (2) n = floor((x << f) / rms) with max|n| and max|gain| for the envelope, (3) y = (n * g) >> f.
// Q1 digit table of a row staged in LDS: wave w takes slabs w, w + nw, ...; then this workgroup's zero-list share.
__device__ inline void prep_row(const int64_t* s_y, int64_t row, const imie_q1::Q1PrepOut& po,
                                const imie_q1::Q1Zero& zero, int tid, int nt) {
  __syncthreads();
  const int lane = tid & 63, wave = tid >> 6, nw = nt >> 6;
  const int64_t cols = po.nb * 128;
  for (int64_t sl = wave; sl < po.nslabs; sl += nw) {
    int64_t v[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int64_t p = imie_q1::prep_pos(lane, sl, q);
      v[q] = p < cols ? s_y[p] : 0;
    }
    imie_q1::prep_slab(v, po, row, sl);
  }
  imie_q1::zero_share(zero, row, (int64_t)gridDim.x, tid, nt);
}

// GEMM digit table of a row staged in LDS (T >= kGemmMinT): wave w takes slabs w, w + nw, ...
__device__ inline void prep_row_gemm(const int64_t* s_y, int64_t row, const imie_q1::GemmPrepOut& gp, int tid, int nt) {
  __syncthreads();
  const int lane = tid & 63, wave = tid >> 6, nw = nt >> 6;
  const int64_t cols = gp.nb * 128;
  for (int64_t sl = wave; sl < gp.nslabs; sl += nw) {
    int64_t v[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int64_t p = imie_q1::prep_pos(lane, sl, q);
      v[q] = p < cols ? s_y[p] : 0;
    }
    imie_q1::prep_gemm_slab(v, gp, row, sl);
  }
}

// NT threads with PER cached columns each (the per-thread serial work is what bounds a single-row launch, so
// wide rows get many threads). PREP: the row (cols = nb * 128 <= NT * PER) is also staged in LDS and turned
// into the Q1 digit table (one wave per 512-slab), and the workgroups clear the zero list of the next matvec.
constexpr int kPrepCols = 4096;

// PREP: 0 none, 1 the matvec digit table (po, zero), 2 the GEMM digit table (gp). With a table, out may be null
// (the GEMM reads only the table: no int64 copy of the normalised rows is written).
template <int PREP, int NT, int kNormPer>
__global__ __launch_bounds__(NT) void rmsnorm_kernel(const int64_t* __restrict__ x, int64_t cols, int frac,
                                                      int64_t eps, const int64_t* __restrict__ gain,
                                                      int64_t* __restrict__ out, int* __restrict__ status,
                                                      imie_q1::Q1PrepOut po, imie_q1::Q1Zero zero,
                                                      imie_q1::GemmPrepOut gp = {}) {
  constexpr int NW = NT / 64;
  __shared__ int64_t s_y[PREP ? kPrepCols : 1];
  __shared__ uint64_t s_hi[NW], s_lo[NW], s_mn[NW], s_mg[NW];
  __shared__ int s_bad[NW], s_fit[NW];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, nt = NT, lane = tid & 63, wave = tid >> 6, nw = NW;
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
  // short path of a cached wave whose |x| are all below 2^26: the 32 x 32 -> 64-bit squares of the wave sum
  // below 2^62 (kNormPer * 64 * 2^52), one 64-bit DPP sum
  uint64_t amax = 0;
  if (cached) {
#pragma unroll
    for (int k = 0; k < kNormPer; ++k) { const uint64_t a = imie_absu64(xv[k]); amax = a > amax ? a : amax; }
  }
  if (cached && kNormPer <= 16 && !__any((int)(amax >> 26) != 0)) {
    uint64_t sq = 0;
#pragma unroll
    for (int k = 0; k < kNormPer; ++k) {
      const uint32_t a = (uint32_t)imie_absu64(xv[k]);
      sq += (uint64_t)a * a;
    }
    lo = imie_wave_sum_u64_full(sq);
    hi = 0;
  } else {
    if (cached) {
#pragma unroll
      for (int k = 0; k < kNormPer; ++k) add_sq(xv[k]);
    } else {
      for (int64_t c = tid; c < cols; c += nt) add_sq(xr[c]);
    }
    wave_sum_u128(hi, lo, bad);
  }
  if (lane == 0) { s_hi[wave] = hi; s_lo[wave] = lo; s_bad[wave] = bad; }
  __syncthreads();
  // every wave: combine the per-wave sums (lane w holds wave w's) and derive rms / reciprocal redundantly
  hi = lane < nw ? s_hi[lane] : 0;
  lo = lane < nw ? s_lo[lane] : 0;
  bad = lane < nw ? s_bad[lane] : 0;
  wave_sum_u128(hi, lo, bad);
  uint64_t rms = 0;
  if (!bad) {
    const u128 mean = div_u128_cols(((u128)hi << 64) | lo, (uint32_t)cols);
    if (mean <= ~(u128)0 - (u128)(uint64_t)eps) rms = isqrt_u128_fast(mean + (u128)(uint64_t)eps);
  }
  if (rms == 0) {
    if (tid == 0) atomicOr(status, IMIE_ERMS);
    return;
  }
  // short path of a cached wave: n = floor((x << f) / rms) in double precision when every |x| << f of the wave
  // is below 2^53 and rms below 2^51 (1 <= f <= 52); otherwise the 64 / 128-bit integer routine
  const bool fast = cached && frac >= 1 && frac <= 52 && (rms >> 51) == 0 &&
                    !__any((int)((amax >> (53 - frac)) != 0));
  const double rms_d = (double)rms, rinv_d = 1.0 / rms_d;
  const uint64_t rinv = fast ? 0 : recip_u64(rms);
  uint64_t mxn = 0, mxg = 0;
  int nfit = 1;
  int64_t nvk[kNormPer];
  auto norm1 = [&](int64_t v, int64_t g, int64_t c, int64_t* keep) {
    bool fits = true;
    const int64_t nv = fast ? norm_elem_f64_fast(v, frac, rms_d, rinv_d) : norm_elem(v, frac, rms, rinv, &fits);
    nfit &= fits ? 1 : 0;
    const uint64_t an = imie_absu64(nv);
    mxn = an > mxn ? an : mxn;
    if (gain) {
      const uint64_t ag = imie_absu64(g);
      mxg = ag > mxg ? ag : mxg;
    } else {
      if (out) out[row * cols + c] = nv;
      if (PREP) s_y[c] = nv;
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
    if (PREP == 1) prep_row(s_y, row, po, zero, tid, nt);
    if (PREP == 2) { prep_row_gemm(s_y, row, gp, tid, nt); imie_q1::zero_share(zero, row, (int64_t)gridDim.x, tid, nt); }
    return;
  }
  mxn = imie_wave_max_u64_full(mxn);
  mxg = imie_wave_max_u64_full(mxg);
  nfit = __all(nfit);
  if (lane == 0) { s_mn[wave] = mxn; s_mg[wave] = mxg; s_fit[wave] = nfit; }
  __syncthreads();
  mxn = lane < nw ? s_mn[lane] : 0;
  mxg = lane < nw ? s_mg[lane] : 0;
  nfit = lane < nw ? s_fit[lane] : 1;
  mxn = imie_wave_max_u64(mxn);
  mxg = imie_wave_max_u64(mxg);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) nfit &= __shfl_xor(nfit, o, 64);
  if (!nfit || (mxn != 0 && mxg > (uint64_t)INT64_MAX / mxn)) {
    if (tid == 0) atomicOr(status, IMIE_ERMS);
    return;
  }
  if (cached) {
#pragma unroll
    for (int k = 0; k < kNormPer; ++k) {
      const int64_t c = tid + (int64_t)k * nt;
      if (c < cols) {
        const int64_t y = imie_floor_shift((int64_t)((uint64_t)nvk[k] * (uint64_t)gv[k]), frac);
        if (out) out[row * cols + c] = y;
        if (PREP) s_y[c] = y;
      }
    }
    if (PREP == 1) prep_row(s_y, row, po, zero, tid, nt);
    if (PREP == 2) { prep_row_gemm(s_y, row, gp, tid, nt); imie_q1::zero_share(zero, row, (int64_t)gridDim.x, tid, nt); }
  } else {
    for (int64_t c = tid; c < cols; c += nt) {
      bool fits;
      const int64_t nv = norm_elem(xr[c], frac, rms, rinv, &fits);
      out[row * cols + c] = imie_floor_shift((int64_t)((uint64_t)nv * (uint64_t)gain[c]), frac);
    }
  }
}


constexpr int kZeroWgs = 8;

// Single-row RMSNorm that writes the Q1 digit table of the next matvec (gain given, cols = nb * 128 <= 4096):
// eight waves, wave w holding slab w's 512 columns at the table's positions (prep_pos), so each wave turns its
// own registers into table entries (no LDS staging). One barrier combines the 128-bit sum of squares with the
// row's largest and smallest x and largest |gain|: n = floor((x << f) / rms) is non-decreasing in x, so max|n|
// (and whether every n fits int64) follows from the two extremes; the result equals the per-element check.
// kZeroWgs further workgroups clear the next matvec's K-split outputs in parallel with the row work.
__global__ __launch_bounds__(512) void rmsnorm_prep_slab_kernel(const int64_t* __restrict__ x, int64_t cols, int frac,
                                                                int64_t eps, const int64_t* __restrict__ gain,
                                                                int64_t* __restrict__ out, int* __restrict__ status,
                                                                imie_q1::Q1PrepOut po, imie_q1::Q1Zero zero) {
  __shared__ uint64_t s_lm[8][4], s_mg[8];
  __shared__ int64_t s_xmax[8], s_xmin[8];
  const int64_t rows = (int64_t)gridDim.x - kZeroWgs;
  if ((int64_t)blockIdx.x >= rows) {                  // the extra workgroups clear the next matvec's outputs
    imie_q1::zero_share(zero, (int64_t)blockIdx.x - rows, kZeroWgs, threadIdx.x, 512);
    return;
  }
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t* xr = x + row * cols;
  int64_t xv[8], gv[8];
  int64_t pos[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    pos[q] = imie_q1::prep_pos(lane, wave, q);
    xv[q] = pos[q] < cols ? xr[pos[q]] : 0;
    gv[q] = pos[q] < cols ? gain[pos[q]] : 0;
  }
  uint64_t hi = 0, lo = 0, mg = 0;
  int64_t xmax = 0, xmin = 0;                          // padding zeros are harmless: n(0) = 0 fits
  int bad = 0;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const uint64_t a = imie_absu64(xv[q]);
    const u128 sq = (u128)a * a;
    const uint64_t sl = (uint64_t)sq, sh = (uint64_t)(sq >> 64);
    const uint64_t nl = lo + sl;
    const uint64_t cy = nl < lo ? 1 : 0;
    const uint64_t nh = hi + sh;
    bad |= (nh < hi ? 1 : 0) | (nh + cy < nh ? 1 : 0);
    hi = nh + cy;
    lo = nl;
    xmax = xv[q] > xmax ? xv[q] : xmax;
    xmin = xv[q] < xmin ? xv[q] : xmin;
    const uint64_t ag = imie_absu64(gv[q]);
    mg = ag > mg ? ag : mg;
  }
  // wave level: DPP reductions (limb sums need no carries); block level: every lane folds the eight
  // wave results read from LDS (broadcast reads)
  uint64_t lm[4];
  u128_limbs(hi, lo, bad, lm);
#pragma unroll
  for (int i = 0; i < 4; ++i) lm[i] = imie_wave_sum_u64_full(lm[i]);
  mg = imie_wave_max_u64_full(mg);
  xmax = imie_wave_max0_i64_full(xmax);
  xmin = imie_wave_min0_i64_full(xmin);
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) s_lm[wave][i] = lm[i];
    s_mg[wave] = mg; s_xmax[wave] = xmax; s_xmin[wave] = xmin;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) lm[i] = 0;
#pragma unroll
  for (int w = 0; w < 8; ++w) {
#pragma unroll
    for (int i = 0; i < 4; ++i) lm[i] += s_lm[w][i];
    mg = s_mg[w] > mg ? s_mg[w] : mg;
    xmax = s_xmax[w] > xmax ? s_xmax[w] : xmax;
    xmin = s_xmin[w] < xmin ? s_xmin[w] : xmin;
  }
  u128_fold(lm, hi, lo, bad);
  uint64_t rms = 0;
  if (!bad) {
    const u128 mean = div_u128_cols(((u128)hi << 64) | lo, (uint32_t)cols);
    if (mean <= ~(u128)0 - (u128)(uint64_t)eps) rms = isqrt_u128(mean + (u128)(uint64_t)eps);
  }
  if (rms == 0) {
    if (tid == 0) atomicOr(status, IMIE_ERMS);
    return;
  }
  const uint64_t rinv = recip_u64(rms);
  // the eight own elements and, alongside, one extreme per lane (even lanes the largest x, odd the smallest)
  int64_t nv[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    bool f;
    nv[q] = norm_elem(xv[q], frac, rms, rinv, &f);
  }
  bool fe = true;
  const uint64_t ne = imie_absu64(norm_elem((lane & 1) ? xmin : xmax, frac, rms, rinv, &fe));
  const uint64_t na = imie_readlane_u64(ne, 0), nb = imie_readlane_u64(ne, 1);
  const int fa = __builtin_amdgcn_readlane(fe ? 1 : 0, 0), fb = __builtin_amdgcn_readlane(fe ? 1 : 0, 1);
  const uint64_t mxn = na > nb ? na : nb;
  if (!fa || !fb || (mxn != 0 && mg > (uint64_t)INT64_MAX / mxn)) {
    if (tid == 0) atomicOr(status, IMIE_ERMS);
    return;
  }
  int64_t y[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    y[q] = imie_floor_shift((int64_t)((uint64_t)nv[q] * (uint64_t)gv[q]), frac);
    if (pos[q] < cols) out[row * cols + pos[q]] = y[q];
  }
  if (wave < po.nslabs) imie_q1::prep_slab(y, po, row, wave);
}

}  // namespace

int imie_rmsnorm_launch(const int64_t* x, int64_t rows, int64_t cols, int64_t frac, int64_t eps,
                        const int64_t* gain, int64_t* out, int* status, hipStream_t st) {
  if (rows <= 0) return IMIE_OK;
  const imie_q1::Q1PrepOut po = {};
  const imie_q1::Q1Zero z = {};
  static const int force_nt = [] { const char* e = getenv("IMIE_NORM_NT"); return e ? atoi(e) : 0; }();  // tuning
  if (force_nt == 64)
    hipLaunchKernelGGL((rmsnorm_kernel<0, 64, 4>), dim3((unsigned)rows), dim3(64), 0, st, x, cols, (int)frac, eps,
                       gain, out, status, po, z);
  else if (force_nt == 256)
    hipLaunchKernelGGL((rmsnorm_kernel<0, 256, 16>), dim3((unsigned)rows), dim3(256), 0, st, x, cols, (int)frac,
                       eps, gain, out, status, po, z);
  else if (force_nt == 512)
    hipLaunchKernelGGL((rmsnorm_kernel<0, 512, 8>), dim3((unsigned)rows), dim3(512), 0, st, x, cols, (int)frac,
                       eps, gain, out, status, po, z);
  else if (cols <= 256)
    hipLaunchKernelGGL((rmsnorm_kernel<0, 64, 4>), dim3((unsigned)rows), dim3(64), 0, st, x, cols, (int)frac, eps,
                       gain, out, status, po, z);
  else if (cols <= 1024)
    hipLaunchKernelGGL((rmsnorm_kernel<0, 256, 4>), dim3((unsigned)rows), dim3(256), 0, st, x, cols, (int)frac,
                       eps, gain, out, status, po, z);
  else if (rows >= 64 && cols <= 4096)
    // many rows (prefill): 256 threads x 16 cached columns keep more rows in flight per CU than 1024 x 4; measured
    // 47 us against 71 us for 2048 rows of 4096 on MI355X (a single row is latency-bound and keeps 1024 threads)
    hipLaunchKernelGGL((rmsnorm_kernel<0, 256, 16>), dim3((unsigned)rows), dim3(256), 0, st, x, cols, (int)frac,
                       eps, gain, out, status, po, z);
  else
    hipLaunchKernelGGL((rmsnorm_kernel<0, 1024, 4>), dim3((unsigned)rows), dim3(1024), 0, st, x, cols, (int)frac,
                       eps, gain, out, status, po, z);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

int imie_rmsnorm_prep_launch(const int64_t* x, int64_t rows, int64_t cols, int64_t frac, int64_t eps,
                             const int64_t* gain, int64_t* out, int* status, const imie_q1::Q1PrepOut& po,
                             const imie_q1::Q1Zero& zero, hipStream_t st) {
  if (rows <= 0) return IMIE_OK;
  if (cols != po.nb * 128 || cols > kPrepCols) return IMIE_EARG;
  if (gain && po.nslabs <= 8)
    hipLaunchKernelGGL(rmsnorm_prep_slab_kernel, dim3((unsigned)(rows + kZeroWgs)), dim3(512), 0, st, x, cols, (int)frac, eps,
                       gain, out, status, po, zero);
  else if (cols <= 1024)
    hipLaunchKernelGGL((rmsnorm_kernel<1, 256, 4>), dim3((unsigned)rows), dim3(256), 0, st, x, cols, (int)frac,
                       eps, gain, out, status, po, zero);
  else
    hipLaunchKernelGGL((rmsnorm_kernel<1, 1024, 4>), dim3((unsigned)rows), dim3(1024), 0, st, x, cols, (int)frac,
                       eps, gain, out, status, po, zero);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

int imie_rmsnorm_gemm_prep_launch(const int64_t* x, int64_t rows, int64_t cols, int64_t frac, int64_t eps,
                                  const int64_t* gain, int64_t* out, int* status, const imie_q1::GemmPrepOut& gp,
                                  const imie_q1::Q1Zero& zero, hipStream_t st) {
  if (rows <= 0) return IMIE_OK;
  if (cols != gp.nb * 128 || cols > kPrepCols || rows < imie_q1::kGemmMinT) return IMIE_EARG;
  const imie_q1::Q1PrepOut po = {};
  static const int nt_env = [] { const char* e = getenv("IMIE_NORM_GEMM_NT"); return e ? atoi(e) : 0; }();  // tuning
  const int nt = nt_env ? nt_env : (rows <= 128 ? 1024 : 256);
  // few rows (batched decode): each row's latency chain is the launch, so more threads per row; many rows
  // (prefill): 256 threads x 16 columns keep more rows in flight per CU
  if (nt == 1024)
    hipLaunchKernelGGL((rmsnorm_kernel<2, 1024, 4>), dim3((unsigned)rows), dim3(1024), 0, st, x, cols, (int)frac, eps,
                       gain, out, status, po, zero, gp);
  else if (nt == 512)
    hipLaunchKernelGGL((rmsnorm_kernel<2, 512, 8>), dim3((unsigned)rows), dim3(512), 0, st, x, cols, (int)frac, eps,
                       gain, out, status, po, zero, gp);
  else
    hipLaunchKernelGGL((rmsnorm_kernel<2, 256, 16>), dim3((unsigned)rows), dim3(256), 0, st, x, cols, (int)frac, eps,
                       gain, out, status, po, zero, gp);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

namespace {
struct NormWs {
  DevBuf x, out, gain, status;
  Q1Ws q1;                        // digit-table target of the fused entry point
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

// Host evaluation of the RMSNorm kernels' exact helpers (CPU test hooks, no reference counterpart):
// floor(sqrt(hi * 2^64 + lo)), floor((2^64 - 1) / d) and floor((hi * 2^64 + lo) / d) (low 64 bits).
// The fused producer (RMSNorm that also writes the next Q1 matvec's digit table, used by the resident decode
// for rows < 8) with bonsai_rmsnorm_gpu's host contract: same outputs and rc, the table goes to a workspace.
// cols must be a multiple of 128 and at most 4096.
int imie_rmsnorm_fused_gpu(const int64_t* x, int64_t rows, int64_t cols, int64_t frac, int64_t eps,
                           const int64_t* gain, int64_t* out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!x || !out || rows < 0 || cols <= 0 || cols % 128 || cols > 4096 || frac < 0 || frac > 62 || eps < 0)
    return IMIE_EARG;
  if (rows == 0) return IMIE_OK;
  if (imie_device_ready() != 0) return IMIE_EARG;
  hipStream_t st = imie_stream();
  const size_t xb = (size_t)(rows * cols) * 8;
  if (g_nws.x.ensure(xb) || g_nws.out.ensure(xb) || g_nws.gain.ensure((size_t)cols * 8) || g_nws.status.ensure(64))
    return IMIE_EARG;
  imie_q1::Q1PrepOut po;
  int rc = imie_q1_prep_target(&g_nws.q1, cols / 128, rows, &po);
  if (rc) return rc;
  IMIE_HIP(hipMemcpyAsync(g_nws.x.p, x, xb, hipMemcpyHostToDevice, st));
  if (gain) IMIE_HIP(hipMemcpyAsync(g_nws.gain.p, gain, (size_t)cols * 8, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemsetAsync(g_nws.status.p, 0, 4, st));
  const imie_q1::Q1Zero z = {};
  rc = imie_rmsnorm_prep_launch((const int64_t*)g_nws.x.p, rows, cols, frac, eps,
                                gain ? (const int64_t*)g_nws.gain.p : nullptr, (int64_t*)g_nws.out.p,
                                (int*)g_nws.status.p, po, z, st);
  if (rc) return rc;
  int stat = 0;
  IMIE_HIP(hipMemcpyAsync(&stat, g_nws.status.p, 4, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipMemcpyAsync(out, g_nws.out.p, xb, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipStreamSynchronize(st));
  return stat ? IMIE_ERMS : IMIE_OK;
}

uint64_t imie_fx_isqrt_u128(uint64_t hi, uint64_t lo) { return imie_fx::isqrt_u128(((imie_fx::u128)hi << 64) | lo); }
uint64_t imie_fx_recip_u64(uint64_t d) { return imie_fx::recip_u64(d); }
uint64_t imie_fx_isqrt_fast(uint64_t hi, uint64_t lo) {
  return imie_fx::isqrt_u128_fast(((imie_fx::u128)hi << 64) | lo);
}
int imie_fx_norm_f64(int64_t x, int frac, uint64_t rms, int64_t* out) {
  if (!out || rms == 0) return -1;
  const double rd = (double)rms;
  return imie_fx::norm_elem_f64(x, frac, rms, rd, 1.0 / rd, out) ? 1 : 0;
}
int64_t imie_silu_mul_host(int64_t g, int64_t u, int64_t frac, int fast) {
  int64_t log2e, dclip;
  imie_silu_consts(frac, &log2e, &dclip);
  return fast ? imie_silu::silu_mul_fast(g, u, (int)frac, log2e, dclip) : imie_silu::silu_mul(g, u, (int)frac, log2e, dclip);
}
// the softmax short paths: exp_clipped (fast != 0: the 32-bit form) and prob_div
int64_t imie_exp_clipped_host(int64_t d, int64_t frac, int fast) {
  int64_t log2e, dclip;
  imie_silu_consts(frac, &log2e, &dclip);
  return imie_silu::exp_clipped(d, (int)frac, log2e, fast != 0 && (dclip >> 32) == 0 && (log2e >> 32) == 0);
}
int64_t imie_prob_div_host(int64_t e, int64_t frac, uint64_t z) {
  return imie_silu::prob_div(e, (int)frac, z, 1.0 / (double)z);
}
uint64_t imie_fx_div_u128(uint64_t hi, uint64_t lo, uint32_t d) {
  return (uint64_t)imie_fx::div_u128_cols(((imie_fx::u128)hi << 64) | lo, d);
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
