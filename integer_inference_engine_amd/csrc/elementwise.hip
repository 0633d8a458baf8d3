// Element-wise integer kernels around the Q1 matmuls (gfx950).
//   RoPE NeoX apply         bonsai/src/trinote/model/rope_v2.py:92-117 (+ guard rope.py:26-39)
//   SiLU / SiLU*up          reference_bonsai.py:245-264, :611-614 over fixedpoint.py:143-174 (wrap mod 2^64)
//   residual add            reference_bonsai.py:960-964 (wrap)
//   embedding rows          reference_bonsai.py:138-146 (sign * scale, no shift)
//   lowest-index argmax     reference_bonsai.py:812-827 (numpy first-max)
#include "imie_common.h"
#include "imie_kernels.h"
#include "imie_silu.h"

namespace {

using namespace imie_silu;
typedef unsigned __int128 u128;

__global__ void silu_mul_kernel(const int64_t* __restrict__ gate, const int64_t* __restrict__ up, int64_t n, int frac,
                                int64_t log2e, int64_t dclip, int64_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t g = gate[i];
  const int64_t silu = (int64_t)((uint64_t)g * (uint64_t)sigmoid_fixed_fast(g, frac, log2e, dclip)) >> frac;
  out[i] = up ? (int64_t)((uint64_t)silu * (uint64_t)up[i]) >> frac : silu;
}

// silu_mul for the GEMM: one wave per (token, 512-slab), four slabs per workgroup, computes h at its eight table
// positions and writes the GEMM digit table directly (the prep of the next projection, without h round-tripping
// through HBM). Every gate / up load of the wave is issued before the first product.
__global__ __launch_bounds__(256) void silu_mul_gemm_prep_kernel(const int64_t* __restrict__ gate,
                                                                 const int64_t* __restrict__ up, int64_t n, int frac,
                                                                 int64_t log2e, int64_t dclip,
                                                                 imie_q1::GemmPrepOut gp) {
  const int lane = threadIdx.x & 63;
  const int64_t sl = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6), t = blockIdx.y;
  if (sl >= gp.nslabs) return;                        // whole wave
  int64_t gv[8], uv[8], v[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int64_t p = imie_q1::prep_pos(lane, sl, q);
    const int64_t pc = p < n ? p : 0;
    gv[q] = gate[t * n + pc];
    uv[q] = up[t * n + pc];
  }
#pragma unroll
  for (int q = 0; q < 8; ++q)
    v[q] = imie_q1::prep_pos(lane, sl, q) < n ? silu_mul_fast(gv[q], uv[q], frac, log2e, dclip) : 0;
  imie_q1::prep_gemm_slab(v, gp, t, sl);
}

// silu_mul for one (token, 512-slab): thread per element into LDS, then wave 0 builds the slab's digit table
__global__ __launch_bounds__(512) void silu_mul_prep_kernel(const int64_t* __restrict__ gate,
                                                            const int64_t* __restrict__ up, int64_t n, int frac,
                                                            int64_t log2e, int64_t dclip, int64_t* __restrict__ out,
                                                            imie_q1::Q1PrepOut po) {
  __shared__ int64_t sh[512];
  const int64_t sl = blockIdx.x, t = blockIdx.y;
  const int64_t p = sl * 512 + threadIdx.x;
  int64_t h = 0;
  if (p < n) {
    h = silu_mul_fast(gate[t * n + p], up[t * n + p], frac, log2e, dclip);
    out[t * n + p] = h;
  }
  sh[threadIdx.x] = h;
  __syncthreads();
  if (threadIdx.x >= 64) return;
  int64_t v[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) v[q] = sh[imie_q1::prep_pos(threadIdx.x, 0, q)];
  imie_q1::prep_slab(v, po, t, sl);
}

__global__ void add_kernel(int64_t* __restrict__ x, const int64_t* __restrict__ y, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] = (int64_t)((uint64_t)x[i] + (uint64_t)y[i]);
}

__device__ inline void atomic_max_u64(uint64_t* p, uint64_t v) {
  atomicMax((unsigned long long*)p, (unsigned long long)v);
}

__global__ __launch_bounds__(256) void rope_kernel(const int64_t* __restrict__ x, int64_t rows, int64_t nh, int64_t hd,
                                                   const int64_t* __restrict__ pos, int64_t pos0,
                                                   const int64_t* __restrict__ cs, const int64_t* __restrict__ sn,
                                                   int frac, int64_t* __restrict__ out, uint64_t* __restrict__ guard) {
  const int64_t half = hd / 2;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint64_t mx = 0, mc = 0;
  if (i < rows * nh * half) {
    const int64_t j = i % half, h = (i / half) % nh, r = i / (half * nh);
    const int64_t p = pos ? pos[r] : pos0 + r;
    const int64_t* xv = x + (r * nh + h) * hd;
    const int64_t x0 = xv[j], x1 = xv[j + half];
    const int64_t c = cs[p * half + j], s = sn[p * half + j];
    int64_t* o = out + (r * nh + h) * hd;
    o[j] = (int64_t)((uint64_t)x0 * (uint64_t)c - (uint64_t)x1 * (uint64_t)s) >> frac;
    o[j + half] = (int64_t)((uint64_t)x0 * (uint64_t)s + (uint64_t)x1 * (uint64_t)c) >> frac;
    const uint64_t a0 = imie_absu64(x0), a1 = imie_absu64(x1), ac = imie_absu64(c), as = imie_absu64(s);
    mx = a0 > a1 ? a0 : a1;
    mc = ac > as ? ac : as;
  }
  // wave-level max, one atomic per wave
  mx = imie_wave_max_u64(mx);
  mc = imie_wave_max_u64(mc);
  if ((threadIdx.x & 63) == 0) {
    atomic_max_u64(&guard[0], mx);
    atomic_max_u64(&guard[1], mc);
  }
}

__global__ void rope_guard_kernel(const uint64_t* __restrict__ guard, int* __restrict__ status) {
  const u128 b = (u128)2 * guard[0] * guard[1];
  if (b > (u128)INT64_MAX) atomicOr(status, IMIE_EOVF);
}

__global__ void embed_kernel(const uint8_t* __restrict__ bits, const int64_t* __restrict__ scale, int64_t nb,
                             const int64_t* __restrict__ ids, int64_t T, int64_t* __restrict__ out) {
  const int64_t d = nb * 128;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= T * d) return;
  const int64_t t = i / d, k = i % d, id = ids[t];
  const int bit = (bits[(id * nb + k / 128) * 16 + (k % 128) / 8] >> (k % 8)) & 1;
  const int64_t sc = scale[id * nb + k / 128];
  out[i] = bit ? sc : (int64_t)(0 - (uint64_t)sc);
}

// lowest-index argmax: stage 1 reduces a contiguous column range per workgroup to (value, index); stage 2
// reduces the partials of a row. Ties keep the lower index at every level, which is numpy's first-max rule.
__device__ inline void amx_merge(int64_t& v, int64_t& i, int64_t v2, int64_t i2) {
  if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
}

__device__ inline void amx_block(int64_t& v, int64_t& i, int64_t* sv, int64_t* si) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) amx_merge(v, i, __shfl_xor(v, o, 64), __shfl_xor(i, o, 64));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if (lane == 0) { sv[wave] = v; si[wave] = i; }
  __syncthreads();
  if (threadIdx.x == 0)
    for (int w = 1; w < nw; ++w) amx_merge(v, i, sv[w], si[w]);
}

__global__ __launch_bounds__(256) void argmax_part_kernel(const int64_t* __restrict__ logits, int64_t cols,
                                                          int64_t per, int64_t* __restrict__ part, int nparts) {
  __shared__ int64_t sv[4], si[4];
  const int64_t row = blockIdx.y;
  const int64_t c0 = (int64_t)blockIdx.x * per, c1 = min(cols, c0 + per);
  const int64_t* lr = logits + row * cols;
  int64_t bv = INT64_MIN, bi = INT64_MAX;
  for (int64_t c = c0 + threadIdx.x; c < c1; c += blockDim.x) amx_merge(bv, bi, lr[c], c);
  amx_block(bv, bi, sv, si);
  if (threadIdx.x == 0) {
    part[(row * nparts + blockIdx.x) * 2] = bv;
    part[(row * nparts + blockIdx.x) * 2 + 1] = bi;
  }
}

__global__ __launch_bounds__(256) void argmax_final_kernel(const int64_t* __restrict__ part, int nparts,
                                                           int64_t* __restrict__ ids) {
  __shared__ int64_t sv[4], si[4];
  const int64_t row = blockIdx.x;
  int64_t bv = INT64_MIN, bi = INT64_MAX;
  for (int p = threadIdx.x; p < nparts; p += blockDim.x)
    amx_merge(bv, bi, part[(row * nparts + p) * 2], part[(row * nparts + p) * 2 + 1]);
  amx_block(bv, bi, sv, si);
  if (threadIdx.x == 0) ids[row] = bi == INT64_MAX ? 0 : bi;
}

}  // namespace

int imie_rope_launch(const int64_t* x, int64_t rows, int64_t nh, int64_t hd, const int64_t* pos, int64_t pos0,
                     const int64_t* cos, const int64_t* sin, int64_t frac, int64_t* out, uint64_t* guard,
                     hipStream_t st) {
  const int64_t n = rows * nh * (hd / 2);
  if (n <= 0) return IMIE_OK;
  hipLaunchKernelGGL(rope_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, rows, nh, hd, pos, pos0,
                     cos, sin, (int)frac, out, guard);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

int imie_rope_guard_check(const uint64_t* guard, int* status, hipStream_t st) {
  hipLaunchKernelGGL(rope_guard_kernel, dim3(1), dim3(1), 0, st, guard, status);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

static void silu_consts(int64_t frac, int64_t* log2e, int64_t* dclip) {
  const int64_t sh = 16 - frac;
  *log2e = sh >= 0 ? (94548 >> sh) : ((int64_t)94548 << -sh);
  const int64_t a = ((frac + 2) << (2 * frac)) / *log2e, b = ((int64_t)1 << 62) / *log2e;
  *dclip = a < b ? a : b;
}

void imie_silu_consts(int64_t frac, int64_t* log2e, int64_t* dclip) { silu_consts(frac, log2e, dclip); }

int imie_silu_mul_launch(const int64_t* gate, const int64_t* up, int64_t n, int64_t frac, int64_t* out,
                         hipStream_t st) {
  if (n <= 0) return IMIE_OK;
  int64_t log2e, dclip;
  silu_consts(frac, &log2e, &dclip);
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, gate, up, n, (int)frac,
                     log2e, dclip, out);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

int imie_silu_mul_prep_launch(const int64_t* gate, const int64_t* up, int64_t T, int64_t n, int64_t frac,
                              int64_t* out, const imie_q1::Q1PrepOut& po, hipStream_t st) {
  if (T <= 0) return IMIE_OK;
  if (!up || n != po.nb * 128) return IMIE_EARG;
  int64_t log2e, dclip;
  silu_consts(frac, &log2e, &dclip);
  hipLaunchKernelGGL(silu_mul_prep_kernel, dim3((unsigned)po.nslabs, (unsigned)T), dim3(512), 0, st, gate, up, n,
                     (int)frac, log2e, dclip, out, po);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

int imie_silu_mul_gemm_prep_launch(const int64_t* gate, const int64_t* up, int64_t T, int64_t n, int64_t frac,
                                   const imie_q1::GemmPrepOut& gp, hipStream_t st) {
  if (T <= 0) return IMIE_OK;
  if (n != gp.nb * 128 || frac < 1 || frac > 62) return IMIE_EARG;
  int64_t log2e, dclip;
  silu_consts(frac, &log2e, &dclip);
  hipLaunchKernelGGL(silu_mul_gemm_prep_kernel, dim3((unsigned)((gp.nslabs + 3) / 4), (unsigned)T), dim3(256), 0, st,
                     gate, up, n,
                     (int)frac, log2e, dclip, gp);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

int imie_silu_launch(const int64_t* x, int64_t n, int64_t frac, int64_t* out, hipStream_t st) {
  return imie_silu_mul_launch(x, nullptr, n, frac, out, st);
}

int imie_add_launch(int64_t* x, const int64_t* y, int64_t n, hipStream_t st) {
  if (n <= 0) return IMIE_OK;
  hipLaunchKernelGGL(add_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, y, n);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

int imie_embed_launch(const uint8_t* bits, const int64_t* scale, int64_t nb, const int64_t* ids, int64_t T,
                      int64_t* out, hipStream_t st) {
  const int64_t n = T * nb * 128;
  if (n <= 0) return IMIE_OK;
  hipLaunchKernelGGL(embed_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, bits, scale, nb, ids, T, out);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

int imie_argmax_launch(const int64_t* logits, int64_t rows, int64_t cols, int64_t* ids, int64_t* scratch,
                       hipStream_t st) {
  if (rows <= 0) return IMIE_OK;
  if (cols <= 0 || !scratch) return IMIE_EARG;
  int64_t per = 2048;
  int nparts = (int)((cols + per - 1) / per);
  if (nparts > kArgmaxParts) { nparts = kArgmaxParts; per = (cols + nparts - 1) / nparts; }
  hipLaunchKernelGGL(argmax_part_kernel, dim3((unsigned)nparts, (unsigned)rows), dim3(256), 0, st, logits, cols, per,
                     scratch, nparts);
  IMIE_HIP(hipGetLastError());
  hipLaunchKernelGGL(argmax_final_kernel, dim3((unsigned)rows), dim3(256), 0, st, scratch, nparts, ids);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

namespace {
struct EwWs {
  DevBuf a, b, c, status;
} g_ews;
}  // namespace

extern "C" {

// bonsai_q1_gpu.cu:848-864 / bonsai_q1_kernel.c:1729-1767 `bonsai_silu_i64` semantics on the GPU:
// out = (x * sigmoid(x)) >> frac, wrapping mod 2^64. Host pointers, synchronous.
int bonsai_silu_gpu(const int64_t* x, int64_t n, int64_t frac, int64_t* out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!x || !out || n < 0 || frac < 1 || frac > 29) return IMIE_EARG;
  if (n == 0) return IMIE_OK;
  if (imie_device_ready() != 0) return IMIE_EARG;
  hipStream_t st = imie_stream();
  const size_t b = (size_t)n * 8;
  if (g_ews.a.ensure(b) || g_ews.b.ensure(b)) return IMIE_EARG;
  IMIE_HIP(hipMemcpyAsync(g_ews.a.p, x, b, hipMemcpyHostToDevice, st));
  int rc = imie_silu_launch((const int64_t*)g_ews.a.p, n, frac, (int64_t*)g_ews.b.p, st);
  if (rc) return rc;
  IMIE_HIP(hipMemcpyAsync(out, g_ews.b.p, b, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipStreamSynchronize(st));
  return IMIE_OK;
}

// NeoX RoPE apply (rope_v2.py:92-117) over x (rows, nh, hd) where row r uses table row pos[r]; cos/sin
// (n_pos, hd/2). Host pointers, synchronous; rc 2 where the oracle raises (2*max|x|*max|cs| > INT64_MAX).
int imie_rope_neox_gpu(const int64_t* x, int64_t rows, int64_t nh, int64_t hd, const int64_t* pos,
                       const int64_t* cos, const int64_t* sin, int64_t n_pos, int64_t frac, int64_t* out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!x || !out || !pos || !cos || !sin || rows < 0 || nh <= 0 || hd <= 0 || (hd & 1) || n_pos <= 0 || frac < 0 ||
      frac > 62)
    return IMIE_EARG;
  for (int64_t r = 0; r < rows; ++r)
    if (pos[r] < 0 || pos[r] >= n_pos) return IMIE_EARG;
  if (rows == 0) return IMIE_OK;
  if (imie_device_ready() != 0) return IMIE_EARG;
  hipStream_t st = imie_stream();
  const size_t xb = (size_t)(rows * nh * hd) * 8, tb = (size_t)(n_pos * hd / 2) * 8;
  if (g_ews.a.ensure(xb + (size_t)rows * 8) || g_ews.b.ensure(xb) || g_ews.c.ensure(2 * tb) ||
      g_ews.status.ensure(64))
    return IMIE_EARG;
  char* a = (char*)g_ews.a.p;
  char* c = (char*)g_ews.c.p;
  IMIE_HIP(hipMemcpyAsync(a, x, xb, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemcpyAsync(a + xb, pos, (size_t)rows * 8, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemcpyAsync(c, cos, tb, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemcpyAsync(c + tb, sin, tb, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemsetAsync(g_ews.status.p, 0, 64, st));
  uint64_t* guard = (uint64_t*)((char*)g_ews.status.p + 16);
  int rc = imie_rope_launch((const int64_t*)a, rows, nh, hd, (const int64_t*)(a + xb), 0, (const int64_t*)c,
                            (const int64_t*)(c + tb), frac, (int64_t*)g_ews.b.p, guard, st);
  if (rc) return rc;
  rc = imie_rope_guard_check(guard, (int*)g_ews.status.p, st);
  if (rc) return rc;
  int stat = 0;
  IMIE_HIP(hipMemcpyAsync(&stat, g_ews.status.p, 4, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipMemcpyAsync(out, g_ews.b.p, xb, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipStreamSynchronize(st));
  return stat ? IMIE_EOVF : IMIE_OK;
}

// Lowest-index argmax over rows of int64 logits (reference_bonsai.py:812-827). Host pointers, synchronous.
int imie_argmax_gpu(const int64_t* logits, int64_t rows, int64_t cols, int64_t* ids) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!logits || !ids || rows < 0 || cols <= 0) return IMIE_EARG;
  if (rows == 0) return IMIE_OK;
  if (imie_device_ready() != 0) return IMIE_EARG;
  hipStream_t st = imie_stream();
  const size_t b = (size_t)(rows * cols) * 8;
  if (g_ews.a.ensure(b) || g_ews.b.ensure((size_t)rows * 8)) return IMIE_EARG;
  IMIE_HIP(hipMemcpyAsync(g_ews.a.p, logits, b, hipMemcpyHostToDevice, st));
  if (g_ews.c.ensure(imie_argmax_scratch_bytes(rows))) return IMIE_EARG;
  int rc = imie_argmax_launch((const int64_t*)g_ews.a.p, rows, cols, (int64_t*)g_ews.b.p, (int64_t*)g_ews.c.p, st);
  if (rc) return rc;
  IMIE_HIP(hipMemcpyAsync(ids, g_ews.b.p, (size_t)rows * 8, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipStreamSynchronize(st));
  return IMIE_OK;
}

}  // extern "C"
