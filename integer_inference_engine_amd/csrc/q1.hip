// Packed Q1_0 linear for gfx950.
//
//   out[t, o] = sum_b ( S[t, o, b] * scale[o, b] ) >> frac        (mod 2^64, floor per 128-block)
//   S[t, o, b] = sum_{i in block b} sign[o, i] * x[t, i] = 2 * pos - total,  pos = sum_{bit=1} x
//
// Reference semantics: bonsai/src/trinote/infer_int/reference_bonsai.py:149-219 (q1_linear_ref) and the C
// producer bonsai/tools/bonsai_q1_kernel.c:85-106. Bit i of byte j of a block is weight 8j+i.
//
// Matvec design (T small): int8 MFMA v_mfma_i32_16x16x64_i8 with
//   * B operand = weight bits of 16 output rows, expanded with ONE v_and per 4 weights:
//       B_s dword d = word_d & (0x01010101 << s)   -> bytes in {0, 2^s}  (s = 0..7, 0x80 reads as -128)
//   * A operand = balanced base-256 digits ("limbs") of x, arranged so the 16 MFMA rows are
//       (block g in the 4-block slab, shift s & 3); one accumulator for s < 4 and one for s >= 4.
//     After the MFMAs lane (grp, n) holds the per-(block, shift) partials of output row n; a shift-and-add
//     plus a 2-step cross-lane reduce-scatter leaves lane (g, n) with pos(block g, row n) for that limb.
//   * The per-(row, block) epilogue (limb recombination, 2*pos - total, * scale, floor shift, add) runs with
//     all 64 lanes busy, in int32 when max|x| <= 2^23 and in wrapping int64 otherwise.
// MFMA int32 accumulation is exact: each D entry is at most 128 * 128 * 2^7 in magnitude.
#include "imie_common.h"
#include <string.h>
#include <stdlib.h>

namespace {

constexpr int kTileRows = 16;      // output rows per MFMA tile
constexpr int kSlabBlocks = 4;     // 128-blocks per slab (= K 512 per wave step)
constexpr int kMaxLimbs = 8;

// ------------------------------------------------------------------------------------------------------
// Registry of resident Q1 weights (process-global, handle = index). Layout per weight:
//   bitsT [tile][slab][lane 64] uint4   (lane = 16*g + j -> row 16*tile + j, block 4*slab + g, 16 bytes)
//   scaleT[tile][slab][lane 64] int32 (narrowed losslessly) or int64
// Padding rows/blocks have zero bits AND zero scale, so they contribute exactly 0.
// ------------------------------------------------------------------------------------------------------
struct Q1Weight {
  int64_t N = 0, nb = 0, ntiles = 0, nslabs = 0;
  uint4* bits = nullptr;
  void* scale = nullptr;
  int scale64 = 0;
  size_t bytes = 0;
  bool live = false;
};

std::vector<Q1Weight>& registry() {
  static std::vector<Q1Weight> r;
  return r;
}
uint64_t g_resident_bytes = 0;

struct Workspace {
  DevBuf x, out, xq, totals, lslab;
} g_ws;

}  // namespace

// Host repack: natural (N, nb, 16) bits + (N, nb) scales -> tiled layout. Exposed for CPU tests.
extern "C" int imie_q1_repack_host(const uint8_t* bits, const int64_t* scale, int64_t N, int64_t nb,
                                   int scale64, uint8_t* bitsT, void* scaleT) {
  if (!bits || !scale || !bitsT || !scaleT || N <= 0 || nb <= 0) return IMIE_EARG;
  const int64_t ntiles = (N + kTileRows - 1) / kTileRows;
  const int64_t nslabs = (nb + kSlabBlocks - 1) / kSlabBlocks;
  for (int64_t tile = 0; tile < ntiles; ++tile)
    for (int64_t sl = 0; sl < nslabs; ++sl)
      for (int lane = 0; lane < 64; ++lane) {
        const int64_t row = tile * kTileRows + (lane & 15);
        const int64_t blk = sl * kSlabBlocks + (lane >> 4);
        const int64_t idx = (tile * nslabs + sl) * 64 + lane;
        uint8_t* dst = bitsT + idx * 16;
        int64_t sc = 0;
        if (row < N && blk < nb) {
          memcpy(dst, bits + (row * nb + blk) * 16, 16);
          sc = scale[row * nb + blk];
        } else {
          memset(dst, 0, 16);
        }
        if (scale64) ((int64_t*)scaleT)[idx] = sc;
        else ((int32_t*)scaleT)[idx] = (int32_t)sc;
      }
  return IMIE_OK;
}

// ------------------------------------------------------------------------------------------------------
// Activation prep: per (token t, slab) one wave computes max|x| -> limb count L, the per-block totals and
// the digit operand table xq[t][l][block][s] (uint4: dword d packs digits of positions 32d + 8c + s,
// c = 0..3, as bytes c). Lane layout: g = lane>>4 (block of slab), s = lane&7, dh = (lane>>3)&1 covering
// d in {2dh, 2dh+1}: 8 positions per lane.
// ------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(64) void q1_prep_kernel(const int64_t* __restrict__ x, int64_t K, int64_t nb,
                                                      int64_t nbp, int64_t nslabs, uint32_t* __restrict__ xq,
                                                      int64_t* __restrict__ totals, int* __restrict__ lslab) {
  const int lane = threadIdx.x;
  const int64_t sl = blockIdx.x;
  const int64_t t = blockIdx.y;
  const int g = lane >> 4, s = lane & 7, dh = (lane >> 3) & 1;
  const int64_t blk = sl * kSlabBlocks + g;
  int64_t v[8];
  uint64_t mx = 0;
  int64_t part = 0;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int d = 2 * dh + (q >> 2), c = q & 3;
    const int64_t pos = blk * 128 + 32 * d + 8 * c + s;
    const int64_t xv = (blk < nb) ? x[t * K + pos] : 0;
    v[q] = xv;
    const uint64_t a = imie_absu64(xv);
    mx = a > mx ? a : mx;
    part = (int64_t)((uint64_t)part + (uint64_t)xv);
  }
  mx = imie_wave_max_u64(mx);
  const int L = imie_limbs_needed(mx);
  // block total: sum over the 16 lanes of group g (xor 1,2,4,8 stays inside the group)
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) part = (int64_t)((uint64_t)part + (uint64_t)__shfl_xor(part, o, 64));
  if ((lane & 15) == 0) totals[t * nbp + blk] = part;
  if (lane == 0) lslab[t * nslabs + sl] = L;
  for (int l = 0; l < L; ++l) {
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int64_t dig = ((v[q] + 128) & 255) - 128;          // balanced digit in [-128, 127]
      v[q] = (int64_t)(((uint64_t)v[q] - (uint64_t)dig)) >> 8;  // exact: v - dig is a multiple of 256
      const uint32_t byte = (uint32_t)(dig & 0xFF) << (8 * (q & 3));
      if (q < 4) w0 |= byte; else w1 |= byte;
    }
    uint32_t* dst = xq + ((((t * kMaxLimbs + l) * nbp + blk) * 8 + s) * 4);
    dst[2 * dh] = w0;
    dst[2 * dh + 1] = w1;
  }
}

// ------------------------------------------------------------------------------------------------------
// MFMA matvec / small-T linear. Grid: (ceil(ntiles / R), token chunks of Tc). Block: W waves; wave w handles
// slabs w, w + W, ... of each of the workgroup's R tiles. The per-row partial sums of the waves meet in an
// LDS int64 accumulator (ds_add_u64; integer addition is order-free, so the result is deterministic).
// The A operands (digit table) are read from the L2-resident xq table by the 16 active lanes only.
// ------------------------------------------------------------------------------------------------------
template <bool S64>
__global__ __launch_bounds__(1024) void q1_gemv_mfma_kernel(
    const uint4* __restrict__ bitsT, const void* __restrict__ scaleT, const uint4* __restrict__ xq,
    const int64_t* __restrict__ totals, const int* __restrict__ lslab, int64_t N, int64_t ntiles,
    int64_t nslabs, int64_t nbp, int T, int Tc, int R, int frac, int64_t* __restrict__ out) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int W = blockDim.x >> 6;
  const int64_t tile0 = (int64_t)blockIdx.x * R;
  const int t0 = blockIdx.y * Tc;
  const int tn = min(Tc, T - t0);

  uint64_t* acc = (uint64_t*)smem;                           // [tn][R*16]
  for (int i = threadIdx.x; i < tn * R * 16; i += blockDim.x) acc[i] = 0;
  __syncthreads();

  const int g = lane >> 4;       // block within slab (B / epilogue view); shift group in the D view
  const int n = lane & 15;       // output row within the tile
  // A-operand activity: lane (m = n, grp = g) carries digits for MFMA shift s iff m == grp + 4 * (s & 3).
  const int arow = n - g;
  const bool aact = arow >= 0 && (arow & 3) == 0;
  const int as = arow >> 2;      // the s & 3 this lane is active for
  const int hi = (g >> 1) & 1, lo = g & 1;

  v4i areg[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) areg[s] = v4i{0, 0, 0, 0};

  for (int r = 0; r < R; ++r) {
    const int64_t tile = tile0 + r;
    if (tile >= ntiles) break;
    for (int64_t sl = wave; sl < nslabs; sl += W) {
      const int64_t idx = (tile * nslabs + sl) * 64 + lane;
      const uint4 wb = bitsT[idx];
      int64_t sc;
      if (S64) sc = ((const int64_t*)scaleT)[idx];
      else sc = ((const int32_t*)scaleT)[idx];
      v4i bq[8];
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const uint32_t m = 0x01010101u << s;
        bq[s] = v4i{(int)(wb.x & m), (int)(wb.y & m), (int)(wb.z & m), (int)(wb.w & m)};
      }
      for (int t = 0; t < tn; ++t) {
        const int L = lslab[(t0 + t) * nslabs + sl];
        const uint4* xt = xq + ((int64_t)(t0 + t) * kMaxLimbs * nbp + sl * kSlabBlocks + g) * 8;
        const int64_t total = totals[(int64_t)(t0 + t) * nbp + sl * kSlabBlocks + g];
        uint64_t pos = 0;
        for (int l = 0; l < L; ++l) {
          // masked loads: only the lanes active for shift s write areg[s]; the others keep zeros
#pragma unroll
          for (int s = 0; s < 8; ++s) {
            if (aact && as == (s & 3)) {
              const uint4 a = xt[(int64_t)l * nbp * 8 + s];
              areg[s] = v4i{(int)a.x, (int)a.y, (int)a.z, (int)a.w};
            }
          }
          v4i d0 = {0, 0, 0, 0}, d1 = {0, 0, 0, 0};
#pragma unroll
          for (int s = 0; s < 4; ++s) d0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(areg[s], bq[s], d0, 0, 0, 0);
#pragma unroll
          for (int s = 4; s < 8; ++s) d1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(areg[s], bq[s], d1, 0, 0, 0);
          // lane (g = shift group, n): v_r = partial of block r over shifts g and g+4 (shift 7 reads -128)
          int v[4];
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const int hiv = d1[rr] >> (g + 4);
            v[rr] = (d0[rr] >> g) + (g == 3 ? -hiv : hiv);
          }
          // reduce-scatter over the 4 lane groups: group g ends with block g
          const int send0 = hi ? v[0] : v[2], send1 = hi ? v[1] : v[3];
          const int keep0 = hi ? v[2] : v[0], keep1 = hi ? v[3] : v[1];
          const int u0 = keep0 + __shfl_xor(send0, 32, 64);
          const int u1 = keep1 + __shfl_xor(send1, 32, 64);
          const int sendq = lo ? u0 : u1, keepq = lo ? u1 : u0;
          const int p = keepq + __shfl_xor(sendq, 16, 64);
          pos += (uint64_t)(int64_t)p << (8 * l);
        }
        const uint64_t S = 2u * pos - (uint64_t)total;
        const int64_t prod = (int64_t)(S * (uint64_t)sc);
        const int64_t term = imie_floor_shift(prod, frac);
        atomicAdd((unsigned long long*)&acc[(t * R + r) * 16 + n], (unsigned long long)term);
      }
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < tn * R * 16; i += blockDim.x) {
    const int t = i / (R * 16), rem = i % (R * 16);
    const int64_t row = (tile0 + rem / 16) * kTileRows + (rem % 16);
    if (row < N) out[(int64_t)(t0 + t) * N + row] = (int64_t)acc[i];
  }
}

// Straightforward exact kernel (thread per output): used for shapes the MFMA path declines and as an
// in-library cross-check. Reads the natural (N, nb, 16) layout.
__global__ void q1_linear_simple_kernel(const int64_t* __restrict__ x, const uint8_t* __restrict__ bits,
                                        const int64_t* __restrict__ scale, int64_t T, int64_t N, int64_t nb,
                                        int frac, int64_t* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= T * N) return;
  const int64_t t = idx / N, o = idx % N;
  const int64_t* xr = x + t * nb * 128;
  uint64_t tot = 0;
  for (int64_t b = 0; b < nb; ++b) {
    const uint8_t* bb = bits + (o * nb + b) * 16;
    uint64_t acc = 0;
    for (int j = 0; j < 16; ++j) {
      const uint32_t by = bb[j];
      for (int i = 0; i < 8; ++i) {
        const uint64_t xv = (uint64_t)xr[b * 128 + 8 * j + i];
        acc += ((by >> i) & 1u) ? xv : (uint64_t)0 - xv;
      }
    }
    const int64_t prod = (int64_t)(acc * (uint64_t)scale[o * nb + b]);
    tot += (uint64_t)imie_floor_shift(prod, frac);
  }
  out[idx] = (int64_t)tot;
}

// ------------------------------------------------------------------------------------------------------
// Launch helpers
// ------------------------------------------------------------------------------------------------------
static int q1_apply_dev(const Q1Weight& w, const int64_t* x_dev, int64_t T, int64_t frac, int64_t* out_dev,
                        hipStream_t st) {
  if (T <= 0) return IMIE_OK;
  const int64_t nbp = w.nslabs * kSlabBlocks;
  if (g_ws.xq.ensure((size_t)T * kMaxLimbs * nbp * 8 * 16) || g_ws.totals.ensure((size_t)T * nbp * 8) ||
      g_ws.lslab.ensure((size_t)T * w.nslabs * 4))
    return IMIE_EARG;
  const int64_t K = w.nb * 128;
  hipLaunchKernelGGL(q1_prep_kernel, dim3((unsigned)w.nslabs, (unsigned)T), dim3(64), 0, st, x_dev, K, w.nb, nbp,
                     w.nslabs, (uint32_t*)g_ws.xq.p, (int64_t*)g_ws.totals.p, (int*)g_ws.lslab.p);
  IMIE_HIP(hipGetLastError());
  int W = (int)(w.nslabs < 16 ? w.nslabs : 16);
  int R = (int)(w.ntiles / 1024);
  R = R < 1 ? 1 : (R > 8 ? 8 : R);
  int Tc = (int)(T < 4 ? T : 4);
  const int fr = (int)(frac > 63 ? 63 : frac);
  const dim3 grid((unsigned)((w.ntiles + R - 1) / R), (unsigned)((T + Tc - 1) / Tc));
  const size_t lds = (size_t)Tc * R * 16 * 8;
  if (w.scale64)
    hipLaunchKernelGGL(q1_gemv_mfma_kernel<true>, grid, dim3(64 * W), lds, st, w.bits, w.scale,
                       (const uint4*)g_ws.xq.p, (const int64_t*)g_ws.totals.p, (const int*)g_ws.lslab.p, w.N,
                       w.ntiles, w.nslabs, nbp, (int)T, Tc, R, fr, out_dev);
  else
    hipLaunchKernelGGL(q1_gemv_mfma_kernel<false>, grid, dim3(64 * W), lds, st, w.bits, w.scale,
                       (const uint4*)g_ws.xq.p, (const int64_t*)g_ws.totals.p, (const int*)g_ws.lslab.p, w.N,
                       w.ntiles, w.nslabs, nbp, (int)T, Tc, R, fr, out_dev);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

static int64_t q1_register(const uint8_t* bits, const void* scale, int64_t N, int64_t nb, int src32) {
  if (!bits || !scale || N <= 0 || nb <= 0 || imie_device_ready() != 0) return -1;
  // narrow the scales to int32 when every value fits (lossless); keep int64 otherwise
  int scale64 = 0;
  std::vector<int64_t> s64((size_t)(N * nb));
  for (int64_t i = 0; i < N * nb; ++i) {
    const int64_t v = src32 ? (int64_t)((const int32_t*)scale)[i] : ((const int64_t*)scale)[i];
    s64[(size_t)i] = v;
    if (v < INT32_MIN || v > INT32_MAX) scale64 = 1;
  }
  Q1Weight w;
  w.N = N;
  w.nb = nb;
  w.ntiles = (N + kTileRows - 1) / kTileRows;
  w.nslabs = (nb + kSlabBlocks - 1) / kSlabBlocks;
  const size_t nlanes = (size_t)(w.ntiles * w.nslabs * 64);
  std::vector<uint8_t> hb(nlanes * 16);
  std::vector<uint8_t> hs(nlanes * (scale64 ? 8 : 4));
  imie_q1_repack_host(bits, s64.data(), N, nb, scale64, hb.data(), hs.data());
  if (hipMalloc((void**)&w.bits, hb.size()) != hipSuccess) return -1;
  if (hipMalloc(&w.scale, hs.size()) != hipSuccess) { (void)hipFree(w.bits); return -1; }
  if (hipMemcpy(w.bits, hb.data(), hb.size(), hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(w.scale, hs.data(), hs.size(), hipMemcpyHostToDevice) != hipSuccess) {
    (void)hipFree(w.bits); (void)hipFree(w.scale); return -1;
  }
  w.scale64 = scale64;
  w.bytes = hb.size() + hs.size();
  w.live = true;
  g_resident_bytes += w.bytes;
  registry().push_back(w);
  return (int64_t)registry().size() - 1;
}

static const Q1Weight* q1_get(int64_t h) {
  if (h < 0 || h >= (int64_t)registry().size() || !registry()[(size_t)h].live) return nullptr;
  return &registry()[(size_t)h];
}

static int q1_host_apply(const Q1Weight& w, const int64_t* x, int64_t T, int64_t frac, int64_t* out) {
  hipStream_t st = imie_stream();
  const size_t xb = (size_t)(T * w.nb * 128) * 8, ob = (size_t)(T * w.N) * 8;
  if (g_ws.x.ensure(xb) || g_ws.out.ensure(ob)) return IMIE_EARG;
  IMIE_HIP(hipMemcpyAsync(g_ws.x.p, x, xb, hipMemcpyHostToDevice, st));
  int rc = q1_apply_dev(w, (const int64_t*)g_ws.x.p, T, frac, (int64_t*)g_ws.out.p, st);
  if (rc) return rc;
  IMIE_HIP(hipMemcpyAsync(out, g_ws.out.p, ob, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipStreamSynchronize(st));
  return IMIE_OK;
}

extern "C" {

// bonsai_q1_gpu.cu:1968-2241 `bonsai_q1_linear_gpu`: per-call upload of weight + x, synchronous.
int bonsai_q1_linear_gpu(const int64_t* x, const uint8_t* bits, const int64_t* scale, int64_t tokens,
                         int64_t out_features, int64_t n_blocks, int64_t frac, int64_t* out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!x || !bits || !scale || !out || tokens < 0 || out_features <= 0 || n_blocks <= 0 || frac < 0) return IMIE_EARG;
  if (tokens == 0) return IMIE_OK;
  const int64_t h = q1_register(bits, scale, out_features, n_blocks, 0);
  if (h < 0) return IMIE_EARG;
  const int rc = q1_host_apply(registry()[(size_t)h], x, tokens, frac, out);
  Q1Weight& w = registry()[(size_t)h];
  (void)hipFree(w.bits); (void)hipFree(w.scale);
  g_resident_bytes -= w.bytes;
  w.live = false;
  if (h == (int64_t)registry().size() - 1) registry().pop_back();
  return rc;
}

// bonsai_q1_gpu.cu `bonsai_q1_register_weight`: handle >= 0, or -1.
int64_t bonsai_q1_register_weight(const uint8_t* bits, const int64_t* scale, int64_t out_features, int64_t n_blocks) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  return q1_register(bits, scale, out_features, n_blocks, 0);
}

// int32-scale registration (bonsai_q1_gpu.cu `bonsai_q1_register_weight_i32`).
int64_t bonsai_q1_register_weight_i32(const uint8_t* bits, const int32_t* scale, int64_t out_features,
                                      int64_t n_blocks) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  return q1_register(bits, scale, out_features, n_blocks, 1);
}

// bonsai_q1_gpu.cu:2388-2423 `bonsai_q1_apply_resident`: host x in, host out, synchronous.
int bonsai_q1_apply_resident(int64_t handle, const int64_t* x, int64_t tokens, int64_t frac, int64_t* out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  const Q1Weight* w = q1_get(handle);
  if (!w || !x || !out || tokens < 0 || frac < 0) return IMIE_EARG;
  if (tokens == 0) return IMIE_OK;
  return q1_host_apply(*w, x, tokens, frac, out);
}

void bonsai_q1_free_weights(void) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  (void)hipStreamSynchronize(imie_stream());
  for (auto& w : registry())
    if (w.live) { (void)hipFree(w.bits); (void)hipFree(w.scale); }
  registry().clear();
  g_resident_bytes = 0;
}

uint64_t bonsai_q1_resident_weight_bytes(void) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  return g_resident_bytes;
}

// Device-resident apply (no reference counterpart; used by the resident pipelines and the benchmark):
// x_dev (T, nb*128) int64 and out_dev (T, N) int64 are device pointers, enqueued on `stream` (nullptr =
// library stream). Asynchronous. Returns 1 on a bad handle.
int imie_q1_apply_dev(int64_t handle, const int64_t* x_dev, int64_t tokens, int64_t frac, int64_t* out_dev,
                      void* stream) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  const Q1Weight* w = q1_get(handle);
  if (!w || !x_dev || !out_dev || tokens < 0 || frac < 0) return IMIE_EARG;
  return q1_apply_dev(*w, x_dev, tokens, frac, out_dev, stream ? (hipStream_t)stream : imie_stream());
}

// Weight geometry of a handle: out_features, n_blocks, scale width in bytes (4 or 8).
int imie_q1_weight_info(int64_t handle, int64_t* out_features, int64_t* n_blocks, int64_t* scale_bytes) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  const Q1Weight* w = q1_get(handle);
  if (!w || !out_features || !n_blocks || !scale_bytes) return IMIE_EARG;
  *out_features = w->N;
  *n_blocks = w->nb;
  *scale_bytes = w->scale64 ? 8 : 4;
  return IMIE_OK;
}

// Exact simple kernel over caller device buffers in the natural layout (cross-check path).
int imie_q1_linear_simple_dev(const int64_t* x_dev, const uint8_t* bits_dev, const int64_t* scale_dev,
                              int64_t tokens, int64_t out_features, int64_t n_blocks, int64_t frac,
                              int64_t* out_dev, void* stream) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!x_dev || !bits_dev || !scale_dev || !out_dev || tokens < 0 || frac < 0) return IMIE_EARG;
  const int64_t n = tokens * out_features;
  if (n == 0) return IMIE_OK;
  hipStream_t st = stream ? (hipStream_t)stream : imie_stream();
  hipLaunchKernelGGL(q1_linear_simple_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x_dev,
                     bits_dev, scale_dev, tokens, out_features, n_blocks, (int)(frac > 63 ? 63 : frac), out_dev);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

}  // extern "C"
