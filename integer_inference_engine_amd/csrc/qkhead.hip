// Fused per-head stage of the Bonsai layer, between the q/k/v projections and the attention:
//   q, k <- head RMSNorm (gain qng / kng)              reference_bonsai.py:286-297 (_head_rmsnorm)
//   q, k <- NeoX RoPE at the row's position            rope_v2.py:92-117, guard rope.py:26-39
//   cache <- (k, v) at that position (int64 rows, or the kv8 digit planes with their envelope guard)
// One 64-lane workgroup per (row, head); lane j owns the rotation pair (j, j + hd/2). The per-head RMSNorm
// follows the whole-row kernel's exact arithmetic (shared helpers); the RoPE envelope
// 2 * max|x| * max|cos, sin| <= INT64_MAX is evaluated over the whole q (and k) tensor through atomic maxima in
// `guard` (q: [0], [1]; k: [2], [3]) and checked by the attention's final kernel.
#include "imie_common.h"
#include "imie_kernels.h"
#include "imie_fixed.h"
#include "imie_kvfmt.h"
#include "imie_head.h"

namespace {

using namespace imie_fx;

__device__ inline void amax_u64(uint64_t* p, uint64_t v) { atomicMax((unsigned long long*)p, (unsigned long long)v); }

template <bool KV8>
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
  // everything else this workgroup reads is requested before the norm's arithmetic: the RoPE entries of the
  // row's position, and for a key head its V row and page
  const int64_t p = a.pos[r];
  const int64_t c = act ? a.cos[p * half + j] : 0, s = act ? a.sin[p * half + j] : 0;
  const int64_t kvh = h - a.H, b = r / a.M;
  int64_t v0 = 0, v1 = 0, pg = 0, slot = 0;
  if (!isq) {
    const uint32_t pq = (uint32_t)p / (uint32_t)a.P;            // positions are below 2^31
    pg = a.pt[b * a.mp + pq];
    slot = (uint32_t)p - pq * (uint32_t)a.P;
    const int64_t* vr = a.v + (r * a.Hkv + kvh) * a.hd;
    v0 = act ? vr[j] : 0;
    v1 = act ? vr[j + half] : 0;
  }
  int64_t o0, o1;
  uint64_t mx, mc;
  if (!imie_head::head_norm_rope(x0, x1, g0, g1, c, s, act, a.hd, a.frac, a.eps, o0, o1, mx, mc)) {
    if (j == 0) atomicOr(a.status, IMIE_ERMS);
    if (j == 0 && a.gpart) { a.gpart[(r * (a.H + a.Hkv) + h) * 2] = 0; a.gpart[(r * (a.H + a.Hkv) + h) * 2 + 1] = 0; }
    return;
  }
  if (j == 0) {
    if (a.gpart) {
      uint64_t* gp = a.gpart + (r * (a.H + a.Hkv) + h) * 2;
      gp[0] = mx;
      gp[1] = mc;
    } else {
      amax_u64(&a.guard[isq ? 0 : 2], mx);
      amax_u64(&a.guard[isq ? 1 : 3], mc);
    }
  }
  if (isq) {
    if (act) {
      a.qo[(r * a.H + h) * a.hd + j] = o0;
      a.qo[(r * a.H + h) * a.hd + j + half] = o1;
    }
    if (a.qd) {                                       // kv8 decode: q digits (8 limbs), max|q| and limb count
      uint64_t mq = imie_absu64(o0) > imie_absu64(o1) ? imie_absu64(o0) : imie_absu64(o1);
      mq = imie_wave_max_u64_full(mq);
      const int64_t qrow = r * a.H + h;
      if (j == 0) { a.qmax[qrow] = mq; a.qlimbs[qrow] = imie_limbs_needed(mq); }
      if (act) {
        int8_t* dst = a.qd + qrow * 8 * a.hd;
        int64_t x0 = o0, x1 = o1;
        for (int lq = 0; lq < 8; ++lq) {
          const int64_t d0 = ((x0 + 128) & 255) - 128, d1 = ((x1 + 128) & 255) - 128;
          x0 = (int64_t)((uint64_t)x0 - (uint64_t)d0) >> 8;
          x1 = (int64_t)((uint64_t)x1 - (uint64_t)d1) >> 8;
          dst[lq * a.hd + j] = (int8_t)d0;
          dst[lq * a.hd + j + half] = (int8_t)d1;
        }
      }
    }
    return;
  }
  if (KV8) {
    uint64_t mk = imie_absu64(o0) > imie_absu64(o1) ? imie_absu64(o0) : imie_absu64(o1);
    uint64_t mv = imie_absu64(v0) > imie_absu64(v1) ? imie_absu64(v0) : imie_absu64(v1);
    mk = imie_wave_max_u64_full(mk);
    mv = imie_wave_max_u64_full(mv);
    if (j == 0) {
      if (mk > (uint64_t)imie_kv8::kCap || mv > (uint64_t)imie_kv8::kCap) atomicOr(a.status, IMIE_EOVF);
      if (a.M == 1) {
        amax_u64(&a.run_k[b * a.Hkv + kvh], mk);
        amax_u64(&a.run_v[b * a.Hkv + kvh], mv);
      } else {
        a.rowk[r * a.Hkv + kvh] = mk;
        a.rowv[r * a.Hkv + kvh] = mv;
      }
    }
    if (!act) return;
    int8_t* blk = (int8_t*)a.kpool + imie_kv8::block_base(pg, kvh, a.Hkv, a.hd, a.P);
    // an element beyond the format's range is stored as 0 (its row is refused through the status bit above),
    // never as the digits of a wrapped value
    const uint32_t wk0 = imie_kv8::encode(imie_kv8::fits(o0) ? o0 : 0);
    const uint32_t wk1 = imie_kv8::encode(imie_kv8::fits(o1) ? o1 : 0);
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      blk[imie_kv8::k_off(slot, db, j, a.hd)] = (int8_t)(wk0 >> (8 * db));
      blk[imie_kv8::k_off(slot, db, j + half, a.hd)] = (int8_t)(wk1 >> (8 * db));
    }
    if (a.M > 1) return;                              // V planes: kv8_v_append_kernel (coalesced over slots)
    int8_t* vblk = (int8_t*)a.vpool + imie_kv8::block_base(pg, kvh, a.Hkv, a.hd, a.P);
    const uint32_t wv0 = imie_kv8::encode(imie_kv8::fits(v0) ? v0 : 0);
    const uint32_t wv1 = imie_kv8::encode(imie_kv8::fits(v1) ? v1 : 0);
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      vblk[imie_kv8::v_off(slot, db, j, a.hd, a.P)] = (int8_t)(wv0 >> (8 * db));
      vblk[imie_kv8::v_off(slot, db, j + half, a.hd, a.P)] = (int8_t)(wv1 >> (8 * db));
    }
    return;
  }
  if (!act) return;
  const int64_t off = pg * (a.Hkv * a.P * a.hd) + kvh * a.P * a.hd + slot * a.hd;
  int64_t* kp = (int64_t*)a.kpool + off;
  int64_t* vp = (int64_t*)a.vpool + off;
  kp[j] = o0;
  kp[j + half] = o1;
  vp[j] = v0;
  vp[j + half] = v1;
}

// RoPE envelope maxima of a many-row head stage: grid-stride max over the per-workgroup partials (256 threads),
// one atomic per workgroup and quantity
__global__ __launch_bounds__(256) void guard_reduce_kernel(const uint64_t* __restrict__ gpart, int64_t n, int64_t H,
                                                           int64_t heads, uint64_t* __restrict__ guard) {
  uint64_t m[4] = {0, 0, 0, 0};
  // n < 2^32 (rows x heads); unrolled so that several iterations' loads are in flight together
#pragma unroll 8
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int k = imie_umod32(e, heads) < H ? 0 : 2;
    const uint64_t a = gpart[2 * e], c = gpart[2 * e + 1];
    if (k == 0) { m[0] = a > m[0] ? a : m[0]; m[1] = c > m[1] ? c : m[1]; }
    else { m[2] = a > m[2] ? a : m[2]; m[3] = c > m[3] ? c : m[3]; }
  }
  // workgroup maxima through LDS, then one atomic per quantity and workgroup (same-address atomics from every
  // wave serialise across the XCDs)
  __shared__ uint64_t s_m[4][4];
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint64_t v = imie_wave_max_u64_full(m[i]);
    if ((threadIdx.x & 63) == 0) s_m[wave][i] = v;
  }
  __syncthreads();
  if (threadIdx.x < 4) {
    uint64_t v = s_m[0][threadIdx.x];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) v = s_m[w][threadIdx.x] > v ? s_m[w][threadIdx.x] : v;
    if (v != 0) amax_u64(&guard[threadIdx.x], v);
  }
}

// kv8 V append of many rows: workgroup = (64 consecutive new positions of sequence b, kv head). The rows'
// digits are transposed through LDS to the cache's [digit][dim][slot] order, so each store instruction writes
// 64 consecutive slots. Each thread's 32 V elements (element tid + 256 k of the 64 x hd tile) are requested in
// one round before any is encoded. The workgroup also folds its rows' max|K| / max|V| into the running maxima.
__global__ __launch_bounds__(256) void kv8_v_append_kernel(QkHeadArgs a) {
  // rows padded from 64 to 68 bytes: the byte writes of 64 consecutive dims (stride one row) then fall in 64
  // distinct banks (at 64 bytes they shared 4)
  __shared__ int8_t sv[4][128][68];
  const int64_t bkv = blockIdx.y, b = imie_udiv32(bkv, a.Hkv), kvh = imie_umod32(bkv, a.Hkv);
  const int64_t m0 = (int64_t)blockIdx.x * 64;
  const int tid = threadIdx.x;
  const int hd = (int)a.hd;                           // <= 128: 64 * hd <= 32 * 256 elements
  // lane's position (slot of the store phase), requested with the V loads
  const int lane = tid & 63, wave = tid >> 6;
  const int64_t m = m0 + lane;
  const bool live = m < a.M;
  int64_t pg = 0, slot = 0;
  uint64_t rk = 0, rv = 0;                            // the rows' max|K|, max|V| (head stage), for run_k / run_v
  if (live) {
    if (wave == 0) { rk = a.rowk[(b * a.M + m) * a.Hkv + kvh]; rv = a.rowv[(b * a.M + m) * a.Hkv + kvh]; }
    const int64_t p = a.pos[b * a.M + m];
    const uint32_t pq = (uint32_t)p / (uint32_t)a.P;
    pg = a.pt[b * a.mp + pq];
    slot = (uint32_t)p - pq * (uint32_t)a.P;
  }
  int64_t vv[32];
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    const int i = tid + 256 * k;
    const int ml = (int)((uint32_t)i / (uint32_t)hd), c = i - ml * hd;
    const int64_t m = m0 + ml;
    vv[k] = (ml < 64 && m < a.M) ? a.v[((b * a.M + m) * a.Hkv + kvh) * hd + c] : 0;
  }
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    const int i = tid + 256 * k;
    const int ml = (int)((uint32_t)i / (uint32_t)hd), c = i - ml * hd;
    if (ml >= 64) break;
    const uint32_t w = imie_kv8::encode(imie_kv8::fits(vv[k]) ? vv[k] : 0);   // out-of-range rows: flagged upstream
#pragma unroll
    for (int db = 0; db < 4; ++db) sv[db][c][ml] = (int8_t)(w >> (8 * db));
  }
  if (wave == 0) {                                   // running maxima of the cache (one atomic per quantity)
    rk = imie_wave_max_u64_full(rk);
    rv = imie_wave_max_u64_full(rv);
    if (lane == 0) { amax_u64(&a.run_k[bkv], rk); amax_u64(&a.run_v[bkv], rv); }
  }
  __syncthreads();
  if (!live) return;
  int8_t* vblk = (int8_t*)a.vpool + imie_kv8::block_base(pg, kvh, a.Hkv, a.hd, a.P);
  for (int e = wave; e < 4 * hd; e += 4) {
    const int db = (int)((uint32_t)e / (uint32_t)hd), c = e - db * hd;
    vblk[imie_kv8::v_off(slot, db, c, a.hd, a.P)] = sv[db][c][lane];
  }
}

}  // namespace

int imie_qk_head_launch(const QkHeadArgs& a, int kv8, hipStream_t st) {
  const int64_t rows = a.rows;
  if (rows <= 0) return IMIE_OK;
  if (a.hd > 128 || (a.hd & 1) || a.hd <= 0) return IMIE_EARG;
  if (kv8 && (!a.run_k || !a.run_v || (a.M > 1 && (!a.rowk || !a.rowv)))) return IMIE_EARG;
  const dim3 grid((unsigned)rows, (unsigned)(a.H + a.Hkv));
  if (kv8) hipLaunchKernelGGL(qk_head_kernel<true>, grid, dim3(64), 0, st, a);
  else hipLaunchKernelGGL(qk_head_kernel<false>, grid, dim3(64), 0, st, a);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

int imie_qk_head_finish_launch(const QkHeadArgs& a, int kv8, hipStream_t st) {
  if (!a.gpart || a.rows <= 0) return IMIE_OK;
  const int64_t heads = a.H + a.Hkv, n = a.rows * heads;
  const unsigned g = (unsigned)((n + 255) / 256 < 64 ? (n + 255) / 256 : 64);
  hipLaunchKernelGGL(guard_reduce_kernel, dim3(g), dim3(256), 0, st, a.gpart, n, a.H, heads, a.guard);
  IMIE_HIP(hipGetLastError());
  if (kv8 && a.M > 1) {
    if (a.hd > 128) return IMIE_EARG;
    const dim3 grid((unsigned)((a.M + 63) / 64), (unsigned)(a.rows / a.M * a.Hkv));
    hipLaunchKernelGGL(kv8_v_append_kernel, grid, dim3(256), 0, st, a);
    IMIE_HIP(hipGetLastError());
  }
  return IMIE_OK;
}
