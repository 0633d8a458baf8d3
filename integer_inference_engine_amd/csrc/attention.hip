// Fixed-point attention for gfx950.
//
// Semantics (reference: bonsai/src/trinote/infer_int/reference_bonsai.py:656-720 numpy path, producers
// bonsai/tools/bonsai_q1_kernel.c:1244-1717):
//   s_j   = (((q . k_j) >> f) * inv_sqrt) >> f               (int64 wrap)
//   e_j   = 2^-(((min(m - s_j, d_clip)) * log2e) >> f)       (cubic polynomial, fixedpoint.py:74-96)
//   p_j   = (e_j << f) // Z,  Z = sum e_j  (Z == 0 -> p = 0)
//   out_d = (sum_j p_j * v_j[d]) >> f
// over the keys a query row may see (causal: j <= start + m; decode: j < length). Keys past the causal limit
// contribute exactly 0 in the oracle's masked softmax, so only visible keys are visited. Fail-loud bounds
// (status bit 2): max|q_row| * max|K| > INT64_MAX / hd, or max|p_row| * max|V| > INT64_MAX / Lv — the producer
// rule of bonsai_q1_kernel.c:1466-1500 (per query row; max|K|, max|V| over the sequence's cached keys).
//
// Structure (integer sums are order-free, so a split over key tiles is exact):
//   1 scores  : WG = (b, kv head, 16-row tile, 64-key tile); q and K tiles staged in LDS; row max by atomicMax
//   2 softmax : WG per row; e_j, Z (exact u64), p_j in place; max|p_row|; QK bound check
//   3 PV      : WG = (b, kv, row tile, key tile); sum_j p_j v_j[d] added into an int64 accumulator atomically
//   4 final   : out = acc >> f; PV bound check
// KV addressing is paged: key j of (b, kv) lives at pool + pt[b * mp + j / P] * (Hkv * P * hd) + kv * P * hd +
// (j % P) * hd; a dense (B, Hkv, cap, hd) cache is the special case P = cap, mp = 1, pt[b] = b.
#include "imie_common.h"
#include "imie_kernels.h"
#include "imie_attention.h"
#include "imie_kvfmt.h"
#include "imie_silu.h"
#include <stdlib.h>

namespace {

typedef unsigned __int128 u128;
constexpr int kRowTile = 16;
constexpr int kKeyTile = 32;   // keeps every kernel's LDS under 64 KB

using imie_silu::exp2_neg_fixed;
using imie_silu::exp_clipped;
using imie_silu::prob_div;

__device__ inline void amax_u64(uint64_t* p, uint64_t v) { atomicMax((unsigned long long*)p, (unsigned long long)v); }
__device__ inline void amax_i64(int64_t* p, int64_t v) { atomicMax((long long*)p, (long long)v); }

// RoPE envelope of the fused head stage: 2 * max|x| * max|cos, sin| <= INT64_MAX for q ([0], [1]) and k
// ([2], [3]) (rope.py:26-39)
__device__ inline void check_rope_guard(const AttnDesc& d) {
  if (!d.rope_guard) return;
  for (int t = 0; t < 2; ++t) {
    const u128 b = (u128)2 * d.rope_guard[2 * t] * d.rope_guard[2 * t + 1];
    if (b > (u128)INT64_MAX) atomicOr(d.status, IMIE_EOVF);
  }
}

struct RowInfo {
  int64_t b, h, m, kv, lv, len;   // len = keys cached for (b): the max|K|/max|V| range
};

__device__ inline RowInfo row_info(const AttnDesc& d, int64_t r) {
  RowInfo ri;
  ri.m = imie_umod32(r, d.M);
  ri.h = imie_umod32(imie_udiv32(r, d.M), d.H);
  ri.b = imie_udiv32(r, d.M * d.H);
  ri.kv = imie_udiv32(ri.h, d.H / d.Hkv);
  if (d.starts) {
    ri.lv = d.starts[ri.b] + ri.m + 1;
    ri.len = d.starts[ri.b] + d.M;
  } else {
    ri.lv = d.lengths[ri.b];
    ri.len = ri.lv;
  }
  return ri;
}

// Page id of page pi of sequence b for a wave-uniform (b, pi), read through the constant address space: the page
// table is not written during an attention launch, so the load is a scalar one (its own counter). A vector load
// of it would be counted with the K / V loads in flight, and the wait for it (the address of the next loads
// depends on it) would wait for all of them.
__device__ inline int64_t page_id_uniform(const AttnDesc& d, int64_t b, int64_t pi) {
  // the address through readfirstlane: kept in scalar registers even where the compiler had moved it to vector
  // ones (a vector address makes the load a vector one)
  const uint64_t a = (uint64_t)(d.pt + b * d.mp + pi);
  const uint64_t u = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a) |
                     ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32)) << 32);
  return *(const __attribute__((address_space(4))) int64_t*)u;
}

// key j -> (page index within the sequence, slot in the page); positions are below 2^31
__device__ inline void page_split(const AttnDesc& d, int64_t j, int64_t& pi, int64_t& in) {
  if (d.pshift >= 0) {
    pi = j >> d.pshift;
    in = j & ((int64_t)1 << d.pshift) - 1;
  } else {
    const uint32_t jj = (uint32_t)j, P = (uint32_t)d.P, q = jj / P;
    pi = q;
    in = jj - q * P;
  }
}

template <typename KT>
__device__ inline const KT* key_ptr(const AttnDesc& d, const void* pool, int64_t b, int64_t kv, int64_t j) {
  int64_t pi, in;
  page_split(d, j, pi, in);
  const int64_t pg = d.pt[b * d.mp + pi];
  return (const KT*)pool + pg * (d.Hkv * d.P * d.hd) + kv * d.P * d.hd + in * d.hd;
}

// rows of one (b, kv) group are ordered h-major: row index within the group g = (h - kv*rep) * M + m.
__device__ inline int64_t group_row(const AttnDesc& d, int64_t b, int64_t kv, int64_t gr) {
  const int64_t rep = d.H / d.Hkv;
  const int64_t hh = imie_udiv32(gr, d.M), m = imie_umod32(gr, d.M);
  return (b * d.H + kv * rep + hh) * d.M + m;
}

// element offset of query row r = ((b * H) + h) * M + m
__device__ inline int64_t qoff(const AttnDesc& d, int64_t r) {
  const int64_t m = imie_umod32(r, d.M), h = imie_umod32(imie_udiv32(r, d.M), d.H), b = imie_udiv32(r, d.M * d.H);
  return b * d.qsb + h * d.qsh + m * d.qsm;
}

template <typename KT>
__global__ __launch_bounds__(256) void attn_scores_kernel(AttnDesc d) {
  __shared__ int64_t sq[kRowTile][129];
  __shared__ int64_t sk[kKeyTile][129];
  const int64_t rep = d.H / d.Hkv;
  const int64_t grows = rep * d.M;
  const int64_t nrt = (grows + kRowTile - 1) / kRowTile;
  const int64_t bkv = blockIdx.x / nrt, rt = blockIdx.x % nrt;
  const int64_t b = imie_udiv32(bkv, d.Hkv), kv = imie_umod32(bkv, d.Hkv);
  const int64_t j0 = (int64_t)blockIdx.y * kKeyTile;
  const int64_t len = d.starts ? d.starts[b] + d.M : d.lengths[b];
  if (j0 >= len) return;
  // largest visible key of this row tile (causal: rows are h-major, so take the max m in the tile)
  int64_t vis = len;
  if (d.starts) {
    int64_t mmax = -1;
    for (int i = 0; i < kRowTile; ++i) {
      const int64_t gr = rt * kRowTile + i;
      if (gr < grows) mmax = max(mmax, imie_umod32(gr, d.M));
    }
    vis = d.starts[b] + mmax + 1;
  }
  if (j0 >= vis) return;
  const int tid = threadIdx.x;
  // stage q rows and the key tile; max|q| per row, max|K| over cached keys
  for (int i = tid; i < kRowTile * d.hd; i += blockDim.x) {
    const int ri = (int)imie_udiv32(i, d.hd), c = (int)imie_umod32(i, d.hd);
    const int64_t gr = rt * kRowTile + ri;
    sq[ri][c] = gr < grows ? d.q[qoff(d, group_row(d, b, kv, gr)) + c] : 0;
  }
  uint64_t mk = 0;
  for (int i = tid; i < kKeyTile * d.hd; i += blockDim.x) {
    const int ki = (int)imie_udiv32(i, d.hd), c = (int)imie_umod32(i, d.hd);
    const int64_t j = j0 + ki;
    int64_t v = 0;
    if (j < len) {
      v = (int64_t)key_ptr<KT>(d, d.K, b, kv, j)[c];
      const uint64_t a = imie_absu64(v);
      mk = a > mk ? a : mk;
    }
    sk[ki][c] = v;
  }
  mk = imie_wave_max_u64(mk);
  if ((tid & 63) == 0) amax_u64(&d.maxk[bkv], mk);
  __syncthreads();
  if (blockIdx.y == 0 && tid < kRowTile) {
    const int64_t gr = rt * kRowTile + tid;
    if (gr < grows) {
      uint64_t mq = 0;
      for (int c = 0; c < d.hd; ++c) {
        const uint64_t a = imie_absu64(sq[tid][c]);
        mq = a > mq ? a : mq;
      }
      d.maxq[group_row(d, b, kv, gr)] = mq;
    }
  }
  for (int pidx = tid; pidx < kRowTile * kKeyTile; pidx += blockDim.x) {
    const int ri = pidx / kKeyTile, ki = pidx % kKeyTile;
    const int64_t gr = rt * kRowTile + ri;
    const int64_t j = j0 + ki;
    if (gr >= grows) continue;
    const int64_t r = group_row(d, b, kv, gr);
    const int64_t lv = d.starts ? d.starts[b] + imie_umod32(gr, d.M) + 1 : len;
    if (j >= lv) continue;
    uint64_t dot = 0;
    for (int c = 0; c < d.hd; ++c) dot += (uint64_t)sq[ri][c] * (uint64_t)sk[ki][c];
    int64_t s = (int64_t)dot >> d.frac;
    s = (int64_t)((uint64_t)s * (uint64_t)d.inv_sqrt) >> d.frac;
    d.scores[r * d.Lmax + j] = s;
    amax_i64(&d.rowmax[r], s);
  }
}

__global__ __launch_bounds__(256) void attn_softmax_kernel(AttnDesc d) {
  __shared__ uint64_t red[256];
  const int64_t r = blockIdx.x;
  const RowInfo ri = row_info(d, r);
  const int tid = threadIdx.x;
  const int64_t bkv = ri.b * d.Hkv + ri.kv;
  if (tid == 0) {
    const u128 qk = (u128)d.maxq[r] * d.maxk[bkv];
    if (qk > (u128)(INT64_MAX / d.hd)) atomicOr(d.status, IMIE_EOVF);
  }
  const int64_t m = d.rowmax[r];
  int64_t* s = d.scores + r * d.Lmax;
  uint64_t z = 0;
  for (int64_t j = tid; j < ri.lv; j += blockDim.x) {
    int64_t dd = (int64_t)((uint64_t)m - (uint64_t)s[j]);
    if (dd > d.dclip) dd = d.dclip;
    const int64_t e = exp2_neg_fixed((int64_t)((uint64_t)dd * (uint64_t)d.log2e) >> d.frac, d.frac);
    s[j] = e;
    z += (uint64_t)e;
  }
  red[tid] = z;
  __syncthreads();
  for (int o = blockDim.x / 2; o > 0; o >>= 1) {
    if (tid < o) red[tid] += red[tid + o];
    __syncthreads();
  }
  const uint64_t Z = red[0];
  __syncthreads();
  uint64_t mp = 0;
  for (int64_t j = tid; j < ri.lv; j += blockDim.x) {
    const int64_t p = Z == 0 ? 0 : (int64_t)(((uint64_t)s[j] << d.frac) / Z);
    s[j] = p;
    mp = (uint64_t)p > mp ? (uint64_t)p : mp;
  }
  red[tid] = mp;
  __syncthreads();
  for (int o = blockDim.x / 2; o > 0; o >>= 1) {
    if (tid < o) red[tid] = red[tid] > red[tid + o] ? red[tid] : red[tid + o];
    __syncthreads();
  }
  if (tid == 0) d.maxp[r] = red[0];
}

template <typename KT>
__global__ __launch_bounds__(256) void attn_pv_kernel(AttnDesc d) {
  __shared__ int64_t sp[kRowTile][kKeyTile + 1];
  __shared__ int64_t sv[kKeyTile][129];
  const int64_t rep = d.H / d.Hkv;
  const int64_t grows = rep * d.M;
  const int64_t nrt = (grows + kRowTile - 1) / kRowTile;
  const int64_t bkv = blockIdx.x / nrt, rt = blockIdx.x % nrt;
  const int64_t b = imie_udiv32(bkv, d.Hkv), kv = imie_umod32(bkv, d.Hkv);
  const int64_t j0 = (int64_t)blockIdx.y * kKeyTile;
  const int64_t len = d.starts ? d.starts[b] + d.M : d.lengths[b];
  if (j0 >= len) return;
  const int tid = threadIdx.x;
  // max|V| over all cached keys (every key tile of the sequence is visited by row tile 0)
  uint64_t mv = 0;
  for (int i = tid; i < kKeyTile * d.hd; i += blockDim.x) {
    const int ki = (int)imie_udiv32(i, d.hd), c = (int)imie_umod32(i, d.hd);
    const int64_t j = j0 + ki;
    int64_t v = 0;
    if (j < len) {
      v = (int64_t)key_ptr<KT>(d, d.V, b, kv, j)[c];
      const uint64_t a = imie_absu64(v);
      mv = a > mv ? a : mv;
    }
    sv[ki][c] = v;
  }
  mv = imie_wave_max_u64(mv);
  if (rt == 0 && (tid & 63) == 0) amax_u64(&d.maxv[bkv], mv);
  int any = 0;
  for (int i = tid; i < kRowTile * kKeyTile; i += blockDim.x) {
    const int ri = i / kKeyTile, ki = i % kKeyTile;
    const int64_t gr = rt * kRowTile + ri;
    const int64_t j = j0 + ki;
    int64_t p = 0;
    if (gr < grows) {
      const int64_t lv = d.starts ? d.starts[b] + imie_umod32(gr, d.M) + 1 : len;
      if (j < lv) { p = d.scores[group_row(d, b, kv, gr) * d.Lmax + j]; any = 1; }
    }
    sp[ri][ki] = p;
  }
  if (!__syncthreads_or(any)) return;
  for (int i = tid; i < kRowTile * d.hd; i += blockDim.x) {
    const int ri = (int)imie_udiv32(i, d.hd), c = (int)imie_umod32(i, d.hd);
    const int64_t gr = rt * kRowTile + ri;
    if (gr >= grows) continue;
    uint64_t acc = 0;
    for (int k = 0; k < kKeyTile; ++k) acc += (uint64_t)sp[ri][k] * (uint64_t)sv[k][c];
    if (acc) atomicAdd((unsigned long long*)&d.acc[group_row(d, b, kv, gr) * d.hd + c], (unsigned long long)acc);
  }
}

__global__ void attn_final_kernel(AttnDesc d) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t rows = d.B * d.H * d.M;
  if (i >= rows * d.hd) return;
  const int64_t r = imie_udiv32(i, d.hd), c = imie_umod32(i, d.hd);
  if (i == 0) check_rope_guard(d);
  d.out[qoff(d, r) + c] = (int64_t)d.acc[i] >> d.frac;
  if (c == 0) {
    const RowInfo ri = row_info(d, r);
    const u128 pv = (u128)d.maxp[r] * d.maxv[ri.b * d.Hkv + ri.kv];
    if (pv > (u128)(INT64_MAX / ri.lv)) atomicOr(d.status, IMIE_EOVF);
    const u128 qk = (u128)d.maxq[r] * d.maxk[ri.b * d.Hkv + ri.kv];
    if (qk > (u128)(INT64_MAX / d.hd)) atomicOr(d.status, IMIE_EOVF);
  }
}

__global__ void attn_init_kernel(AttnDesc d) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t rows = d.B * d.H * d.M;
  if (i < rows * d.hd) d.acc[i] = 0;
  if (i < rows) d.rowmax[i] = INT64_MIN;
  if (i < d.B * d.Hkv) { d.maxk[i] = 0; d.maxv[i] = 0; }
}

// ---------------------------------------------------------------------------------------------------------
// Decode fast path (M == 1): one query per (b, head); the rep = H / Hkv heads of a KV group share every K/V read.
// The keys of each (b, kv) are split into nch chunks of `chunk` keys (a multiple of 64, sized so the grid has
// ~4096 workgroups); grid = (B * Hkv, nch). Every cross-chunk quantity (row max, Z, max|K|, max|V|, max|p|, the
// PV sums) is written per chunk and reduced by its consumer: no same-address atomics, which serialize across
// the XCDs' L2 slices.
//   D1 scores : wave = 4 keys x 16 lanes (8 dims per lane, 32 B vector loads), rep dots per key, 16-lane shuffle
//               reduction; scores[(b,h)][j]; chunk max per head -> cmax[chunk][row], chunk max|K| -> ckm
//   D2 exp    : row max = max over cmax; e_j = 2^-(...); chunk Z -> cz[chunk][row]; e_j stored in place for the
//               int64 cache's PV (the kv8 PV recomputes e_j from the score and the row max: no write-back)
//   D3 PV     : Z = sum over cz; per 256-key tile p_j = (e_j << f) / Z through a 2^64 / Z reciprocal with a
//               correction loop (exact for every e_j << f < 2^64), staged in LDS; a wave covers 2 keys per step
//               (32 lanes x 4 dims); chunk PV sums -> part[chunk][row][dim], chunk max|p| / max|V| -> cmp / cvm
//   D4 final  : out = (sum over chunks of part) >> f, plus the bound checks from the chunk maxima
// ---------------------------------------------------------------------------------------------------------
constexpr int kMaxRep = 8;

__device__ inline int64_t page_off(const AttnDesc& d, int64_t b, int64_t kv, int64_t j) {
  int64_t pi, in;
  page_split(d, j, pi, in);
  const int64_t pg = d.pt[b * d.mp + pi];
  return pg * (d.Hkv * d.P * d.hd) + kv * d.P * d.hd + in * d.hd;
}

// element offsets of the keys r0 .. r0+63 of (b, kv) into s_off (threads 0..63; the caller synchronizes)
__device__ inline void round_offsets(const AttnDesc& d, int64_t b, int64_t kv, int64_t r0, int64_t jend,
                                     int64_t* s_off) {
  const int t = threadIdx.x;
  if (t < 64) s_off[t] = r0 + t < jend ? page_off(d, b, kv, r0 + t) : 0;
}

__device__ inline int64_t dec_len(const AttnDesc& d, int64_t b) { return d.starts ? d.starts[b] + 1 : d.lengths[b]; }

// 8 consecutive KV elements as int64 (two 16 B loads for int32, four for int64); p is 32 B aligned
template <typename KT>
__device__ inline void load8(const KT* p, int64_t v[8]);
template <>
__device__ inline void load8<int32_t>(const int32_t* p, int64_t v[8]) {
  const v4i a = ((const v4i*)p)[0], b = ((const v4i*)p)[1];
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
template <>
__device__ inline void load8<int64_t>(const int64_t* p, int64_t v[8]) {
#pragma unroll
  for (int c = 0; c < 8; ++c) v[c] = p[c];
}
template <typename KT>
__device__ inline void load4(const KT* p, int64_t v[4]);
template <>
__device__ inline void load4<int32_t>(const int32_t* p, int64_t v[4]) {
  const v4i w = *(const v4i*)p;
  v[0] = w.x; v[1] = w.y; v[2] = w.z; v[3] = w.w;
}
template <>
__device__ inline void load4<int64_t>(const int64_t* p, int64_t v[4]) {
#pragma unroll
  for (int c = 0; c < 4; ++c) v[c] = p[c];
}

template <typename KT, int REP>
__global__ __launch_bounds__(256) void dec_scores_kernel(AttnDesc d) {
  __shared__ int64_t s_max[4][REP];
  __shared__ uint64_t s_mk[4];
  __shared__ int64_t s_off[64];
  const int64_t bkv = blockIdx.x, b = imie_udiv32(bkv, d.Hkv), kv = imie_umod32(bkv, d.Hkv);
  const int64_t rows = d.B * d.H;
  const int64_t L = dec_len(d, b);
  const int64_t j0 = (int64_t)blockIdx.y * d.chunk;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane >> 4, l16 = lane & 15;          // key within the 4-key group, lane within the key
  const bool dims = l16 * 8 < d.hd;
  int64_t q[REP][8];
#pragma unroll
  for (int r = 0; r < REP; ++r) {
    const int64_t* qr = d.q + b * d.qsb + (kv * REP + r) * d.qsh;
#pragma unroll
    for (int c = 0; c < 8; ++c) q[r][c] = dims ? qr[l16 * 8 + c] : 0;
  }
  if (blockIdx.y == 0 && wave == 0 && sub == 0) {
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      uint64_t m = 0;
#pragma unroll
      for (int c = 0; c < 8; ++c) { const uint64_t a = imie_absu64(q[r][c]); m = a > m ? a : m; }
#pragma unroll
      for (int o = 8; o >= 1; o >>= 1) { const uint64_t w = __shfl_xor(m, o, 64); m = w > m ? w : m; }
      if (l16 == 0) d.maxq[b * d.H + kv * REP + r] = m;
    }
  }
  int64_t smax[REP];
#pragma unroll
  for (int r = 0; r < REP; ++r) smax[r] = INT64_MIN;
  uint64_t mk = 0;
  const int64_t jend = min(j0 + d.chunk, L);
  // rounds of 64 keys: wave w owns keys 16w .. 16w+15 of the round as 4 groups of 4; all 4 groups' K slices
  // are loaded before any dot product (4 loads in flight per lane)
  for (int64_t r0 = j0; r0 < jend; r0 += 64) {
    __syncthreads();                                  // previous round's offsets consumed
    round_offsets(d, b, kv, r0, jend, s_off);
    __syncthreads();
    int64_t kvv[4][8];
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const int64_t j = r0 + wave * 16 + gq * 4 + sub;
#pragma unroll
      for (int c = 0; c < 8; ++c) kvv[gq][c] = 0;
      if (j < jend && dims) load8<KT>((const KT*)d.K + s_off[j - r0] + l16 * 8, kvv[gq]);
    }
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const int64_t j = r0 + wave * 16 + gq * 4 + sub;
      const bool live = j < jend;
#pragma unroll
      for (int c = 0; c < 8; ++c) { const uint64_t a = imie_absu64(kvv[gq][c]); mk = a > mk ? a : mk; }
#pragma unroll
      for (int r = 0; r < REP; ++r) {
        uint64_t dot = 0;
#pragma unroll
        for (int c = 0; c < 8; ++c) dot += (uint64_t)q[r][c] * (uint64_t)kvv[gq][c];
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) dot += (uint64_t)__shfl_xor((int64_t)dot, o, 64);
        if (live) {
          int64_t sc = (int64_t)dot >> d.frac;
          sc = (int64_t)((uint64_t)sc * (uint64_t)d.inv_sqrt) >> d.frac;
          if (l16 == 0) d.scores[(b * d.H + kv * REP + r) * d.Lmax + j] = sc;
          smax[r] = sc > smax[r] ? sc : smax[r];
        }
      }
    }
  }
  mk = imie_wave_max_u64(mk);
#pragma unroll
  for (int r = 0; r < REP; ++r) {
    int64_t m = smax[r];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) { const int64_t w = __shfl_xor(m, o, 64); m = w > m ? w : m; }
    smax[r] = m;
  }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < REP; ++r) s_max[wave][r] = smax[r];
    s_mk[wave] = mk;
  }
  __syncthreads();
  if (threadIdx.x < REP) {
    const int r = threadIdx.x;
    int64_t m = s_max[0][r];
    for (int w = 1; w < 4; ++w) m = s_max[w][r] > m ? s_max[w][r] : m;
    d.cmax[blockIdx.y * rows + b * d.H + kv * REP + r] = m;          // INT64_MIN for an empty chunk
  }
  if (threadIdx.x == 0) {
    uint64_t m = s_mk[0];
    for (int w = 1; w < 4; ++w) m = s_mk[w] > m ? s_mk[w] : m;
    d.ckm[blockIdx.y * d.B * d.Hkv + bkv] = m;
  }
}

// STORE = false (kv8 path): only the chunk Z sums are written; the PV kernel recomputes each e_j from its score
// and the row maximum, so the scores are not rewritten in place (half of this kernel's traffic)
template <int REP, bool STORE = true>
__global__ __launch_bounds__(256) void dec_exp_kernel(AttnDesc d) {
  __shared__ int64_t s_rmax[REP];
  __shared__ uint64_t s_z[4][REP];
  const int64_t bkv = blockIdx.x, b = imie_udiv32(bkv, d.Hkv), kv = imie_umod32(bkv, d.Hkv);
  const int64_t rows = d.B * d.H;
  const int64_t j0 = (int64_t)blockIdx.y * d.chunk;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // requested before the sequence length arrives (none of them depends on it): this thread's scores (chunks of
  // up to 256 keys; the row stride Lmax bounds the index, keys past the length are masked below) and the first
  // 128 chunk maxima of the rows this wave reduces, two per lane (an empty chunk's maximum is INT64_MIN)
  const bool one = d.chunk <= 256;
  const int64_t jt = j0 + threadIdx.x;
  int64_t sv[REP];
#pragma unroll
  for (int r = 0; r < REP; ++r) sv[r] = (one && jt < d.Lmax) ? d.scores[(b * d.H + kv * REP + r) * d.Lmax + jt] : 0;
  constexpr int RW = (REP + 3) / 4;
  int64_t cm[RW];
#pragma unroll
  for (int k = 0; k < RW; ++k) {
    const int r = wave + 4 * k;
    const int64_t a0 = (r < REP && lane < d.nch) ? d.cmax[(int64_t)lane * rows + b * d.H + kv * REP + r] : INT64_MIN;
    const int64_t a1 =
        (r < REP && lane + 64 < d.nch) ? d.cmax[(int64_t)(lane + 64) * rows + b * d.H + kv * REP + r] : INT64_MIN;
    cm[k] = a0 > a1 ? a0 : a1;
  }
  const int64_t L = dec_len(d, b);
  if (j0 >= L) {
    if (threadIdx.x < REP) d.cz[blockIdx.y * rows + b * d.H + kv * REP + threadIdx.x] = 0;
    return;
  }
  const int64_t jend = min(j0 + d.chunk, L);
  const bool fx32 = (d.dclip >> 32) == 0 && (d.log2e >> 32) == 0;
  // row max over all chunks (wave r reduces row r)
#pragma unroll
  for (int k = 0; k < RW; ++k) {
    const int r = wave + 4 * k;
    if (r >= REP) break;
    int64_t m = cm[k];
    for (int64_t c = lane + 128; c < d.nch; c += 64) {
      const int64_t v = d.cmax[c * rows + b * d.H + kv * REP + r];
      m = v > m ? v : m;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) { const int64_t w = __shfl_xor(m, o, 64); m = w > m ? w : m; }
    if (lane == 0) s_rmax[r] = m;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < REP; ++r) {
    const int64_t row = b * d.H + kv * REP + r;
    const int64_t mx = s_rmax[r];
    uint64_t z = 0;
    auto one_e = [&](int64_t j, int64_t s) {
      int64_t dd = (int64_t)((uint64_t)mx - (uint64_t)s);
      if (dd > d.dclip) dd = d.dclip;
      const uint64_t e = (uint64_t)exp_clipped(dd, d.frac, d.log2e, fx32);
      if (STORE) d.scores[row * d.Lmax + j] = (int64_t)e;
      z += e;
    };
    if (one) {
      if (jt < jend) one_e(jt, sv[r]);
    } else {
      // long chunks: eight of the thread's scores requested per round (a load per iteration would wait for
      // each in turn); keys past jend read an in-bounds score and are not used
      for (int64_t j = j0 + threadIdx.x; j < jend; j += 8 * 256) {
        int64_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = d.scores[row * d.Lmax + min(j + 256 * u, jend - 1)];
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (j + 256 * u < jend) one_e(j + 256 * u, v[u]);
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) z += (uint64_t)__shfl_xor((int64_t)z, o, 64);
    if (lane == 0) s_z[wave][r] = z;
  }
  __syncthreads();
  if (threadIdx.x < REP) {
    const int r = threadIdx.x;
    d.cz[blockIdx.y * rows + b * d.H + kv * REP + r] = s_z[0][r] + s_z[1][r] + s_z[2][r] + s_z[3][r];
  }
}

template <typename KT, int REP>
__global__ __launch_bounds__(256) void dec_pv_kernel(AttnDesc d) {
  __shared__ int64_t sp[REP][64];
  __shared__ uint64_t red[4][REP][128];
  __shared__ int64_t s_off[64];
  __shared__ uint64_t s_z[REP], s_mp[4][REP], s_mv[4];
  const int64_t bkv = blockIdx.x, b = imie_udiv32(bkv, d.Hkv), kv = imie_umod32(bkv, d.Hkv);
  const int64_t L = dec_len(d, b);
  const int64_t j0 = (int64_t)blockIdx.y * d.chunk;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, c0 = (lane & 31) * 4;     // key parity within the wave step, first dim
  const bool dims = c0 < d.hd;
  const int64_t rows = d.B * d.H;
  uint64_t* part = d.part + (int64_t)blockIdx.y * rows * d.hd;
  if (j0 >= L) {                                      // an empty chunk still owns its partial slots
    for (int i = tid; i < REP * d.hd; i += blockDim.x)
      part[(b * d.H + kv * REP + imie_udiv32(i, d.hd)) * d.hd + imie_umod32(i, d.hd)] = 0;
    if (tid < REP) d.cmp[blockIdx.y * rows + b * d.H + kv * REP + tid] = 0;
    if (tid == 0) d.cvm[blockIdx.y * d.B * d.Hkv + bkv] = 0;
    return;
  }
  const int64_t nlive = imie_udiv32(L + d.chunk - 1, d.chunk);
  for (int r = wave; r < REP; r += 4) {
    uint64_t z = 0;
    for (int64_t c = lane; c < nlive; c += 64) z += d.cz[c * rows + b * d.H + kv * REP + r];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) z += (uint64_t)__shfl_xor((int64_t)z, o, 64);
    if (lane == 0) s_z[r] = z;
  }
  __syncthreads();
  const int64_t jend = min(j0 + d.chunk, L);
  uint64_t Z[REP], rz[REP];
#pragma unroll
  for (int r = 0; r < REP; ++r) {
    Z[r] = s_z[r];
    rz[r] = Z[r] > 1 ? (~(uint64_t)0) / Z[r] : 0;
  }
  uint64_t acc[REP][4];
#pragma unroll
  for (int r = 0; r < REP; ++r) acc[r][0] = acc[r][1] = acc[r][2] = acc[r][3] = 0;
  uint64_t mp[REP];
#pragma unroll
  for (int r = 0; r < REP; ++r) mp[r] = 0;
  uint64_t mv = 0;
  // rounds of 64 keys: p for the round's keys is staged in LDS (thread t: key t % 64, rows t / 64 + 4k); wave w
  // owns keys 16w .. 16w+15, 2 per step (lane halves), all 8 steps' V slices loaded before accumulating
  for (int64_t t0 = j0; t0 < jend; t0 += 64) {
    const int64_t tn = min((int64_t)64, jend - t0);
    __syncthreads();                                  // previous round's sp / offsets fully consumed
    round_offsets(d, b, kv, t0, jend, s_off);
    {
      const int kk = tid & 63;
      for (int r = tid >> 6; r < REP; r += 4) {
        const int64_t row = b * d.H + kv * REP + r;
        int64_t p = 0;
        if (kk < tn && Z[r] != 0) {
          const uint64_t num = (uint64_t)d.scores[row * d.Lmax + t0 + kk] << d.frac;
          if (Z[r] == 1) p = (int64_t)num;
          else {
            uint64_t qq = __umul64hi(num, rz[r]);
            uint64_t rem = num - qq * Z[r];
            while (rem >= Z[r]) { ++qq; rem -= Z[r]; }
            p = (int64_t)qq;
          }
        }
        sp[r][kk] = p;
        mp[r] = (uint64_t)p > mp[r] ? (uint64_t)p : mp[r];
      }
    }
    __syncthreads();
    int64_t v[8][4];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = wave * 16 + 2 * u + half;
#pragma unroll
      for (int c = 0; c < 4; ++c) v[u][c] = 0;
      if (dims && i < tn) load4<KT>((const KT*)d.V + s_off[i] + c0, v[u]);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = wave * 16 + 2 * u + half;
#pragma unroll
      for (int c = 0; c < 4; ++c) { const uint64_t a = imie_absu64(v[u][c]); mv = a > mv ? a : mv; }
#pragma unroll
      for (int r = 0; r < REP; ++r) {
        const uint64_t pp = (uint64_t)sp[r][i];      // 0 beyond tn (and v is 0 there)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[r][c] += pp * (uint64_t)v[u][c];
      }
    }
  }
#pragma unroll
  for (int r = 0; r < REP; ++r) {
    const uint64_t m = imie_wave_max_u64(mp[r]);
    if (lane == 0) s_mp[wave][r] = m;
  }
  mv = imie_wave_max_u64(mv);
  if (lane == 0) s_mv[wave] = mv;
#pragma unroll
  for (int r = 0; r < REP; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[r][c] += (uint64_t)__shfl_xor((int64_t)acc[r][c], 32, 64);
  if (half == 0 && dims) {
#pragma unroll
    for (int r = 0; r < REP; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) red[wave][r][c0 + c] = acc[r][c];
  }
  __syncthreads();
  for (int i = tid; i < REP * d.hd; i += blockDim.x) {
    const int r = i / (int)d.hd, c = i % (int)d.hd;
    part[(b * d.H + kv * REP + r) * d.hd + c] = red[0][r][c] + red[1][r][c] + red[2][r][c] + red[3][r][c];
  }
  if (tid < REP) {
    uint64_t m = s_mp[0][tid];
    for (int w = 1; w < 4; ++w) m = s_mp[w][tid] > m ? s_mp[w][tid] : m;
    d.cmp[blockIdx.y * rows + b * d.H + kv * REP + tid] = m;
  }
  if (tid == 0) {
    uint64_t m = s_mv[0];
    for (int w = 1; w < 4; ++w) m = s_mv[w] > m ? s_mv[w] : m;
    d.cvm[blockIdx.y * d.B * d.Hkv + bkv] = m;
  }
}

// WG = 32 consecutive outputs (within one row) x 8 chunk groups: thread (o, g) sums chunks g, g + 8, ... of
// output o over all nch chunks (an empty chunk's partials are zero, so no sequence length is needed first; the
// loads of a round are all issued before any is added), and the 8 group sums are added through LDS. The bound
// checks run in separate workgroups at the end of the grid, alongside the sums: one wave per row reads the
// row's chunk maxima (lane c: chunk c, c + 64, ...), the sequence length and the K / V maxima at once.
__global__ __launch_bounds__(256) void dec_final_kernel(AttnDesc d) {
  __shared__ uint64_t s_sum[8][32];
  const int t = threadIdx.x, o = t & 31, g = t >> 5;
  const int64_t rows = d.B * d.H;
  const int64_t nsum = (rows * d.hd + 31) / 32;
  if ((int64_t)blockIdx.x >= nsum) {
    const int lane = t & 63;
    const int64_t r = ((int64_t)blockIdx.x - nsum) * 4 + (t >> 6);
    if ((int64_t)blockIdx.x == nsum && t == 0) check_rope_guard(d);
    if (r >= rows) return;
    const int64_t b = imie_udiv32(r, d.H), kv = imie_udiv32(imie_umod32(r, d.H), d.H / d.Hkv);
    const int64_t bkv = b * d.Hkv + kv;
    const int64_t L = dec_len(d, b);
    const uint64_t mq = d.maxq[r];
    const uint64_t rk = d.run_k ? d.run_k[bkv] : 0, rv = d.run_k ? d.run_v[bkv] : 0;
    uint64_t mp = 0, mv = 0, mk = 0;
    for (int64_t c0 = 0; c0 < d.nch; c0 += 128) {
      uint64_t a[2], v[2], k[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int64_t c = c0 + 64 * h + lane;
        const bool in = c < d.nch;
        a[h] = in ? d.cmp[c * rows + r] : 0;
        v[h] = (in && !d.run_k) ? d.cvm[c * d.B * d.Hkv + bkv] : 0;
        k[h] = (in && !d.run_k) ? d.ckm[c * d.B * d.Hkv + bkv] : 0;
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        mp = a[h] > mp ? a[h] : mp;
        mv = v[h] > mv ? v[h] : mv;
        mk = k[h] > mk ? k[h] : mk;
      }
    }
    mp = imie_wave_max_u64_full(mp);
    if (d.run_k) { mk = rk; mv = rv; }
    else { mv = imie_wave_max_u64_full(mv); mk = imie_wave_max_u64_full(mk); }
    if (lane == 0 && L > 0) {
      if ((u128)mp * mv > (u128)(INT64_MAX / L)) atomicOr(d.status, IMIE_EOVF);
      if ((u128)mq * mk > (u128)(INT64_MAX / d.hd)) atomicOr(d.status, IMIE_EOVF);
    }
    return;
  }
  const int64_t i = (int64_t)blockIdx.x * 32 + o;
  const int64_t r = imie_udiv32((int64_t)blockIdx.x * 32, d.hd);
  const int64_t stride = rows * d.hd;
  const bool live_o = i < rows * d.hd;
  uint64_t acc = 0;
  for (int64_t c0 = g; c0 < d.nch; c0 += 128) {
    uint64_t pv[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int64_t c = c0 + 8 * u;
      pv[u] = (c < d.nch && live_o) ? d.part[c * stride + i] : 0;
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) acc += pv[u];
  }
  s_sum[g][o] = acc;
  __syncthreads();
  if (t < 32 && live_o) {
    uint64_t tot = 0;
#pragma unroll
    for (int gg = 0; gg < 8; ++gg) tot += s_sum[gg][t];
    d.out[qoff(d, r) + imie_umod32(i, d.hd)] = (int64_t)tot >> d.frac;
  }
}


// ---------------------------------------------------------------------------------------------------------
// kv8 cache (imie_kvfmt.h): the dot products run as int8 MFMAs on the stored digit bytes.
//   scores: A = balanced base-256 digits of q (limb lq), B = K digit plane b; sum_c q k = sum_{lq,b} 256^(lq+b) D
//   PV    : A = digits of p (limb lp, keys on the K axis), B = V digit plane b (keys x dims)
// MFMA int32 sums are exact (|D| <= 64 * 128 * 128 per MFMA; partial sums bounded below 2^31 as noted); every
// recombination into the int64 result wraps mod 2^64 like the oracle's int64 arithmetic.
// max|K| / max|V| for the fail-loud bounds are the running maxima kept by the cache writes (run_k / run_v).
// ---------------------------------------------------------------------------------------------------------
__device__ inline int64_t bal_digit(int64_t x, int l) {
  for (int i = 0; i < l; ++i) {
    const int64_t dg = ((x + 128) & 255) - 128;
    x = (int64_t)((uint64_t)x - (uint64_t)dg) >> 8;
  }
  return ((x + 128) & 255) - 128;
}

__device__ inline v4i pack16(const int8_t* v) {
  v4i r;
#pragma unroll
  for (int k = 0; k < 4; ++k)
    r[k] = (int)((uint32_t)(uint8_t)v[4 * k] | ((uint32_t)(uint8_t)v[4 * k + 1] << 8) |
                 ((uint32_t)(uint8_t)v[4 * k + 2] << 16) | ((uint32_t)(uint8_t)v[4 * k + 3] << 24));
  return r;
}

__device__ inline v4i mfma8(v4i a, v4i b, v4i c) { return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0); }

// keep the first n (0..16) bytes of a 16-byte operand
__device__ inline v4i keep_bytes(v4i v, int n) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int nb = n - 4 * k;
    const uint32_t mk = nb >= 4 ? 0xFFFFFFFFu : (nb <= 0 ? 0u : ((1u << (8 * nb)) - 1u));
    v[k] = (int)((uint32_t)v[k] & mk);
  }
  return v;
}

__device__ inline int64_t kv8_row_base(const AttnDesc& d, int64_t b, int64_t kv, int64_t j, int64_t* slot) {
  int64_t pi, in;
  page_split(d, j, pi, in);
  *slot = in;
  return imie_kv8::block_base(d.pt[b * d.mp + pi], kv, d.Hkv, d.hd, d.P);
}

// Decode scores (M == 1). Workgroup = (b, kv, chunk); wave w takes 16-key tiles w, w + 4, ... MFMA rows are
// (head r, limb lq): row 4 (r % 4) + (lq % 4) of row block (r / 4, lq / 4); a D lane (g, n) then holds the 4
// limbs of head 4 * hb + g for key n and recombines them in place. With d.qd set, the head stage has already
// written q's digit planes, limb counts and max|q|, and the A operands are read from memory directly;
// otherwise the first wave-pass digitizes q into LDS.
// Three waves per SIMD (at most 168 VGPRs) up to four heads per kv head; eight heads keep two (no spills in the loop).
template <int REP, int KS>
__global__ __launch_bounds__(256, REP <= 4 ? 3 : 2) void dec_scores8_kernel(AttnDesc d) {
  constexpr int RBH = (REP + 3) / 4;
  __shared__ int64_t s_max[4][REP];
  __shared__ uint64_t s_mq[4];
  __shared__ __align__(16) int8_t sQd[RBH][2][16][128];
  const int64_t bkv = blockIdx.x, b = imie_udiv32(bkv, d.Hkv), kv = imie_umod32(bkv, d.Hkv);
  const int64_t rows = d.B * d.H;
  const int64_t L = dec_len(d, b);
  const int64_t j0 = (int64_t)blockIdx.y * d.chunk;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), m = lane & 15,
            g = lane >> 4;
  const int64_t* qg = d.q + b * d.qsb + kv * REP * d.qsh;
  v4i av[RBH][2][2];
  int Lq = 0, LB = 0;
  static_assert(KS == 1 || KS == 2, "KS: 64-dim K steps, (hd + 63) / 64");
  int64_t smax[RBH];
#pragma unroll
  for (int hb = 0; hb < RBH; ++hb) smax[hb] = INT64_MIN;
  const int64_t jend = min(j0 + d.chunk, L);
  const int8_t* Kb = (const int8_t*)d.K;
  // page ids of the chunk's keys in lane registers (lane i: page pi0 + i, up to 64 pages): a tile's K addresses
  // then come from a cross-lane move, not from a page-table load that would wait behind the previous tile's K
  // loads (the vector memory counter is in order), so the next tile's loads really are in flight
  int64_t pi0, pin0, pi1, pin1;
  page_split(d, j0, pi0, pin0);
  page_split(d, max(j0, min(j0 + d.chunk, d.Lmax) - 1), pi1, pin1);
  const bool pgreg = pi1 - pi0 < 64;
  int64_t pgl = (pgreg && lane <= pi1 - pi0) ? d.pt[b * d.mp + pi0 + lane] : 0;
  // 16-key tiles t = j0 + 16 wave + 64 i; the next tile's K slices are loaded before this tile's MFMAs. PG (a
  // compile-time copy of pgreg): the loop of the common case holds no page-table load, whose possible pending
  // write on the other path would make the compiler wait for every load in flight
  // The loads are issued whether or not the tile exists (live false: every lane reads the pool's first 16 bytes,
  // one cache line): a load that may be skipped leaves the compiler unable to count the loads in flight, and it
  // then waits for all of them before the MFMAs.
  // A tile's scores are stored at the start of the next load_tile, before that tile's loads, and their registers
  // are kept live across those loads: the compiler waits for a store before its data registers are rewritten, and
  // the vector memory counter is in order, so a store issued after the loads would make that wait include them.
  int64_t pend_v[RBH], pend_i[RBH];
#pragma unroll
  for (int hb = 0; hb < RBH; ++hb) { pend_v[hb] = 0; pend_i[hb] = -1; }
  auto flush = [&]() {
#pragma unroll
    for (int hb = 0; hb < RBH; ++hb)
      if (pend_i[hb] >= 0) d.scores[pend_i[hb]] = pend_v[hb];
  };
  auto load_tile = [&](auto pgc, bool live, int64_t t, int64_t lim, v4i (&bk)[4][2]) {   // keys below lim
    constexpr bool PG = decltype(pgc)::value;
    flush();
    const int64_t j = t + m;
    const bool valid = live && j < lim;
    int64_t base = 0, slot = 0;
    if constexpr (PG) {                               // every lane active here (t is wave-uniform)
      int64_t pi;
      page_split(d, valid ? j : j0, pi, slot);
      const int64_t pg = __shfl(pgl, (int)(pi - pi0), 64);
      base = imie_kv8::block_base(pg, kv, d.Hkv, d.hd, d.P) + imie_kv8::k_off(slot, 0, 0, d.hd);
    } else if (valid) {
      base = kv8_row_base(d, b, kv, j, &slot) + imie_kv8::k_off(slot, 0, 0, d.hd);
    }
    // every lane loads, with no select on the data: a conditional load is a branch, after which the compiler
    // waits for every load in flight (vmcnt 0, the next tile's prefetch too) before the MFMAs, and a select
    // waits for its load at once. Lanes of keys past `lim` read an in-bounds address (their score columns are
    // never stored); dims at or past hd read dims 0.. of the same slot, which meet zero q digits.
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int h = 0; h < KS; ++h) {
        const int64_t c = 64 * h + 16 * g;
        bk[db][h] = *(const v4i*)(Kb + (live ? base + imie_kv8::k_piece(db, c < d.hd ? c : 0, d.hd) : 0));
      }
    // keeps the loads here: otherwise they sink into the block that consumes them, or the consumer's MFMAs (and
    // their waits) are scheduled above them
    asm volatile("" ::: "memory");
#pragma unroll
    for (int hb = 0; hb < RBH; ++hb) asm volatile("" ::"v"(pend_v[hb]), "v"(pend_i[hb]));
    __builtin_amdgcn_sched_barrier(0);
  };
  auto score_tile = [&](int64_t t, const v4i (&bk)[4][2]) {
    const int64_t j = t + m;
    const bool valid = j < jend;
#pragma unroll
    for (int hb = 0; hb < RBH; ++hb) {
      uint64_t S = 0;
      for (int lb = 0; lb < LB; ++lb)
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          v4i D = mfma8(av[hb][lb][0], bk[db][0], v4i{0, 0, 0, 0});
          if constexpr (KS > 1) D = mfma8(av[hb][lb][1], bk[db][1], D);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int e = 4 * lb + i + db;              // 256^e = 0 mod 2^64 for e >= 8
            if (e < 8) S += (uint64_t)(int64_t)D[i] << (8 * e);
          }
        }
      const int r = 4 * hb + g;
      int64_t sc = (int64_t)S >> d.frac;
      sc = (int64_t)((uint64_t)sc * (uint64_t)d.inv_sqrt) >> d.frac;
      pend_v[hb] = sc;
      pend_i[hb] = (valid && r < REP) ? (b * d.H + kv * REP + r) * d.Lmax + j : -1;
      if (valid && r < REP) smax[hb] = sc > smax[hb] ? sc : smax[hb];
    }
  };
  v4i bkA[4][2], bkB[4][2];
  int64_t t = j0 + 16 * wave;
  // the first K tile in flight during the q setup, bounded by the score row stride rather than the sequence length
  // (no wait for the length): keys past it give scores that are never stored
  const int64_t lim0 = min(j0 + d.chunk, d.Lmax);
  if (pgreg) load_tile(std::true_type{}, t < lim0, t, lim0, bkA);
  else load_tile(std::false_type{}, t < lim0, t, lim0, bkA);
  if (d.qd) {
    // digits prepared by the head stage (all eight limb planes written): A operands straight from memory, loaded
    // together with the limb counts and masked once those arrive
#pragma unroll
    for (int hb = 0; hb < RBH; ++hb)
#pragma unroll
      for (int lb = 0; lb < 2; ++lb)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int r = 4 * hb + (m >> 2), lq = 4 * lb + (m & 3);
          av[hb][lb][h] = (r < REP && 64 * h + 16 * g < d.hd)
                              ? *(const v4i*)(d.qd + ((b * d.H + kv * REP + r) * 8 + lq) * d.hd + 64 * h + 16 * g)
                              : v4i{0, 0, 0, 0};
        }
    int lrs[REP];
#pragma unroll
    for (int r = 0; r < REP; ++r) lrs[r] = d.qlimbs[b * d.H + kv * REP + r];
#pragma unroll
    for (int r = 0; r < REP; ++r) Lq = lrs[r] > Lq ? lrs[r] : Lq;
#pragma unroll
    for (int hb = 0; hb < RBH; ++hb)
#pragma unroll
      for (int lb = 0; lb < 2; ++lb)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          if (4 * lb + (m & 3) >= Lq) av[hb][lb][h] = v4i{0, 0, 0, 0};
  } else {
    uint64_t mq = 0;
    for (int i = tid; i < REP * d.hd; i += 256) {
      const uint64_t a = imie_absu64(qg[imie_udiv32(i, d.hd) * d.qsh + imie_umod32(i, d.hd)]);
      mq = a > mq ? a : mq;
    }
    mq = imie_wave_max_u64(mq);
    if (lane == 0) s_mq[wave] = mq;
    if (blockIdx.y == 0 && tid < REP) {
      uint64_t mr = 0;
      for (int c = 0; c < d.hd; ++c) { const uint64_t a = imie_absu64(qg[tid * d.qsh + c]); mr = a > mr ? a : mr; }
      d.maxq[b * d.H + kv * REP + tid] = mr;
    }
    __syncthreads();
    uint64_t mqa = s_mq[0];
    for (int w = 1; w < 4; ++w) mqa = s_mq[w] > mqa ? s_mq[w] : mqa;
    Lq = imie_limbs_needed(mqa);
    // digits of every q element once (thread per element) into LDS rows [head block][4 (r % 4) + lq % 4][limb
    // block][dim]; each lane then reads its 16-byte A operands directly
    for (int i = tid; i < RBH * 2 * 16 * 128; i += 256) (&sQd[0][0][0][0])[i] = 0;
    __syncthreads();
    for (int i = tid; i < REP * d.hd; i += 256) {
      const int r = (int)imie_udiv32(i, d.hd), c = (int)imie_umod32(i, d.hd);
      int64_t x = qg[r * d.qsh + c];
      for (int lq = 0; lq < Lq; ++lq) {
        const int64_t dg = ((x + 128) & 255) - 128;
        x = (int64_t)((uint64_t)x - (uint64_t)dg) >> 8;
        sQd[r >> 2][lq >> 2][4 * (r & 3) + (lq & 3)][c] = (int8_t)dg;
      }
    }
    __syncthreads();
#pragma unroll
    for (int hb = 0; hb < RBH; ++hb)
#pragma unroll
      for (int lb = 0; lb < 2; ++lb)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          av[hb][lb][h] = (64 * h + 16 * g < d.hd) ? *(const v4i*)&sQd[hb][lb][m][64 * h + 16 * g] : v4i{0, 0, 0, 0};
  }
  // at least one limb block (zero digits score 0): the tile's MFMAs, and with them the waits for its loads, are
  // then on every path, and no load of a consumed tile is still counted at the loop's back edge
  LB = Lq > 4 ? 2 : 1;
  // the loop's loop-invariant operands loaded before it (page ids, q digits) are re-defined here by empty asm
  // statements (one wait for them, here): as load results, their age is lost over the loop's back edge and the
  // compiler would wait for every load in flight (vmcnt 0, the K prefetch too) before each use in the loop
  asm volatile("" : "+v"(pgl));
#pragma unroll
  for (int hb = 0; hb < RBH; ++hb)
#pragma unroll
    for (int lb = 0; lb < 2; ++lb)
#pragma unroll
      for (int h = 0; h < 2; ++h) asm volatile("" : "+v"(av[hb][lb][h]));
  auto walk = [&](auto pgc) {
    // every load so far (the first K tile, the q digits) is complete at the loop's entry: a load still in flight
    // there would make the compiler's wait tracking conservative in every iteration
    __builtin_amdgcn_s_waitcnt(0x0F70);             // vmcnt(0)
    while (t < jend) {
      const int64_t t2 = t + 64;
      load_tile(pgc, t2 < jend, t2, jend, bkB);
      score_tile(t, bkA);
      if (t2 >= jend) break;
      const int64_t t3 = t2 + 64;
      load_tile(pgc, t3 < jend, t3, jend, bkA);
      score_tile(t2, bkB);
      t = t3;
    }
  };
  if (pgreg) walk(std::true_type{});
  else walk(std::false_type{});
  flush();
#pragma unroll
  for (int hb = 0; hb < RBH; ++hb) {
    int64_t mx = smax[hb];
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) { const int64_t w2 = __shfl_xor(mx, o, 64); mx = w2 > mx ? w2 : mx; }
    const int r = 4 * hb + g;
    if (m == 0 && r < REP) s_max[wave][r] = mx;
  }
  __syncthreads();
  if (tid < REP) {
    int64_t mx = s_max[0][tid];
    for (int w = 1; w < 4; ++w) mx = s_max[w][tid] > mx ? s_max[w][tid] : mx;
    d.cmax[blockIdx.y * rows + b * d.H + kv * REP + tid] = mx;
  }
}

// Decode PV (M == 1). Workgroup = (b, kv, chunk); per 64-key step the p digits of the REP heads are staged in LDS
// as the A operand (row 4 (r % 4) + lp of head block r / 4); wave w owns dim tiles w and w + 4. RECOMP: e_j is
// recomputed here from the score and the row maximum (dec_exp_kernel<REP, false> wrote no e); otherwise the
// scores array holds e_j.
template <int REP, bool RECOMP>
__global__ __launch_bounds__(256) void dec_pv8_kernel(AttnDesc d) {
  constexpr int RBH = (REP + 3) / 4;
  __shared__ __align__(16) int8_t sPd[RBH][16][64];
  __shared__ uint64_t s_z[REP], s_mp[4][REP];
  __shared__ int64_t s_m[REP];
  __shared__ double s_rzd[REP];
  const int64_t bkv = blockIdx.x, b = imie_udiv32(bkv, d.Hkv), kv = imie_umod32(bkv, d.Hkv);
  const int64_t j0 = (int64_t)blockIdx.y * d.chunk;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, m = lane & 15, g = lane >> 4;
  const int64_t rows = d.B * d.H;
  uint64_t* part = d.part + (int64_t)blockIdx.y * rows * d.hd;
  const int DT = (int)(d.hd / 16);
  const int8_t* Vb = (const int8_t*)d.V;
  // one 64-key step's operands: the V slices of this wave's dim tiles and the scores of thread (key tid % 64,
  // heads tid / 64 + 4k), bounded by `lim` (keys past the sequence length are masked where p is formed); the
  // first step's, and the chunk Z sums (an empty chunk's is 0), are requested before the sequence length is
  // known, later steps' one step ahead
  constexpr int RW = (REP + 3) / 4;
  // page ids of the chunk's keys in lane registers (lane i: page pi0 + i, up to 64 pages): a step's V address
  // comes from a lane read, not from a page-table load queued behind the previous step's V loads
  int64_t pi0, pin0, pi1, pin1;
  page_split(d, j0, pi0, pin0);
  page_split(d, max(j0, min(j0 + d.chunk, d.Lmax) - 1), pi1, pin1);
  const bool pgreg = pi1 - pi0 < 64;
  const int64_t pgl = (pgreg && lane <= pi1 - pi0) ? d.pt[b * d.mp + pi0 + lane] : 0;
  auto load_step = [&](int64_t t0, int64_t lim, v4i (&bv)[2][4], int64_t (&sc)[RW]) {
    const int64_t tn = min((int64_t)64, lim - t0);
    int64_t pi, slot0;
    page_split(d, t0, pi, slot0);
    const int64_t pg = pgreg ? (int64_t)imie_readlane_u64((uint64_t)pgl, (int)(pi - pi0)) : d.pt[b * d.mp + pi];
    const int8_t* vblk = Vb + imie_kv8::block_base(pg, kv, d.Hkv, d.hd, d.P);
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int tile = wave + 4 * tt;
#pragma unroll
      for (int db = 0; db < 4; ++db)
        bv[tt][db] = tile < DT ? *(const v4i*)(vblk + imie_kv8::v_off(slot0 + 16 * g, db, 16 * tile + m, d.hd, d.P))
                               : v4i{0, 0, 0, 0};
    }
    const int kk = tid & 63;
#pragma unroll
    for (int k = 0; k < RW; ++k) {
      const int r = (tid >> 6) + 4 * k;
      sc[k] = (r < REP && kk < tn) ? d.scores[(b * d.H + kv * REP + r) * d.Lmax + t0 + kk] : 0;
    }
  };
  v4i bvA[2][4], bvB[2][4];
  int64_t scA[RW], scB[RW];
  load_step(j0, d.Lmax, bvA, scA);
  uint64_t cz0[RW];
  int64_t cm0[RW];
#pragma unroll
  for (int k = 0; k < RW; ++k) {
    const int r = wave + 4 * k;
    const int64_t ri = b * d.H + kv * REP + r;
    const uint64_t z0 = (r < REP && lane < d.nch) ? d.cz[(int64_t)lane * rows + ri] : 0;
    const uint64_t z1 = (r < REP && lane + 64 < d.nch) ? d.cz[(int64_t)(lane + 64) * rows + ri] : 0;
    cz0[k] = z0 + z1;
    const int64_t m0 = (r < REP && lane < d.nch) ? d.cmax[(int64_t)lane * rows + ri] : INT64_MIN;
    const int64_t m1 = (r < REP && lane + 64 < d.nch) ? d.cmax[(int64_t)(lane + 64) * rows + ri] : INT64_MIN;
    cm0[k] = m0 > m1 ? m0 : m1;
  }
  const int64_t L = dec_len(d, b);
  if (j0 >= L) {
    for (int i = tid; i < REP * d.hd; i += blockDim.x)
      part[(b * d.H + kv * REP + imie_udiv32(i, d.hd)) * d.hd + imie_umod32(i, d.hd)] = 0;
    if (tid < REP) d.cmp[blockIdx.y * rows + b * d.H + kv * REP + tid] = 0;
    return;
  }
  const int64_t jend = min(j0 + d.chunk, L);
#pragma unroll
  for (int k = 0; k < RW; ++k) {
    const int r = wave + 4 * k;
    if (r >= REP) break;
    uint64_t z = cz0[k];
    int64_t mx = cm0[k];
    for (int64_t c = lane + 128; c < d.nch; c += 64) {
      z += d.cz[c * rows + b * d.H + kv * REP + r];
      const int64_t v = d.cmax[c * rows + b * d.H + kv * REP + r];
      mx = v > mx ? v : mx;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      z += (uint64_t)__shfl_xor((int64_t)z, o, 64);
      const int64_t w2 = __shfl_xor(mx, o, 64);
      mx = w2 > mx ? w2 : mx;
    }
    if (lane == 0) { s_z[r] = z; s_rzd[r] = z != 0 ? 1.0 / (double)z : 0.0; s_m[r] = mx; }
  }
  const bool fx32 = (d.dclip >> 32) == 0 && (d.log2e >> 32) == 0;
  for (int i = tid; i < RBH * 16 * 64; i += 256) (&sPd[0][0][0])[i] = 0;
  __syncthreads();
  const int Lp = imie_limbs_needed((uint64_t)1 << d.frac);
  uint64_t mp[REP];
#pragma unroll
  for (int r = 0; r < REP; ++r) mp[r] = 0;
  v4i acc[RBH][4][2];
#pragma unroll
  for (int hb = 0; hb < RBH; ++hb)
#pragma unroll
    for (int db = 0; db < 4; ++db) acc[hb][db][0] = acc[hb][db][1] = v4i{0, 0, 0, 0};
  for (int64_t t0 = j0; t0 < jend; t0 += 64) {
    const int64_t tn = min((int64_t)64, jend - t0);
    v4i bv[2][4];
    int64_t scv[RW];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int db = 0; db < 4; ++db) bv[tt][db] = bvA[tt][db];
#pragma unroll
    for (int k = 0; k < RW; ++k) scv[k] = scA[k];
    if (t0 + 64 < jend) {
      load_step(t0 + 64, jend, bvB, scB);
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int db = 0; db < 4; ++db) bvA[tt][db] = bvB[tt][db];
#pragma unroll
      for (int k = 0; k < RW; ++k) scA[k] = scB[k];
    }
    __syncthreads();                                  // previous step's digits consumed
    {
      const int kk = tid & 63;
#pragma unroll
      for (int k = 0; k < RW; ++k) {
        const int r = (tid >> 6) + 4 * k;
        if (r >= REP) break;
        const uint64_t Z = s_z[r];
        int64_t p = 0;
        if (kk < tn && Z != 0) {
          int64_t e = scv[k];
          if (RECOMP) {                                  // e_j of dec_exp_kernel from the score and the row maximum
            int64_t dd = (int64_t)((uint64_t)s_m[r] - (uint64_t)scv[k]);
            if (dd > d.dclip) dd = d.dclip;
            e = exp_clipped(dd, d.frac, d.log2e, fx32);
          }
          p = prob_div(e, d.frac, Z, s_rzd[r]);
        }
        mp[r] = (uint64_t)p > mp[r] ? (uint64_t)p : mp[r];
        int64_t x = p;
        for (int lp = 0; lp < 4; ++lp) {
          const int64_t dg = ((x + 128) & 255) - 128;
          x = (int64_t)((uint64_t)x - (uint64_t)dg) >> 8;
          sPd[r >> 2][4 * (r & 3) + lp][kk] = lp < Lp ? (int8_t)dg : (int8_t)0;
        }
      }
    }
    __syncthreads();
    v4i av[RBH];
#pragma unroll
    for (int hb = 0; hb < RBH; ++hb) av[hb] = *(const v4i*)&sPd[hb][m][16 * g];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int tile = wave + 4 * tt;
      if (tile >= DT) continue;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int hb = 0; hb < RBH; ++hb) acc[hb][db][tt] = mfma8(av[hb], bv[tt][db], acc[hb][db][tt]);
    }
  }
#pragma unroll
  for (int r = 0; r < REP; ++r) {
    const uint64_t mm = imie_wave_max_u64(mp[r]);
    if (lane == 0) s_mp[wave][r] = mm;
  }
#pragma unroll
  for (int hb = 0; hb < RBH; ++hb)
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int tile = wave + 4 * tt;
      const int r = 4 * hb + g;
      if (tile >= DT || r >= REP) continue;
      uint64_t o = 0;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) o += (uint64_t)(int64_t)acc[hb][db][tt][i] << (8 * (i + db));
      part[(b * d.H + kv * REP + r) * d.hd + 16 * tile + m] = o;
    }
  __syncthreads();
  if (tid < REP) {
    uint64_t mm = s_mp[0][tid];
    for (int w = 1; w < 4; ++w) mm = s_mp[w][tid] > mm ? s_mp[w][tid] : mm;
    d.cmp[blockIdx.y * rows + b * d.H + kv * REP + tid] = mm;
  }
}

// Prefill scores (M > 1, causal). Workgroup = (b, kv, 16 group rows, 256 keys); wave w takes keys 64w .. 64w+63
// as 4 MFMA tiles of 16. MFMA rows are the 16 query rows; each limb lq is a separate A operand and the products
// are summed per exponent e = lq + b in int32 (|T_e| <= 4 * 2 * 2^20), then S = sum_e T_e << 8e in int64.
constexpr int kPfKeys = 256;
constexpr int kPfTilesPerWg = 8;                      // key tiles per workgroup, all sharing one q setup
__global__ __launch_bounds__(256) void pf_scores8_kernel(AttnDesc d) {
  __shared__ __align__(16) int8_t sQ[8][16][128];
  __shared__ uint64_t s_mq[16];
  __shared__ int64_t s_pm[4][16];
  const int64_t rep = d.H / d.Hkv, grows = rep * d.M;
  const int64_t nrt = (grows + 15) / 16;
  const int64_t bkv = imie_udiv32(blockIdx.x, nrt), rt = imie_umod32(blockIdx.x, nrt);
  const int64_t b = imie_udiv32(bkv, d.Hkv), kv = imie_umod32(bkv, d.Hkv);
  const int64_t rows = d.B * d.H * d.M;
  const int64_t jw = (int64_t)blockIdx.y * kPfKeys * kPfTilesPerWg;
  const int64_t len = d.starts ? d.starts[b] + d.M : d.lengths[b];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, m = lane & 15, g = lane >> 4;
  int64_t vismax = 0;
  for (int i = 0; i < 16; ++i) {
    const int64_t gr = rt * 16 + i;
    if (gr < grows) {
      const int64_t lv = d.starts ? d.starts[b] + imie_umod32(gr, d.M) + 1 : len;
      vismax = lv > vismax ? lv : vismax;
    }
  }
  if (jw >= vismax) return;
  // q rows: thread -> row tid / 16, dims 8 * (tid % 16) .. + 7
  const int qi = tid >> 4, qc = 8 * (tid & 15);
  const int64_t qgr = rt * 16 + qi;
  const bool qrow = qgr < grows;
  const int64_t qr = qrow ? group_row(d, b, kv, qgr) : 0;
  int64_t qv[8];
  uint64_t mq = 0;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    qv[c] = (qrow && qc + c < d.hd) ? d.q[qoff(d, qr) + qc + c] : 0;
    const uint64_t a = imie_absu64(qv[c]);
    mq = a > mq ? a : mq;
  }
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) { const uint64_t w2 = __shfl_xor(mq, o, 64); mq = w2 > mq ? w2 : mq; }
  if ((tid & 15) == 0) s_mq[qi] = mq;
  __syncthreads();
  if (blockIdx.y == 0 && (tid & 15) == 0 && qrow) d.maxq[qr] = mq;
  uint64_t mqa = 0;
  for (int i = 0; i < 16; ++i) mqa = s_mq[i] > mqa ? s_mq[i] : mqa;
  const int Lq = imie_limbs_needed(mqa);
  for (int lq = 0; lq < Lq; ++lq)
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int64_t x = qv[c];
      sQ[lq][qi][qc + c] = (int8_t)bal_digit(x, lq);
    }
  __syncthreads();
  const int KS = (int)((d.hd + 63) / 64);
  // rows of this lane's D values: 4g + i
  int64_t rr[4], lvr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t gr = rt * 16 + 4 * g + i;
    rr[i] = gr < grows ? group_row(d, b, kv, gr) : -1;
    lvr[i] = gr < grows ? (d.starts ? d.starts[b] + imie_umod32(gr, d.M) + 1 : len) : 0;
  }
  const int8_t* Kb = (const int8_t*)d.K;
  for (int kti = 0; kti < kPfTilesPerWg; ++kti) {
    const int64_t kt = (int64_t)blockIdx.y * kPfTilesPerWg + kti, j0 = kt * kPfKeys;
    if (j0 >= vismax) break;                            // uniform: later tiles see no row of this workgroup
    int64_t pm[4] = {INT64_MIN, INT64_MIN, INT64_MIN, INT64_MIN};
    for (int st = 0; st < 4; ++st) {
      const int64_t t = j0 + 64 * wave + 16 * st;
      if (t >= vismax) break;
      const int64_t j = t + m;
      const bool valid = j < len;
      v4i bk[4][2];
      int64_t base = 0, slot = 0;
      if (valid) base = kv8_row_base(d, b, kv, j, &slot) + imie_kv8::k_off(slot, 0, 0, d.hd);
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          bk[db][h] = (valid && h < KS && 64 * h + 16 * g < d.hd)
                          ? *(const v4i*)(Kb + base + imie_kv8::k_piece(db, 64 * h + 16 * g, d.hd))
                          : v4i{0, 0, 0, 0};
      v4i T[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) T[e] = v4i{0, 0, 0, 0};
#pragma unroll
      for (int lq = 0; lq < 8; ++lq) {                  // compile-time limb index: T stays in registers
        if (lq < Lq) {
          v4i a0 = *(const v4i*)&sQ[lq][m][16 * g];
          v4i a1 = KS > 1 ? *(const v4i*)&sQ[lq][m][64 + 16 * g] : v4i{0, 0, 0, 0};
          if (16 * g >= d.hd) a0 = v4i{0, 0, 0, 0};
          if (64 + 16 * g >= d.hd) a1 = v4i{0, 0, 0, 0};
#pragma unroll
          for (int db = 0; db < 4; ++db) {
            if (lq + db >= 8) continue;                 // 256^(lq+db) = 0 mod 2^64
            v4i x = mfma8(a0, bk[db][0], T[lq + db]);
            if (KS > 1) x = mfma8(a1, bk[db][1], x);
            T[lq + db] = x;
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint64_t S = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) S += (uint64_t)(int64_t)T[e][i] << (8 * e);   // 256^e = 0 mod 2^64, e >= 8
        if (rr[i] >= 0 && j < lvr[i]) {
          int64_t sc = (int64_t)S >> d.frac;
          sc = (int64_t)((uint64_t)sc * (uint64_t)d.inv_sqrt) >> d.frac;
          d.scores[rr[i] * d.Lmax + j] = sc;
          pm[i] = sc > pm[i] ? sc : pm[i];
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int64_t mx = pm[i];
#pragma unroll
      for (int o = 8; o >= 1; o >>= 1) { const int64_t w2 = __shfl_xor(mx, o, 64); mx = w2 > mx ? w2 : mx; }
      if (m == 0) s_pm[wave][4 * g + i] = mx;
    }
    __syncthreads();
    if (tid < 16) {
      const int64_t gr = rt * 16 + tid;
      if (gr < grows) {
        int64_t mx = s_pm[0][tid];
        for (int w = 1; w < 4; ++w) mx = s_pm[w][tid] > mx ? s_pm[w][tid] : mx;
        d.pmax[kt * rows + group_row(d, b, kv, gr)] = mx;
      }
    }
    __syncthreads();                                    // s_pm is reused by the next key tile
  }
}

// Prefill softmax (kv8): workgroup per query row; row max from the score kernel's per-256-key maxima; exact e_j, Z,
// p_j = floor((e_j << f) / Z) by a 2^64 / Z reciprocal with correction; p written as Lp digit planes pd[lp][r][j].
__global__ __launch_bounds__(256) void pf_softmax8_kernel(AttnDesc d) {
  __shared__ uint64_t red[256];
  __shared__ int64_t s_m;
  const int64_t r = blockIdx.x;
  const RowInfo ri = row_info(d, r);
  const int tid = threadIdx.x;
  const int64_t rows = d.B * d.H * d.M;
  const int64_t bkv = ri.b * d.Hkv + ri.kv;
  if (tid == 0) {
    const u128 qk = (u128)d.maxq[r] * d.run_k[bkv];
    if (qk > (u128)(INT64_MAX / d.hd)) atomicOr(d.status, IMIE_EOVF);
  }
  const int64_t nkt = (ri.lv + kPfKeys - 1) / kPfKeys;
  int64_t mx = INT64_MIN;
  for (int64_t kt = tid; kt < nkt; kt += 256) { const int64_t v = d.pmax[kt * rows + r]; mx = v > mx ? v : mx; }
  red[tid] = (uint64_t)mx;
  __syncthreads();
  if (tid == 0) {
    int64_t m2 = INT64_MIN;
    for (int i = 0; i < 256; ++i) m2 = (int64_t)red[i] > m2 ? (int64_t)red[i] : m2;
    s_m = m2;
  }
  __syncthreads();
  const int64_t m = s_m;
  int64_t* s = d.scores + r * d.Lmax;
  const bool fx32 = (d.dclip >> 32) == 0 && (d.log2e >> 32) == 0;
  uint64_t z = 0;
  for (int64_t j = tid; j < ri.lv; j += 256) {
    int64_t dd = (int64_t)((uint64_t)m - (uint64_t)s[j]);
    if (dd > d.dclip) dd = d.dclip;
    const int64_t e = exp_clipped(dd, d.frac, d.log2e, fx32);
    s[j] = e;
    z += (uint64_t)e;
  }
  z = (uint64_t)imie_wave_sum_i64((int64_t)z);
  __syncthreads();
  if ((tid & 63) == 0) red[tid >> 6] = z;
  __syncthreads();
  const uint64_t Z = red[0] + red[1] + red[2] + red[3];
  const double rzd = Z != 0 ? 1.0 / (double)Z : 0.0;
  const int Lp = imie_limbs_needed((uint64_t)1 << d.frac);
  uint64_t mp = 0;
  for (int64_t j = tid; j < ri.lv; j += 256) {
    const int64_t p = Z != 0 ? prob_div(s[j], d.frac, Z, rzd) : 0;
    mp = (uint64_t)p > mp ? (uint64_t)p : mp;
    int64_t x = p;
    for (int lp = 0; lp < Lp; ++lp) {
      const int64_t dg = ((x + 128) & 255) - 128;
      x = (int64_t)((uint64_t)x - (uint64_t)dg) >> 8;
      d.pd[((int64_t)lp * rows + r) * d.pdL + j] = (int8_t)dg;
    }
  }
  mp = imie_wave_max_u64(mp);
  __syncthreads();
  if ((tid & 63) == 0) red[tid >> 6] = mp;
  __syncthreads();
  if (tid == 0) {
    uint64_t a = red[0];
    for (int w = 1; w < 4; ++w) a = red[w] > a ? red[w] : a;
    d.maxp[r] = a;
  }
}

// The same softmax with one wave per row (4 rows per workgroup) for rows of at most 64 * kSmPer keys: e_j stay in
// registers between the Z sum and the p pass, every reduction is a whole-wave DPP one (no barriers, no LDS).
constexpr int kSmPer = 32;
__global__ __launch_bounds__(256) void pf_softmax8_wave_kernel(AttnDesc d) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t rows = d.B * d.H * d.M;
  if (r >= rows) return;                              // whole wave
  const RowInfo ri = row_info(d, r);
  const int64_t bkv = ri.b * d.Hkv + ri.kv;
  if (lane == 0) {
    const u128 qk = (u128)d.maxq[r] * d.run_k[bkv];
    if (qk > (u128)(INT64_MAX / d.hd)) atomicOr(d.status, IMIE_EOVF);
  }
  const int64_t nkt = (ri.lv + kPfKeys - 1) / kPfKeys;
  // row max over the score kernel's per-256-key maxima (a set that may not contain 0: offset by INT64_MIN so the
  // unsigned maximum of the shifted values is the signed maximum)
  uint64_t mo = 0;
  for (int64_t kt = lane; kt < nkt; kt += 64) {
    const uint64_t v = (uint64_t)d.pmax[kt * rows + r] ^ 0x8000000000000000ull;
    mo = v > mo ? v : mo;
  }
  const int64_t m = (int64_t)(imie_wave_max_u64_full(mo) ^ 0x8000000000000000ull);
  const int64_t* s = d.scores + r * d.Lmax;
  const bool fx32 = (d.dclip >> 32) == 0 && (d.log2e >> 32) == 0;
  int64_t e[kSmPer];
  uint64_t z = 0;
#pragma unroll
  for (int i = 0; i < kSmPer; ++i) {
    const int64_t j = lane + 64 * i;
    e[i] = 0;
    if (j < ri.lv) {
      int64_t dd = (int64_t)((uint64_t)m - (uint64_t)s[j]);
      if (dd > d.dclip) dd = d.dclip;
      e[i] = exp_clipped(dd, d.frac, d.log2e, fx32);
      z += (uint64_t)e[i];
    }
  }
  const uint64_t Z = imie_wave_sum_u64_full(z);
  const double rzd = Z != 0 ? 1.0 / (double)Z : 0.0;
  const int Lp = imie_limbs_needed((uint64_t)1 << d.frac);
  uint64_t mp = 0;
#pragma unroll
  for (int i = 0; i < kSmPer; ++i) {
    const int64_t j = lane + 64 * i;
    if (j >= ri.lv) continue;
    const int64_t p = Z != 0 ? prob_div(e[i], d.frac, Z, rzd) : 0;
    mp = (uint64_t)p > mp ? (uint64_t)p : mp;
    // p <= 2^frac < 2^30: the balanced digits in 32-bit arithmetic
    int32_t x = (int32_t)p;
#pragma unroll
    for (int lp = 0; lp < 4; ++lp) {                  // Lp <= 4 (frac <= 29)
      if (lp >= Lp) break;
      const int32_t dg = ((x + 128) & 255) - 128;
      x = (x - dg) >> 8;
      d.pd[((int64_t)lp * rows + r) * d.pdL + j] = (int8_t)dg;
    }
  }
  mp = imie_wave_max_u64_full(mp);
  if (lane == 0) d.maxp[r] = mp;
}

// Prefill PV (kv8) + final: workgroup = (b, kv, 16 group rows); wave w owns dim tiles w and w + 4. Per 64-key
// step: A = p digit plane lp of the 16 rows (keys past a row's causal limit masked to 0), B = V digit plane b;
// T_e (e = lp + b) in int32, folded into int64 every 4096 keys (|T_e| < 2^27 before a fold).
__global__ __launch_bounds__(256) void pf_pv8_kernel(AttnDesc d) {
  const int64_t rep = d.H / d.Hkv, grows = rep * d.M;
  const int64_t nrt = (grows + 15) / 16;
  const int64_t bkv = imie_udiv32(blockIdx.x, nrt), rt = imie_umod32(blockIdx.x, nrt);
  const int64_t b = imie_udiv32(bkv, d.Hkv), kv = imie_umod32(bkv, d.Hkv);
  const int64_t rows = d.B * d.H * d.M;
  const int64_t len = d.starts ? d.starts[b] + d.M : d.lengths[b];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, m = lane & 15, g = lane >> 4;
  if (blockIdx.x == 0 && tid == 0) check_rope_guard(d);
  const int64_t agr = rt * 16 + m;                    // A row of this lane
  const bool arow = agr < grows;
  const int64_t ar = arow ? group_row(d, b, kv, agr) : 0;
  const int64_t alv = arow ? (d.starts ? d.starts[b] + imie_umod32(agr, d.M) + 1 : len) : 0;
  int64_t vismax = 0;
  for (int i = 0; i < 16; ++i) {
    const int64_t gr = rt * 16 + i;
    if (gr < grows) {
      const int64_t lv = d.starts ? d.starts[b] + imie_umod32(gr, d.M) + 1 : len;
      vismax = lv > vismax ? lv : vismax;
    }
  }
  const int Lp = imie_limbs_needed((uint64_t)1 << d.frac);
  const int DT = (int)(d.hd / 16);
  v4i T[7][2];
  uint64_t O[2][4];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
    for (int e = 0; e < 7; ++e) T[e][tt] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; ++i) O[tt][i] = 0;
  }
  auto fold = [&]() {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int e = 0; e < 7; ++e) {
#pragma unroll
        for (int i = 0; i < 4; ++i) O[tt][i] += (uint64_t)(int64_t)T[e][tt][i] << (8 * e);
        T[e][tt] = v4i{0, 0, 0, 0};
      }
  };
  const int8_t* Vb = (const int8_t*)d.V;
  int steps = 0;
  for (int64_t t0 = 0; t0 < vismax; t0 += 64) {
    int64_t pi, slot0;
    page_split(d, t0, pi, slot0);
    const int8_t* vblk = Vb + imie_kv8::block_base(d.pt[b * d.mp + pi], kv, d.Hkv, d.hd, d.P);
    const int nv = (int)max((int64_t)0, min((int64_t)16, alv - (t0 + 16 * g)));
#pragma unroll
    for (int lp = 0; lp < 4; ++lp) {                  // Lp <= 4 (frac <= 29): T stays in registers
      if (lp >= Lp) break;
      v4i a = nv > 0 ? *(const v4i*)(d.pd + ((int64_t)lp * rows + ar) * d.pdL + t0 + 16 * g) : v4i{0, 0, 0, 0};
      a = keep_bytes(a, nv);
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int tile = wave + 4 * tt;
        if (tile >= DT) continue;
        const int64_t c = 16 * tile + m;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const v4i bv = *(const v4i*)(vblk + imie_kv8::v_off(slot0 + 16 * g, db, c, d.hd, d.P));
          T[lp + db][tt] = mfma8(a, bv, T[lp + db][tt]);
        }
      }
    }
    if (++steps == 64) { fold(); steps = 0; }
  }
  fold();
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int tile = wave + 4 * tt;
    if (tile >= DT) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t gr = rt * 16 + 4 * g + i;
      if (gr >= grows) continue;
      const int64_t r = group_row(d, b, kv, gr);
      d.out[qoff(d, r) + 16 * tile + m] = (int64_t)O[tt][i] >> d.frac;
      if (tile == 0 && m == 0) {
        const int64_t lv = d.starts ? d.starts[b] + imie_umod32(gr, d.M) + 1 : len;
        const u128 pv = (u128)d.maxp[r] * d.run_v[bkv];
        if (pv > (u128)(INT64_MAX / lv)) atomicOr(d.status, IMIE_EOVF);
      }
    }
  }
}

// Prefill PV (kv8), 64 group rows per workgroup: 8 waves, wave w owns dim tile w (16 dims). The p digits of the
// 64 rows x 64 keys of a step are staged once in LDS (keys past a row's causal limit zeroed); each wave's V
// loads (4 digit planes of its 16 dims) serve all 4 row tiles and all Lp limbs. T_e (e = lp + b) in int32 per row
// tile, folded into int64 every 64 steps (|T_e| < 2^28 before a fold).
constexpr int kPvRows = 64;
__global__ __launch_bounds__(512) void pf_pv8w_kernel(AttnDesc d) {
  __shared__ __align__(16) int8_t sA[4][kPvRows][64];
  __shared__ int64_t s_vis;
  const int64_t rep = d.H / d.Hkv, grows = rep * d.M;
  const int64_t nrt = (grows + kPvRows - 1) / kPvRows;
  const int64_t bkv = imie_udiv32(blockIdx.x, nrt), rt = imie_umod32(blockIdx.x, nrt);
  const int64_t b = imie_udiv32(bkv, d.Hkv), kv = imie_umod32(bkv, d.Hkv);
  const int64_t rows = d.B * d.H * d.M;
  const int64_t len = d.starts ? d.starts[b] + d.M : d.lengths[b];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, m = lane & 15, g = lane >> 4;
  if (blockIdx.x == 0 && tid == 0) check_rope_guard(d);
  // staging role: thread -> (row sr, 8-key chunk sc)
  const int sr = tid >> 3, sc = tid & 7;
  const int64_t sgr = rt * kPvRows + sr;
  const bool srow = sgr < grows;
  const int64_t sar = srow ? group_row(d, b, kv, sgr) : 0;
  const int64_t salv = srow ? (d.starts ? d.starts[b] + imie_umod32(sgr, d.M) + 1 : len) : 0;
  if (tid == 0) s_vis = 0;
  __syncthreads();
  if (sc == 0 && salv > 0) atomicMax((unsigned long long*)&s_vis, (unsigned long long)salv);
  __syncthreads();
  const int64_t vismax = s_vis;
  const int Lp = imie_limbs_needed((uint64_t)1 << d.frac);
  const int DT = (int)(d.hd / 16);
  const bool wt = wave < DT;
  v4i T[4][7];
  uint64_t O[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int e = 0; e < 7; ++e) T[i][e] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int r = 0; r < 4; ++r) O[i][r] = 0;
  }
  auto fold = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 7; ++e) {
#pragma unroll
        for (int r = 0; r < 4; ++r) O[i][r] += (uint64_t)(int64_t)T[i][e][r] << (8 * e);
        T[i][e] = v4i{0, 0, 0, 0};
      }
  };
  const int8_t* Vb = (const int8_t*)d.V;
  int steps = 0;
  for (int64_t t0 = 0; t0 < vismax; t0 += 64) {
    // stage the p digits (masked past each row's visible length)
    {
      const int nvis = (int)max((int64_t)0, min((int64_t)8, salv - (t0 + 8 * sc)));
#pragma unroll
      for (int lp = 0; lp < 4; ++lp) {
        if (lp >= Lp) break;
        uint2 v = uint2{0, 0};
        if (nvis > 0) v = *(const uint2*)(d.pd + ((int64_t)lp * rows + sar) * d.pdL + t0 + 8 * sc);
        const uint32_t m0 = nvis >= 4 ? 0xFFFFFFFFu : ((1u << (8 * nvis)) - 1u);
        const uint32_t m1 = nvis >= 8 ? 0xFFFFFFFFu : (nvis <= 4 ? 0u : ((1u << (8 * (nvis - 4))) - 1u));
        v.x &= m0;
        v.y &= m1;
        *(uint2*)&sA[lp][sr][8 * sc] = v;
      }
    }
    __syncthreads();
    if (wt) {
      int64_t pi, slot0;
      page_split(d, t0, pi, slot0);
      const int8_t* vblk = Vb + imie_kv8::block_base(d.pt[b * d.mp + pi], kv, d.Hkv, d.hd, d.P);
      const int64_t c = 16 * wave + m;
      v4i bv[4];
#pragma unroll
      for (int db = 0; db < 4; ++db) bv[db] = *(const v4i*)(vblk + imie_kv8::v_off(slot0 + 16 * g, db, c, d.hd, d.P));
#pragma unroll
      for (int lp = 0; lp < 4; ++lp) {
        if (lp >= Lp) break;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const v4i a = *(const v4i*)&sA[lp][16 * i + m][16 * g];
#pragma unroll
          for (int db = 0; db < 4; ++db) T[i][lp + db] = mfma8(a, bv[db], T[i][lp + db]);
        }
      }
    }
    if (++steps == 64) { fold(); steps = 0; }
    __syncthreads();                                  // the stage is consumed
  }
  if (!wt) return;
  fold();
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t gr = rt * kPvRows + 16 * i + 4 * g + r;
      if (gr >= grows) continue;
      const int64_t row = group_row(d, b, kv, gr);
      d.out[qoff(d, row) + 16 * wave + m] = (int64_t)O[i][r] >> d.frac;
      if (wave == 0 && m == 0) {
        const int64_t lv = d.starts ? d.starts[b] + imie_umod32(gr, d.M) + 1 : len;
        const u128 pv = (u128)d.maxp[row] * d.run_v[bkv];
        if (pv > (u128)(INT64_MAX / lv)) atomicOr(d.status, IMIE_EOVF);
      }
    }
}

// Prefill attention over the kv8 cache in one launch (M > 1). Workgroup = (b, head h, 16 consecutive query rows);
// wave w takes keys 16 w .. 16 w + 15 of every 64-key step. The integer softmax needs the row maximum before any
// e_j and Z before any p_j, so the keys are walked three times and QK^T is recomputed each time instead of being
// stored: pass 1 the row maxima, pass 2 Z = sum e_j, pass 3 p_j = floor((e_j << f) / Z) as balanced digits into
// LDS and the PV MFMAs (wave w owns dim tiles 2 w, 2 w + 1). Nothing but q, K, V and the outputs touches HBM.
// Scores: per 16-key tile T_e = sum over (q limb lq, K digit db) with lq + db = e of the int8 MFMA products
// (|T_e| < 2^23), S = sum_e T_e << 8 e in int64 (256^e = 0 mod 2^64 for e >= 8), s = ((S >> f) * inv_sqrt) >> f.
// PV: T'_e (e = lp + db) in int32 over up to 64 steps (|T'_e| < 2^28), folded into int64.
constexpr int kFfRows = 16;
// 16 bytes at a wave-uniform base plus a 32-bit lane offset, as a buffer load (the base goes to scalar registers,
// no 64-bit address arithmetic per lane); bytes: the extent of the block read from the base
__device__ inline v4i ld16u(const void* base, uint32_t off, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;                        // wave-uniform by the caller's construction
  const uint64_t u = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a) |
                     ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32)) << 32);
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc((void*)u, (short)0, (int)bytes, 0x00020000);
  return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

// rows padded from 128 to 144 bytes: the 16-byte operand reads of 8 consecutive rows then start in distinct banks
constexpr int kFfPad = 144;
struct FfShared {
  int8_t sQ[8][kFfRows][kFfPad];                               // q digit planes (limb, row, dim)
  int8_t sP[2][4][kFfRows][kFfPad];                            // p digit planes of one key step, double buffer
  uint64_t s_red[8][kFfRows];
  uint64_t s_mq[kFfRows];
};

template <int LQ, int HD, bool F32, int PASSES, int NW>
__device__ __forceinline__ void pf_fused8_body(const AttnDesc& d, FfShared& S, int64_t b, int64_t h, int64_t kv, int64_t pt,
                               int64_t row0, int64_t len);

// MODE 0: head dim 128, frac 16 and tiles whose scores fit the 32-bit form (see pf_fused8_body), the common case;
// a workgroup whose tile does not records it in d.rowmax[workgroup] and leaves the tile to the MODE 1 launch that
// follows, which does only those tiles (or every tile when the head dim is not 128) in general int64 arithmetic.
template <int MODE, int NW>
__global__ __launch_bounds__(64 * NW) void pf_fused8_kernel(AttnDesc d) {
  __shared__ __align__(16) FfShared S;
  if (MODE == 1 && d.hd == 128 && d.rowmax[blockIdx.x] == 0) return;
  if (MODE == 2 && d.rowmax[blockIdx.x] != 0) return;
  auto& sQ = S.sQ;
  auto& s_mq = S.s_mq;
  const int64_t npt = (d.M + kFfRows - 1) / kFfRows;
  const int64_t bh = imie_udiv32(blockIdx.x, npt);
  const int64_t pt = npt - 1 - imie_umod32(blockIdx.x, npt);   // longest rows first
  const int64_t b = imie_udiv32(bh, d.H), h = imie_umod32(bh, d.H), kv = imie_udiv32(h, d.H / d.Hkv);
  const int64_t bkv = b * d.Hkv + kv;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), m = lane & 15, g = lane >> 4;
  if (blockIdx.x == 0 && tid == 0) check_rope_guard(d);
  const int64_t row0 = bh * d.M + pt * kFfRows;                // query row r = (b * H + h) * M + m
  const int64_t len = d.starts ? d.starts[b] + d.M : d.lengths[b];
  auto row_lv = [&](int i) -> int64_t {                         // keys visible to tile row i (0: no row)
    const int64_t mm = pt * kFfRows + i;
    if (mm >= d.M) return 0;
    return d.starts ? d.starts[b] + mm + 1 : len;
  };
  int64_t vis = 0;
  for (int i = 0; i < kFfRows; ++i) vis = max(vis, row_lv(i));
  // q of the tile: thread -> row tid / 16, dims 8 (tid % 16) .. + 7 (threads 0 .. 255); digits of every limb the
  // tile needs
  {
    const int qi = (tid >> 4) & 15, qc = 8 * (tid & 15);
    const bool qrow = tid < 256 && pt * kFfRows + qi < d.M;
    // the tile's rows are consecutive positions of one (b, h): q offsets by stride, no per-row index division
    const int64_t qrow_off = b * d.qsb + h * d.qsh + (pt * kFfRows + qi) * d.qsm;
    int64_t qv[8];
    uint64_t mq = 0;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      qv[c] = (qrow && qc + c < d.hd) ? d.q[qrow_off + qc + c] : 0;
      const uint64_t a = imie_absu64(qv[c]);
      mq = a > mq ? a : mq;
    }
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) { const uint64_t w2 = __shfl_xor(mq, o, 64); mq = w2 > mq ? w2 : mq; }
    if ((tid & 15) == 0 && tid < 256) s_mq[qi] = mq;
    __syncthreads();
    uint64_t mqa = 0;
    for (int i = 0; i < kFfRows; ++i) mqa = s_mq[i] > mqa ? s_mq[i] : mqa;
    const int Lq0 = imie_limbs_needed(mqa);
    // balanced base-256 digits, limb by limb: the digit is the low byte read as int8, and the rest of the value
    // is (x - digit) >> 8; a thread's 8 dims of one limb go to LDS as one 8-byte store
    if (tid < 256)
#pragma unroll
      for (int lq = 0; lq < 8; ++lq) {
        uint64_t pk = 0;
        if (lq < Lq0) {                                        // uniform: limbs above the count are zero
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            pk |= (uint64_t)(uint8_t)qv[c] << (8 * c);
            qv[c] = (int64_t)((uint64_t)qv[c] - (uint64_t)(int64_t)(int8_t)qv[c]) >> 8;
          }
        }
        *(uint64_t*)&sQ[lq][qi][qc] = pk;
      }
    __syncthreads();
  }
  uint64_t mqa = 0;
  for (int i = 0; i < kFfRows; ++i) mqa = s_mq[i] > mqa ? s_mq[i] : mqa;
  const int Lq = imie_limbs_needed(mqa);
  // the limb count is uniform over the workgroup: one specialization per count range (no per-limb predication)
  if (MODE == 0) {
    const int64_t bkv = b * d.Hkv + kv;
    const bool fast = Lq <= 3 && d.frac == 16 && d.inv_sqrt < ((int64_t)1 << 31) && len <= 16384 &&
                      d.dclip >= 0 && d.dclip < ((int64_t)1 << 20) && d.log2e >= 0 && d.log2e < ((int64_t)1 << 17) &&
                      (u128)mqa * d.run_k[bkv] * 128 < ((u128)1 << 47);
    if (tid == 0) d.rowmax[blockIdx.x] = fast ? 0 : 1;
    if (fast) pf_fused8_body<3, 128, true, 1, NW>(d, S, b, h, kv, pt, row0, len);
  } else if (MODE == 2) {
    pf_fused8_body<3, 128, true, 2, NW>(d, S, b, h, kv, pt, row0, len);
  } else {
    pf_fused8_body<8, 0, false, 3, NW>(d, S, b, h, kv, pt, row0, len);  // any hd (multiple of 16, <= 128), any limbs
  }
}

// F32 (frac 16, head dim 128, at most 3 q limbs, 128 max|q| max|K| < 2^47 so |q . k| < 2^47): the scores are formed
// in 32-bit arithmetic. With 3 limbs every T_e sums at most 3 products of 128-term int8 dots (|.| <= 2^21 each),
// so U0 = T0 + 256 T1, U1 = T2 + 256 T3, U2 = T4 + 256 T5 are exact int32 and S = U0 + 2^16 U1 + 2^32 U2; then
// S >> 16 = U1 + 2^16 U2 + (U0 >> 16) fits int32 (evaluated mod 2^32, exact since the result fits) and
// ((S >> 16) * inv_sqrt) >> 16 comes from one 32 x 32 -> 64 product.
// PASSES: 1 = passes 1 and 2 (the row maxima and Z go to d.acc[r] and d.acc[rows + r]), 2 = pass 3 from them,
// 3 = all three in one launch.
// NW waves: wave w scores keys 16 w .. 16 w + 15 of every 16 NW-key step and (pass 3) owns 8 / NW of the 16-dim
// output tiles.
template <int LQ, int HD, bool F32, int PASSES, int NW>
__device__ __forceinline__ void pf_fused8_body(const AttnDesc& d, FfShared& S, int64_t b, int64_t h, int64_t kv, int64_t pt,
                               int64_t row0, int64_t len) {
  constexpr int STEP = 16 * NW, DPW = 8 / NW, KSP = NW / 4;   // keys per step, dim tiles per wave, 64-key K steps
  auto& sQ = S.sQ;
  auto& sP = S.sP;
  auto& s_red = S.s_red;
  auto& s_mq = S.s_mq;
  constexpr int NE = LQ + 3 < 8 ? LQ + 3 : 8;                 // exponents lq + db below 8 (256^8 = 0 mod 2^64)
  // F32: scores, row maxima, Z (at most 16384 keys: Z < 2^30) and p (<= 2^16) in 32 bits, 3 p limbs
  using ST = std::conditional_t<F32, int32_t, int64_t>;
  using UT = std::conditional_t<F32, uint32_t, uint64_t>;
  constexpr ST SMIN = F32 ? (ST)INT32_MIN : (ST)INT64_MIN;
  constexpr UT SBIT = (UT)1 << (8 * sizeof(UT) - 1);
  constexpr int NTP = F32 ? 6 : 7;                             // PV exponents lp + db (lp < 3 when F32)
  const int64_t bkv = b * d.Hkv + kv;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), m = lane & 15, g = lane >> 4;
  auto row_lv = [&](int i) -> int64_t {                         // keys visible to tile row i (0: no row)
    const int64_t mm = pt * kFfRows + i;
    if (mm >= d.M) return 0;
    return d.starts ? d.starts[b] + mm + 1 : len;
  };
  int64_t vis = 0;
  for (int i = 0; i < kFfRows; ++i) vis = max(vis, row_lv(i));
  vis = (int64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)vis) |
        ((int64_t)__builtin_amdgcn_readfirstlane((int)(vis >> 32)) << 32);   // uniform: scalar loop bounds
  const int64_t HDv = HD ? HD : d.hd;                          // head dim (compile-time for the 128 case)
  const int KS = (int)((HDv + 63) / 64);
  int32_t lvr[4];                                              // visible keys of this lane's rows 4 g + i
#pragma unroll
  for (int i = 0; i < 4; ++i) lvr[i] = (int32_t)row_lv(4 * g + i);
  const int8_t* Kb = (const int8_t*)d.K;
  // K digits of the 16-key tile t (keys t .. t + 15 lie in one page: pages hold a multiple of 64 keys and t is a
  // multiple of 16): the page is wave-uniform, lane m takes key t + m
  auto load_k = [&](int64_t t, v4i (&bk)[4][2]) {
    const int64_t tu = (int64_t)__builtin_amdgcn_readfirstlane((int)t);   // wave-uniform: scalar page arithmetic
    int64_t pi, slot;
    page_split(d, tu, pi, slot);
    // wave-uniform 64-bit base (scalar registers) plus 32-bit lane offsets: no 64-bit address arithmetic per load
    const int8_t* kblk = Kb + imie_kv8::block_base(page_id_uniform(d, b, pi), kv, d.Hkv, HDv, d.P) +
                         imie_kv8::k_off(slot, 0, 0, HDv);
    // keys past the sequence length are loaded from their (allocated) slots and masked where the scores are used
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        if (hh >= KS) { bk[db][hh] = v4i{0, 0, 0, 0}; continue; }
        const int c = 64 * hh + 16 * g;
        const uint32_t off = 16u * (uint32_t)m + ((uint32_t)db * (uint32_t)HDv + (uint32_t)(c < HDv ? c : 0)) * 16u;
        const v4i v = ld16u(kblk, off, (uint32_t)(4 * 16 * HDv));
        bk[db][hh] = c < HDv ? v : v4i{0, 0, 0, 0};
      }
    // keeps the loads here: otherwise the scheduler sinks them to their consumer or lifts its MFMAs above them
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };
  // the q digit operands of this lane (row m, dims 16 g .. and 64 + 16 g ..) for every limb: with at most 3 limbs
  // they stay in registers for all passes (24 VGPRs) instead of being read from LDS for every key tile
  constexpr bool QREG = LQ <= 3;
  auto q_operand = [&](int lq, int hh) -> v4i {
    if (hh == 1 && KS < 2) return v4i{0, 0, 0, 0};
    if (64 * hh + 16 * g >= HDv) return v4i{0, 0, 0, 0};
    return *(const v4i*)&sQ[lq][m][64 * hh + 16 * g];
  };
  v4i qreg[QREG ? LQ : 1][2];
#pragma unroll
  for (int lq = 0; lq < (QREG ? LQ : 0); ++lq) {
    qreg[lq][0] = q_operand(lq, 0);
    qreg[lq][1] = q_operand(lq, 1);
  }
  // scores of the lane's 4 rows for key t + m from the tile's K digits; invalid entries INT64_MIN. Transposed
  // (TR, pass 3): the same MFMAs with the operands swapped give S^T, whose lane holds keys t + 4 g + i of row m
  const int32_t lvm = (int32_t)row_lv(m);                      // visible keys of row m
  auto scores = [&](int64_t t, const v4i (&bk)[4][2], ST sc[4], auto tr) {
    constexpr bool TR = decltype(tr)::value;
    const int32_t j = (int32_t)t + (TR ? 4 * g : m);
    v4i T[NE];
#pragma unroll
    for (int e = 0; e < NE; ++e) T[e] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int lq = 0; lq < LQ; ++lq) {                          // limbs above the tile's count hold zero digits
      const v4i a0 = QREG ? qreg[QREG ? lq : 0][0] : q_operand(lq, 0);
      const v4i a1 = QREG ? qreg[QREG ? lq : 0][1] : q_operand(lq, 1);
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        if (lq + db >= NE) continue;
        v4i x = TR ? mfma8(bk[db][0], a0, T[lq + db]) : mfma8(a0, bk[db][0], T[lq + db]);
        if (KS > 1) x = TR ? mfma8(bk[db][1], a1, x) : mfma8(a1, bk[db][1], x);
        T[lq + db] = x;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int64_t s;
      if constexpr (F32) {
        static_assert(NE == 6, "3 q limbs");
        const uint32_t U0 = (uint32_t)T[0][i] + ((uint32_t)T[1][i] << 8);
        const uint32_t U1 = (uint32_t)T[2][i] + ((uint32_t)T[3][i] << 8);
        const uint32_t U2 = (uint32_t)T[4][i] + ((uint32_t)T[5][i] << 8);
        const int32_t V = (int32_t)(U1 + (U2 << 16) + (uint32_t)((int32_t)U0 >> 16));
        s = (int64_t)V * (int32_t)d.inv_sqrt >> 16;
      } else {
        uint64_t Sx = 0;
#pragma unroll
        for (int e = NE - 1; e >= 0; --e) Sx = (Sx << 8) + (uint64_t)(int64_t)T[e][i];
        s = (int64_t)Sx >> d.frac;
        s = (int64_t)((uint64_t)s * (uint64_t)d.inv_sqrt) >> d.frac;
      }
      sc[i] = (TR ? j + i < lvm : j < lvr[i]) ? (ST)s : SMIN;
    }
  };
  // cross-lane (16 keys) and cross-wave reduction of per-row values held as lanes (g, i)
  auto reduce_rows = [&](uint64_t v[4], bool is_max, uint64_t out[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int o = 8; o >= 1; o >>= 1) {
        const uint64_t w2 = (uint64_t)__shfl_xor((int64_t)v[i], o, 64);
        v[i] = is_max ? (w2 > v[i] ? w2 : v[i]) : v[i] + w2;
      }
      if (m == 0) s_red[wave][4 * g + i] = v[i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint64_t a = s_red[0][4 * g + i];
      for (int w = 1; w < NW; ++w) a = is_max ? (s_red[w][4 * g + i] > a ? s_red[w][4 * g + i] : a) : a + s_red[w][4 * g + i];
      out[i] = a;
    }
    __syncthreads();
  };
  // pass 1: row maxima (signed max as the unsigned max of values offset by INT64_MIN)
  // this wave's tiles t = 16 wave, + 64, ... below vis, the next tile's K in flight while one is scored
  // The next tile's loads are issued whatever it is (past vis: the current tile again, whose page is allocated):
  // a load that may be skipped leaves the compiler unable to count the loads in flight, and it then waits for
  // all of them before the MFMAs.
  auto walk = [&](auto&& use) {
    v4i bkA[4][2], bkB[4][2];
    int64_t t = 16 * wave;
    if (t < vis) load_k(t, bkA);
    __builtin_amdgcn_s_waitcnt(0x0F70);             // vmcnt(0): nothing in flight at the loop's entry
    while (t < vis) {
      const int64_t t2 = t + STEP;
      load_k(t2 < vis ? t2 : t, bkB);
      ST sc[4];
      scores(t, bkA, sc, std::false_type{});
      use(sc);
      if (t2 >= vis) break;
      const int64_t t3 = t2 + STEP;
      load_k(t3 < vis ? t3 : t2, bkA);
      scores(t2, bkB, sc, std::false_type{});
      use(sc);
      t = t3;
    }
  };
  ST Mx[4];
  UT Z[4];
  const int64_t rows_all = d.B * d.H * d.M;
  const bool fx32 = (d.dclip >> 32) == 0 && (d.log2e >> 32) == 0;
  auto expv = [&](ST s, int i) -> int64_t {
    if constexpr (F32) {
      // exp2_neg_fixed32 at frac 16 with dclip < 2^20 and log2e < 2^17: every product fits 32 bits. Evaluated
      // for every entry and masked at the end (a select, not a branch per row)
      uint32_t dd = (uint32_t)(Mx[i] - s);
      if (dd > (uint32_t)d.dclip) dd = (uint32_t)d.dclip;
      const uint32_t u = (uint32_t)(((uint64_t)dd * (uint32_t)d.log2e) >> 16);
      const uint32_t k = u >> 16, f = u & 0xFFFFu;
      const uint32_t f2 = (f * f) >> 16, f3 = (f2 * f) >> 16;
      const int32_t poly = 65536 - (int32_t)((45426u * f) >> 16) + (int32_t)((15743u * f2) >> 16) -
                           (int32_t)((3638u * f3) >> 16);
      const uint32_t e = poly <= 0 ? 0u : (uint32_t)poly >> k;   // k < 32 (u < 2^21)
      return (int64_t)(s == SMIN ? 0u : e);
    } else {
      if (s == SMIN) return 0;
      int64_t dd = (int64_t)((uint64_t)Mx[i] - (uint64_t)s);
      if (dd > d.dclip) dd = d.dclip;
      return exp_clipped(dd, d.frac, d.log2e, fx32);
    }
  };
  if constexpr (PASSES != 2) {
  UT mo[4] = {0, 0, 0, 0};
  walk([&](const ST (&sc)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const UT v = (UT)sc[i] ^ SBIT;
      mo[i] = v > mo[i] ? v : mo[i];
    }
  });
  uint64_t M4[4];
  {
    uint64_t mo64[4] = {mo[0], mo[1], mo[2], mo[3]};
    reduce_rows(mo64, true, M4);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) Mx[i] = (ST)((UT)M4[i] ^ SBIT);
  // pass 2: Z
  UT zs[4] = {0, 0, 0, 0};
  walk([&](const ST (&sc)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) zs[i] += (UT)expv(sc[i], i);
  });
  {
    uint64_t z64[4] = {zs[0], zs[1], zs[2], zs[3]}, zo[4];
    reduce_rows(z64, false, zo);
#pragma unroll
    for (int i = 0; i < 4; ++i) Z[i] = (UT)zo[i];
  }
  }
  if constexpr (PASSES == 1) {                                 // hand the row maxima and Z to the pass-3 launch
    if (m == 0)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (lvr[i] == 0 || wave != 0) continue;
        d.acc[row0 + 4 * g + i] = (uint64_t)(int64_t)Mx[i];
        d.acc[rows_all + row0 + 4 * g + i] = (uint64_t)Z[i];
      }
    return;
  }
  // pass 3 works on S^T: each lane's entries belong to row m, whose maximum and Z it needs
  ST Mr;
  UT Zr;
  if constexpr (PASSES == 2) {
    Mr = lvm ? (ST)(int64_t)d.acc[row0 + m] : (ST)0;
    Zr = lvm ? (UT)d.acc[rows_all + row0 + m] : (UT)0;
  } else {
    // row m's values sit in element m & 3 of the lanes with g = m >> 2
    Mr = 0;
    Zr = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const ST mv = (ST)__shfl((int64_t)Mx[i], 16 * (m >> 2), 64);
      const UT zv = (UT)(uint64_t)__shfl((int64_t)(uint64_t)Z[i], 16 * (m >> 2), 64);
      if ((m & 3) == i) { Mr = mv; Zr = zv; }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) { Mx[i] = Mr; Z[i] = Zr; }     // expv / probv read row m's values
  double rz[4];
  float rzf[4];                                                 // F32: 2^16 / Z for the single-precision quotient
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    rz[i] = Zr != 0 ? 1.0 / (double)Zr : 0.0;
    rzf[i] = Zr != 0 ? (float)(65536.0 / (double)Zr) : 0.0f;
  }
  // p = floor((e << frac) / Z). F32 (e <= 2^16, Z < 2^30): the float estimate e * (2^16 / Z) is within 2^-5 of the
  // quotient (< 2^17), so its floor is off by at most one; the remainder (e << 16) - q Z lies in (-Z, 2Z), below
  // 2^31 in magnitude, so it is exact in wrapping 32-bit arithmetic and settles q
  auto probv = [&](int64_t e, int i) -> int64_t {
    if constexpr (F32) {
      uint32_t q = (uint32_t)((float)(uint32_t)e * rzf[i]);
      const int32_t r = (int32_t)(((uint32_t)e << 16) - q * (uint32_t)Z[i]);
      q = r < 0 ? q - 1 : ((uint32_t)r >= (uint32_t)Z[i] ? q + 1 : q);
      return (int64_t)(Z[i] == 0 ? 0u : q);                    // Z = 0: a row with no visible keys
    } else {
      if (Z[i] == 0) return 0;
      return prob_div(e, d.frac, Z[i], rz[i]);
    }
  };
  // pass 3: p digits of each 64-key step into LDS, then PV
  const int Lp = F32 ? 3 : imie_limbs_needed((uint64_t)1 << d.frac);   // <= 4 (frac <= 29); 3 at frac 16
  const int DT = (int)(HDv / 16);
  const int64_t qtile = b * d.qsb + h * d.qsh + pt * kFfRows * d.qsm;   // offset of the tile's first row
  // every wave's dim tiles exist when the waves cover the head dim exactly (head dim 128, 4 waves of 2 tiles)
  constexpr bool ALLT = HD != 0 && 16 * DPW * NW == HD;
  const int8_t* Vb = (const int8_t*)d.V;
  v4i Tp[DPW][NTP];
  uint64_t O[DPW][4];
#pragma unroll
  for (int tt = 0; tt < DPW; ++tt) {
#pragma unroll
    for (int e = 0; e < NTP; ++e) Tp[tt][e] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; ++i) O[tt][i] = 0;
  }
  auto fold = [&]() {
#pragma unroll
    for (int tt = 0; tt < DPW; ++tt)
#pragma unroll
      for (int e = 0; e < NTP; ++e) {
#pragma unroll
        for (int i = 0; i < 4; ++i) O[tt][i] += (uint64_t)(int64_t)Tp[tt][e][i] << (8 * e);
        Tp[tt][e] = v4i{0, 0, 0, 0};
      }
  };
  UT mp[4] = {0, 0, 0, 0};
  int steps = 0, buf = 0;
  // K of this wave's tile and V of the step are loaded one step ahead, into the registers the current step has
  // just consumed: the loads are in flight during the p digits, the barrier and the PV MFMAs
  auto load_v = [&](int64_t t0, v4i (&bv)[DPW][KSP][4]) {
#pragma unroll
    for (int ks = 0; ks < KSP; ++ks) {                         // each 64 keys lie in one page
      // a 64-key block past vis re-reads the step's first block (allocated); its p digits are 0
      const int64_t tw = t0 + 64 * ks < vis ? t0 + 64 * ks : t0;
      const int64_t tu = (int64_t)__builtin_amdgcn_readfirstlane((int)tw);
      int64_t pi, slot0;
      page_split(d, tu, pi, slot0);
      const int8_t* vblk = Vb + imie_kv8::block_base(page_id_uniform(d, b, pi), kv, d.Hkv, HDv, d.P);
      const int8_t* vs = vblk + slot0;                         // uniform; lane offsets below are 32-bit
#pragma unroll
      for (int tt = 0; tt < DPW; ++tt) {
        const int tile = DPW * wave + tt;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const uint32_t off = ((uint32_t)db * (uint32_t)HDv + (uint32_t)(16 * tile + m)) * (uint32_t)d.P + 16u * g;
          bv[tt][ks][db] = (ALLT || tile < DT) ? ld16u(vs, off, (uint32_t)(4 * HDv * d.P)) : v4i{0, 0, 0, 0};
        }
      }
    }
    asm volatile("" ::: "memory");                            // keeps the loads here (see load_k)
    __builtin_amdgcn_sched_barrier(0);
  };
  v4i bk[4][2], bv[DPW][KSP][4];
  if (16 * wave < vis) load_k(16 * wave, bk);
  load_v(0, bv);
  for (int64_t t0 = 0; t0 < vis; t0 += STEP, buf ^= 1) {
    const int64_t t = t0 + 16 * wave;
    ST sc[4] = {SMIN, SMIN, SMIN, SMIN};
    if (t < vis) scores(t, bk, sc, std::true_type{});
    // issued whatever the next step is (past vis: this tile again; see walk)
    load_k(t + STEP < vis ? t + STEP : (t < vis ? t : 16 * wave), bk);
    uint32_t pk[4] = {0, 0, 0, 0};                              // per limb: the digits of keys 4 g .. 4 g + 3
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t e = expv(sc[i], i);
      const int64_t p = probv(e, i);
      mp[0] = (UT)p > mp[0] ? (UT)p : mp[0];
      // balanced base-256 digits of 0 <= p <= 2^frac < 2^30: the bytes of p + 0x80808080, each less 0x80
      const uint32_t dg = ((uint32_t)p + 0x80808080u) ^ 0x80808080u;
#pragma unroll
      for (int lp = 0; lp < 4; ++lp) pk[lp] |= ((dg >> (8 * lp)) & 0xFFu) << (8 * i);
    }
#pragma unroll
    for (int lp = 0; lp < 4; ++lp)                            // one 4-byte store per limb: row m, 4 keys
      if (lp < Lp) *(uint32_t*)&sP[buf][lp][m][16 * wave + 4 * g] = pk[lp];
    __syncthreads();                                          // the step's p digits are in LDS
#pragma unroll
    for (int ks = 0; ks < KSP; ++ks)
#pragma unroll
      for (int lp = 0; lp < 4; ++lp) {
        if (lp >= Lp) break;
        const v4i a = *(const v4i*)&sP[buf][lp][m][64 * ks + 16 * g];
#pragma unroll
        for (int tt = 0; tt < DPW; ++tt) {
          if (!ALLT && DPW * wave + tt >= DT) continue;
#pragma unroll
          for (int db = 0; db < 4; ++db)
            if (lp + db < NTP) Tp[tt][lp + db] = mfma8(a, bv[tt][ks][db], Tp[tt][lp + db]);
        }
      }
    load_v(t0 + STEP < vis ? t0 + STEP : t0, bv);
    if (++steps == 64) { fold(); steps = 0; }
  }
  fold();
  // p maxima of the rows for the PV bound: row m's over the lanes m + 16 g, then per wave into s_red
  {
    uint64_t v = mp[0];
#pragma unroll
    for (int o = 16; o <= 32; o <<= 1) {
      const uint64_t w2 = (uint64_t)__shfl_xor((int64_t)v, o, 64);
      v = w2 > v ? w2 : v;
    }
    if (g == 0) s_red[wave][m] = v;
    __syncthreads();
  }
#pragma unroll
  for (int tt = 0; tt < DPW; ++tt) {
    const int tile = DPW * wave + tt;
    if (tile >= DT) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rr = 4 * g + i;
      if (lvr[i] == 0) continue;
      d.out[qtile + rr * d.qsm + 16 * tile + m] = (int64_t)O[tt][i] >> d.frac;
    }
  }
  if (tid < kFfRows && row_lv(tid) > 0) {
    const int64_t r = row0 + tid;
    d.maxq[r] = s_mq[tid];
    uint64_t mpr = 0;
    for (int w = 0; w < NW; ++w) mpr = s_red[w][tid] > mpr ? s_red[w][tid] : mpr;
    const u128 qk = (u128)s_mq[tid] * d.run_k[bkv];
    if (qk > (u128)(INT64_MAX / d.hd)) atomicOr(d.status, IMIE_EOVF);
    const u128 pv = (u128)mpr * d.run_v[bkv];
    if (pv > (u128)(INT64_MAX / row_lv(tid))) atomicOr(d.status, IMIE_EOVF);
  }
}

// the one-launch prefill attention (IMIE_PF_FUSED=0 selects the three-kernel path; tuning and tests)
bool pf_fused() {
  static const bool v = [] { const char* e = getenv("IMIE_PF_FUSED"); return !(e && atoi(e) == 0); }();
  return v;
}

// prefill PV with 64-row workgroups (IMIE_PV_WIDE=0 selects the 16-row kernel; tuning and tests)
bool pv_wide() {
  static const bool v = [] { const char* e = getenv("IMIE_PV_WIDE"); return !(e && atoi(e) == 0); }();
  return v;
}

// decode chunking: ~4096 workgroups over the (b, kv) groups, chunks of >= 64 keys (multiple of 64). Config 5
// (32 sequences, contexts 1K..32K) measured 41.2 ms a step at 4096, 42.2-42.5 at 2048 / 3072 / 8192, 43.2 at 16384
// and 52.3 at 32768; a single sequence of 4K keys is at the 64-key minimum either way.
void dec_geometry(int64_t B, int64_t Hkv, int64_t Lmax, int64_t* chunk, int64_t* nch) {
  static const int64_t target = [] {               // workgroups to aim for (IMIE_DEC_WGS overrides, tuning)
    const char* e = getenv("IMIE_DEC_WGS");
    const long v = e ? atol(e) : 0;
    return v > 0 ? (int64_t)v : (int64_t)4096;        // config 5 (32 ragged rows): 41.2 ms a step against 42.4 at 8192
  }();
  const int64_t groups = B * Hkv;
  int64_t want = target / (groups > 0 ? groups : 1);
  if (want < 1) want = 1;
  int64_t c = (Lmax + want - 1) / want;
  c = ((c + 63) / 64) * 64;
  if (c < 64) c = 64;
  if (c > 8192) c = 8192;                            // kv8 PV: int32 sums stay below 2^27 per chunk
  *chunk = c;
  *nch = (Lmax + c - 1) / c;
  if (*nch < 1) *nch = 1;
}

}  // namespace

static void attn_set_pshift(AttnDesc& d) {
  d.pshift = -1;
  if (d.P > 0 && (d.P & (d.P - 1)) == 0) { d.pshift = 0; while (((int64_t)1 << d.pshift) < d.P) ++d.pshift; }
}

size_t imie_attn_scratch_bytes(int64_t B, int64_t H, int64_t Hkv, int64_t M, int64_t hd, int64_t Lmax) {
  const int64_t rows = B * H * M;
  int64_t chunk = 0, nch = 0;
  dec_geometry(B, Hkv, Lmax, &chunk, &nch);
  // decode: per-chunk partials + q digit planes (8 * hd bytes per row) and limb counts from the head stage
  const int64_t part = M == 1 ? nch * (rows * hd + 3 * rows + 2 * B * Hkv) + rows * hd + rows + 2 : 0;
  // prefill kv8: per-256-key row maxima + 4 digit planes of p (bytes)
  const int64_t pdL = (Lmax + 15) / 16 * 16;
  const int64_t pf = M > 1 ? ((Lmax + kPfKeys - 1) / kPfKeys) * rows + (4 * rows * pdL + 7) / 8 + 2 : 0;
  return (size_t)(rows * Lmax + rows * hd + rows + 3 * rows + 2 * B * Hkv + part + pf) * 8 + 256;
}

void imie_attn_bind_scratch(AttnDesc& d, void* scratch) {
  const int64_t rows = d.B * d.H * d.M;
  int64_t* p = (int64_t*)scratch;
  d.scores = p;            p += rows * d.Lmax;
  d.acc = (uint64_t*)p;    p += rows * d.hd + rows;   // + Z sums of the decode path
  d.rowmax = p;            p += rows;
  d.maxq = (uint64_t*)p;   p += rows;
  d.maxp = (uint64_t*)p;   p += rows;
  d.maxk = (uint64_t*)p;   p += d.B * d.Hkv;
  d.maxv = (uint64_t*)p;   p += d.B * d.Hkv;
  // decode per-chunk partials (sized by imie_attn_scratch_bytes for M == 1)
  int64_t chunk = 0, nch = 0;
  dec_geometry(d.B, d.Hkv, d.Lmax, &chunk, &nch);
  d.part = (uint64_t*)p;   p += nch * rows * d.hd;
  d.cmax = p;              p += nch * rows;
  d.cz = (uint64_t*)p;     p += nch * rows;
  d.cmp = (uint64_t*)p;    p += nch * rows;
  d.ckm = (uint64_t*)p;    p += nch * d.B * d.Hkv;
  d.cvm = (uint64_t*)p;
  if (d.M > 1) {                                      // prefill kv8 (decode partials are not used)
    p = (int64_t*)d.part;
    d.pmax = p;            p += ((d.Lmax + kPfKeys - 1) / kPfKeys) * rows;
    d.pd = (int8_t*)(((uintptr_t)p + 15) & ~(uintptr_t)15);
    d.pdL = (d.Lmax + 15) / 16 * 16;
  }
}

void imie_attn_qdigit_scratch(const AttnDesc& d, int8_t** qd, int** qlimbs) {
  int64_t chunk = 0, nch = 0;
  dec_geometry(d.B, d.Hkv, d.Lmax, &chunk, &nch);
  const int64_t rows = d.B * d.H * d.M;
  int64_t* p = (int64_t*)d.cvm + nch * d.B * d.Hkv;
  *qd = (int8_t*)(((uintptr_t)p + 15) & ~(uintptr_t)15);
  *qlimbs = (int*)(*qd + rows * 8 * d.hd);
}

int imie_attention_launch(AttnDesc d, hipStream_t st) {
  if (d.frac < 1 || d.frac > 29 || d.H % d.Hkv != 0 || d.hd > 128 || d.hd <= 0) return IMIE_EARG;
  attn_set_pshift(d);
  const int64_t sh = 16 - d.frac;
  d.log2e = sh >= 0 ? (94548 >> sh) : ((int64_t)94548 << -sh);
  const int64_t a = (((int64_t)d.frac + 2) << (2 * d.frac)) / d.log2e, bb = ((int64_t)1 << 62) / d.log2e;
  d.dclip = a < bb ? a : bb;
  const int64_t rows = d.B * d.H * d.M;
  const int64_t grows = (d.H / d.Hkv) * d.M;
  const int64_t nrt = (grows + kRowTile - 1) / kRowTile;
  const int64_t nkt = (d.Lmax + kKeyTile - 1) / kKeyTile;
  const int64_t ninit = rows * d.hd > d.B * d.Hkv ? rows * d.hd : d.B * d.Hkv;
  imie_prof_mark(IMIE_K_ATTN, st, true);
  const int64_t rp = d.H / d.Hkv;
  if (d.M == 1 && (rp == 1 || rp == 2 || rp == 4 || rp == 8) && d.hd <= 128 && d.hd % 32 == 0) {
    dec_geometry(d.B, d.Hkv, d.Lmax, &d.chunk, &d.nch);
    const dim3 gd((unsigned)(d.B * d.Hkv), (unsigned)d.nch);
    const int rep = (int)rp;
#define IMIE_DEC(K_, KT_, R_) hipLaunchKernelGGL((K_<KT_, R_>), gd, dim3(256), 0, st, d)
#define IMIE_DEC_R(K_, KT_)                                                                                \
    if (rep == 1) IMIE_DEC(K_, KT_, 1); else if (rep == 2) IMIE_DEC(K_, KT_, 2);                           \
    else if (rep == 4) IMIE_DEC(K_, KT_, 4); else IMIE_DEC(K_, KT_, 8)
    if (d.kv32) {
#define IMIE_SC8(R_)                                                                                          \
      if (d.hd > 64) hipLaunchKernelGGL((dec_scores8_kernel<R_, 2>), gd, dim3(256), 0, st, d);                \
      else hipLaunchKernelGGL((dec_scores8_kernel<R_, 1>), gd, dim3(256), 0, st, d)
      if (rep == 1) { IMIE_SC8(1); }
      else if (rep == 2) { IMIE_SC8(2); }
      else if (rep == 4) { IMIE_SC8(4); }
      else { IMIE_SC8(8); }
#undef IMIE_SC8
    } else {
      IMIE_DEC_R(dec_scores_kernel, int64_t);
    }
    IMIE_HIP(hipGetLastError());
    // kv8 with several sequences: PV recomputes e from the scores (no write-back of e, the bytes a big batch is
    // bound by); one sequence: e is written back, which keeps the exponentials off PV's per-step latency chain
    const bool recomp = d.kv32 && d.B > 1;
    if (recomp) {
      if (rep == 1) hipLaunchKernelGGL((dec_exp_kernel<1, false>), gd, dim3(256), 0, st, d);
      else if (rep == 2) hipLaunchKernelGGL((dec_exp_kernel<2, false>), gd, dim3(256), 0, st, d);
      else if (rep == 4) hipLaunchKernelGGL((dec_exp_kernel<4, false>), gd, dim3(256), 0, st, d);
      else hipLaunchKernelGGL((dec_exp_kernel<8, false>), gd, dim3(256), 0, st, d);
    } else {
      if (rep == 1) hipLaunchKernelGGL(dec_exp_kernel<1>, gd, dim3(256), 0, st, d);
      else if (rep == 2) hipLaunchKernelGGL(dec_exp_kernel<2>, gd, dim3(256), 0, st, d);
      else if (rep == 4) hipLaunchKernelGGL(dec_exp_kernel<4>, gd, dim3(256), 0, st, d);
      else hipLaunchKernelGGL(dec_exp_kernel<8>, gd, dim3(256), 0, st, d);
    }
    IMIE_HIP(hipGetLastError());
    if (d.kv32 && recomp) {
      if (rep == 1) hipLaunchKernelGGL((dec_pv8_kernel<1, true>), gd, dim3(256), 0, st, d);
      else if (rep == 2) hipLaunchKernelGGL((dec_pv8_kernel<2, true>), gd, dim3(256), 0, st, d);
      else if (rep == 4) hipLaunchKernelGGL((dec_pv8_kernel<4, true>), gd, dim3(256), 0, st, d);
      else hipLaunchKernelGGL((dec_pv8_kernel<8, true>), gd, dim3(256), 0, st, d);
    } else if (d.kv32) {
      if (rep == 1) hipLaunchKernelGGL((dec_pv8_kernel<1, false>), gd, dim3(256), 0, st, d);
      else if (rep == 2) hipLaunchKernelGGL((dec_pv8_kernel<2, false>), gd, dim3(256), 0, st, d);
      else if (rep == 4) hipLaunchKernelGGL((dec_pv8_kernel<4, false>), gd, dim3(256), 0, st, d);
      else hipLaunchKernelGGL((dec_pv8_kernel<8, false>), gd, dim3(256), 0, st, d);
    } else {
      IMIE_DEC_R(dec_pv_kernel, int64_t);
    }
#undef IMIE_DEC_R
#undef IMIE_DEC
    IMIE_HIP(hipGetLastError());
    hipLaunchKernelGGL(dec_final_kernel, dim3((unsigned)((rows * d.hd + 31) / 32 + (rows + 3) / 4)), dim3(256), 0, st,
                       d);
    IMIE_HIP(hipGetLastError());
    imie_prof_mark(IMIE_K_ATTN, st, false);
    return IMIE_OK;
  }
  if (d.kv32) {                                      // kv8 prefill: MFMA scores, softmax to p digits, MFMA PV
    if (d.hd % 16 != 0 || !d.run_k || !d.run_v) return IMIE_EARG;
    if (d.hd <= 128 && pf_fused()) {
      const int64_t npt = (d.M + kFfRows - 1) / kFfRows;
      if (d.hd == 128) {
        hipLaunchKernelGGL((pf_fused8_kernel<0, 4>), dim3((unsigned)(d.B * d.H * npt)), dim3(256), 0, st, d);
        hipLaunchKernelGGL((pf_fused8_kernel<2, 4>), dim3((unsigned)(d.B * d.H * npt)), dim3(256), 0, st, d);
      }
      hipLaunchKernelGGL((pf_fused8_kernel<1, 4>), dim3((unsigned)(d.B * d.H * npt)), dim3(256), 0, st, d);
      IMIE_HIP(hipGetLastError());
      imie_prof_mark(IMIE_K_ATTN, st, false);
      return IMIE_OK;
    }
    const int64_t nrt16 = (grows + 15) / 16, nkt8 = (d.Lmax + kPfKeys - 1) / kPfKeys;
    const int64_t nkg = (nkt8 + kPfTilesPerWg - 1) / kPfTilesPerWg;
    hipLaunchKernelGGL(pf_scores8_kernel, dim3((unsigned)(d.B * d.Hkv * nrt16), (unsigned)nkg), dim3(256), 0, st, d);
    IMIE_HIP(hipGetLastError());
    if (d.Lmax <= 64 * kSmPer)
      hipLaunchKernelGGL(pf_softmax8_wave_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, d);
    else
      hipLaunchKernelGGL(pf_softmax8_kernel, dim3((unsigned)rows), dim3(256), 0, st, d);
    IMIE_HIP(hipGetLastError());
    if (d.hd <= 128 && pv_wide())
      hipLaunchKernelGGL(pf_pv8w_kernel, dim3((unsigned)(d.B * d.Hkv * ((grows + kPvRows - 1) / kPvRows))), dim3(512), 0,
                         st, d);
    else
      hipLaunchKernelGGL(pf_pv8_kernel, dim3((unsigned)(d.B * d.Hkv * nrt16)), dim3(256), 0, st, d);
    IMIE_HIP(hipGetLastError());
    imie_prof_mark(IMIE_K_ATTN, st, false);
    return IMIE_OK;
  }
  hipLaunchKernelGGL(attn_init_kernel, dim3((unsigned)((ninit + 255) / 256)), dim3(256), 0, st, d);
  IMIE_HIP(hipGetLastError());
  const dim3 g2((unsigned)(d.B * d.Hkv * nrt), (unsigned)nkt);
  hipLaunchKernelGGL(attn_scores_kernel<int64_t>, g2, dim3(256), 0, st, d);
  IMIE_HIP(hipGetLastError());
  hipLaunchKernelGGL(attn_softmax_kernel, dim3((unsigned)rows), dim3(256), 0, st, d);
  IMIE_HIP(hipGetLastError());
  hipLaunchKernelGGL(attn_pv_kernel<int64_t>, g2, dim3(256), 0, st, d);
  IMIE_HIP(hipGetLastError());
  hipLaunchKernelGGL(attn_final_kernel, dim3((unsigned)((rows * d.hd + 255) / 256)), dim3(256), 0, st, d);
  IMIE_HIP(hipGetLastError());
  imie_prof_mark(IMIE_K_ATTN, st, false);
  return IMIE_OK;
}

namespace {
struct AttnWs {
  DevBuf q, k, v, out, scratch, meta, status;
} g_aws;
}  // namespace

extern "C" {

// bonsai_q1_gpu.cu:731-797 / gpu_native.py:418-446 `bonsai_attention_prefill_gpu`: q (H, M, hd) post q-norm +
// RoPE, k/v (Hkv, L, hd) with L == start + M, out (H, M, hd). Host pointers, synchronous; rc 2 on the bounds.
int bonsai_attention_prefill_gpu(const int64_t* q, const int64_t* k, const int64_t* v, int64_t H, int64_t Hkv,
                                 int64_t hd, int64_t M, int64_t L, int64_t start, int64_t frac, int64_t inv_sqrt,
                                 int64_t* out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!q || !k || !v || !out || H <= 0 || Hkv <= 0 || H % Hkv || hd <= 0 || hd > 128 || M <= 0 || start < 0 ||
      L != start + M || frac < 1 || frac > 29)
    return IMIE_EARG;
  if (imie_device_ready() != 0) return IMIE_EARG;
  hipStream_t st = imie_stream();
  const size_t qb = (size_t)(H * M * hd) * 8, kb = (size_t)(Hkv * L * hd) * 8;
  const size_t sb = imie_attn_scratch_bytes(1, H, Hkv, M, hd, L);
  if (g_aws.q.ensure(qb) || g_aws.k.ensure(kb) || g_aws.v.ensure(kb) || g_aws.out.ensure(qb) ||
      g_aws.scratch.ensure(sb) || g_aws.meta.ensure(64) || g_aws.status.ensure(64))
    return IMIE_EARG;
  IMIE_HIP(hipMemcpyAsync(g_aws.q.p, q, qb, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemcpyAsync(g_aws.k.p, k, kb, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemcpyAsync(g_aws.v.p, v, kb, hipMemcpyHostToDevice, st));
  int64_t meta[2] = {start, 0};
  IMIE_HIP(hipMemcpyAsync(g_aws.meta.p, meta, 16, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemsetAsync(g_aws.status.p, 0, 4, st));
  AttnDesc d = {};
  d.B = 1; d.H = H; d.Hkv = Hkv; d.hd = hd; d.M = M;
  d.qsb = H * M * hd; d.qsh = M * hd; d.qsm = hd;
  d.q = (const int64_t*)g_aws.q.p;
  d.K = g_aws.k.p; d.V = g_aws.v.p; d.kv32 = 0;
  d.pt = (const int64_t*)g_aws.meta.p + 1;    // page 0 of sequence 0 (meta[1] == 0)
  d.P = L; d.mp = 1;
  d.starts = (const int64_t*)g_aws.meta.p;
  d.Lmax = L; d.frac = (int)frac; d.inv_sqrt = inv_sqrt;
  d.out = (int64_t*)g_aws.out.p; d.status = (int*)g_aws.status.p;
  imie_attn_bind_scratch(d, g_aws.scratch.p);
  int rc = imie_attention_launch(d, st);
  if (rc) return rc;
  int stat = 0;
  IMIE_HIP(hipMemcpyAsync(&stat, g_aws.status.p, 4, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipMemcpyAsync(out, g_aws.out.p, qb, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipStreamSynchronize(st));
  return stat ? IMIE_EOVF : IMIE_OK;
}

// bonsai_q1_gpu.cu:1409-1470 / gpu_native.py:449-468 `bonsai_attention_decode_batched_gpu`: q (B, H, hd), K/V
// padded (B, Hkv, cap, hd), lengths (B,) >= 1, out (B, H, hd). Host pointers, synchronous; rc 2 on the bounds.
int bonsai_attention_decode_batched_gpu(const int64_t* q, const int64_t* K, const int64_t* V, const int64_t* lengths,
                                        int64_t B, int64_t H, int64_t Hkv, int64_t hd, int64_t cap, int64_t frac,
                                        int64_t inv_sqrt, int64_t* out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!q || !K || !V || !lengths || !out || B <= 0 || H <= 0 || Hkv <= 0 || H % Hkv || hd <= 0 || hd > 128 ||
      cap <= 0 || frac < 1 || frac > 29)
    return IMIE_EARG;
  int64_t lmax = 0;
  for (int64_t b = 0; b < B; ++b) {
    if (lengths[b] < 1 || lengths[b] > cap) return IMIE_EARG;
    lmax = lengths[b] > lmax ? lengths[b] : lmax;
  }
  if (imie_device_ready() != 0) return IMIE_EARG;
  hipStream_t st = imie_stream();
  const size_t qb = (size_t)(B * H * hd) * 8, kb = (size_t)(B * Hkv * cap * hd) * 8;
  const size_t sb = imie_attn_scratch_bytes(B, H, Hkv, 1, hd, lmax);
  if (g_aws.q.ensure(qb) || g_aws.k.ensure(kb) || g_aws.v.ensure(kb) || g_aws.out.ensure(qb) ||
      g_aws.scratch.ensure(sb) || g_aws.meta.ensure((size_t)B * 16) || g_aws.status.ensure(64))
    return IMIE_EARG;
  std::vector<int64_t> meta((size_t)(2 * B));
  for (int64_t b = 0; b < B; ++b) { meta[(size_t)b] = lengths[b]; meta[(size_t)(B + b)] = b; }
  IMIE_HIP(hipMemcpyAsync(g_aws.q.p, q, qb, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemcpyAsync(g_aws.k.p, K, kb, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemcpyAsync(g_aws.v.p, V, kb, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemcpyAsync(g_aws.meta.p, meta.data(), (size_t)B * 16, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemsetAsync(g_aws.status.p, 0, 4, st));
  AttnDesc d = {};
  d.B = B; d.H = H; d.Hkv = Hkv; d.hd = hd; d.M = 1;
  d.qsb = H * hd; d.qsh = hd; d.qsm = hd;
  d.q = (const int64_t*)g_aws.q.p;
  d.K = g_aws.k.p; d.V = g_aws.v.p; d.kv32 = 0;
  d.lengths = (const int64_t*)g_aws.meta.p;
  d.pt = (const int64_t*)g_aws.meta.p + B;
  d.P = cap; d.mp = 1;
  d.Lmax = lmax; d.frac = (int)frac; d.inv_sqrt = inv_sqrt;
  d.out = (int64_t*)g_aws.out.p; d.status = (int*)g_aws.status.p;
  imie_attn_bind_scratch(d, g_aws.scratch.p);
  int rc = imie_attention_launch(d, st);
  if (rc) return rc;
  int stat = 0;
  IMIE_HIP(hipMemcpyAsync(&stat, g_aws.status.p, 4, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipMemcpyAsync(out, g_aws.out.p, qb, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipStreamSynchronize(st));
  return stat ? IMIE_EOVF : IMIE_OK;
}

}  // extern "C"

extern "C" {

// Attention stage probe for tests: runs the init + scores kernels of a causal problem (q (H,M,hd), k (Hkv,L,hd),
// L == start + M) and returns the raw scores (H*M, L) and per-row maxima (H*M).
int imie_attention_scores_probe(const int64_t* q, const int64_t* k, int64_t H, int64_t Hkv, int64_t hd, int64_t M,
                                int64_t L, int64_t start, int64_t frac, int64_t inv_sqrt, int64_t* scores,
                                int64_t* rowmax, int stage, int64_t* acc_out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!q || !k || !scores || !rowmax || L != start + M || H % Hkv || hd > 128) return IMIE_EARG;
  if (imie_device_ready() != 0) return IMIE_EARG;
  hipStream_t st = imie_stream();
  const size_t qb = (size_t)(H * M * hd) * 8, kb = (size_t)(Hkv * L * hd) * 8;
  const size_t sb = imie_attn_scratch_bytes(1, H, Hkv, M, hd, L);
  if (g_aws.q.ensure(qb) || g_aws.k.ensure(kb) || g_aws.scratch.ensure(sb) || g_aws.meta.ensure(64) ||
      g_aws.status.ensure(64))
    return IMIE_EARG;
  IMIE_HIP(hipMemcpyAsync(g_aws.q.p, q, qb, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemcpyAsync(g_aws.k.p, k, kb, hipMemcpyHostToDevice, st));
  int64_t meta[2] = {start, 0};
  IMIE_HIP(hipMemcpyAsync(g_aws.meta.p, meta, 16, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemsetAsync(g_aws.scratch.p, 0, sb, st));
  AttnDesc d = {};
  d.B = 1; d.H = H; d.Hkv = Hkv; d.hd = hd; d.M = M;
  d.qsb = H * M * hd; d.qsh = M * hd; d.qsm = hd;
  d.q = (const int64_t*)g_aws.q.p;
  d.K = g_aws.k.p; d.V = g_aws.k.p; d.kv32 = 0;
  d.pt = (const int64_t*)g_aws.meta.p + 1;
  d.P = L; d.mp = 1;
  d.starts = (const int64_t*)g_aws.meta.p;
  d.Lmax = L; d.frac = (int)frac; d.inv_sqrt = inv_sqrt;
  d.status = (int*)g_aws.status.p;
  attn_set_pshift(d);
  imie_attn_bind_scratch(d, g_aws.scratch.p);
  const int64_t rows = H * M, grows = (H / Hkv) * M;
  const int64_t nrt = (grows + kRowTile - 1) / kRowTile, nkt = (L + kKeyTile - 1) / kKeyTile;
  hipLaunchKernelGGL(attn_init_kernel, dim3((unsigned)((rows * hd + 255) / 256)), dim3(256), 0, st, d);
  IMIE_HIP(hipGetLastError());
  hipLaunchKernelGGL(attn_scores_kernel<int64_t>, dim3((unsigned)(Hkv * nrt), (unsigned)nkt), dim3(256), 0, st, d);
  IMIE_HIP(hipGetLastError());
  {
    const int64_t sh = 16 - d.frac;
    d.log2e = sh >= 0 ? (94548 >> sh) : ((int64_t)94548 << -sh);
    const int64_t a = (((int64_t)d.frac + 2) << (2 * d.frac)) / d.log2e, bb = ((int64_t)1 << 62) / d.log2e;
    d.dclip = a < bb ? a : bb;
  }
  if (stage >= 2) {
    hipLaunchKernelGGL(attn_softmax_kernel, dim3((unsigned)rows), dim3(256), 0, st, d);
    IMIE_HIP(hipGetLastError());
  }
  if (stage >= 3) {
    hipLaunchKernelGGL(attn_pv_kernel<int64_t>, dim3((unsigned)(Hkv * nrt), (unsigned)nkt), dim3(256), 0, st, d);
    IMIE_HIP(hipGetLastError());
    IMIE_HIP(hipMemcpyAsync(acc_out, d.acc, (size_t)(rows * hd) * 8, hipMemcpyDeviceToHost, st));
  }
  IMIE_HIP(hipMemcpyAsync(scores, d.scores, (size_t)(rows * L) * 8, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipMemcpyAsync(rowmax, d.rowmax, (size_t)rows * 8, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipStreamSynchronize(st));
  return IMIE_OK;
}

}  // extern "C"
