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

namespace {

typedef unsigned __int128 u128;
constexpr int kRowTile = 16;
constexpr int kKeyTile = 32;   // keeps every kernel's LDS under 64 KB

__device__ inline int64_t rshift_np(int64_t a, int64_t s) {
  if (s < 0 || s >= 64) return a < 0 ? -1 : 0;
  return a >> s;
}

__device__ inline int64_t exp2_neg_fixed(int64_t u, int frac) {
  const int64_t fp = (int64_t)1 << frac;
  const int64_t k = u >> frac, f = u & (fp - 1);
  const int sh = 16 - frac;
  int64_t c0, c1, c2, c3;
  if (sh >= 0) { c0 = 65536 >> sh; c1 = 45426 >> sh; c2 = 15743 >> sh; c3 = 3638 >> sh; }
  else { c0 = (int64_t)65536 << -sh; c1 = (int64_t)45426 << -sh; c2 = (int64_t)15743 << -sh; c3 = (int64_t)3638 << -sh; }
  const int64_t f2 = (int64_t)((uint64_t)f * (uint64_t)f) >> frac;
  const int64_t f3 = (int64_t)((uint64_t)f2 * (uint64_t)f) >> frac;
  int64_t poly = c0 - ((int64_t)((uint64_t)c1 * (uint64_t)f) >> frac) + ((int64_t)((uint64_t)c2 * (uint64_t)f2) >> frac) -
                 ((int64_t)((uint64_t)c3 * (uint64_t)f3) >> frac);
  if (poly < 0) poly = 0;
  return rshift_np(poly, k < 63 ? k : 63);
}

__device__ inline void amax_u64(uint64_t* p, uint64_t v) { atomicMax((unsigned long long*)p, (unsigned long long)v); }
__device__ inline void amax_i64(int64_t* p, int64_t v) { atomicMax((long long*)p, (long long)v); }

struct RowInfo {
  int64_t b, h, m, kv, lv, len;   // len = keys cached for (b): the max|K|/max|V| range
};

__device__ inline RowInfo row_info(const AttnDesc& d, int64_t r) {
  RowInfo ri;
  ri.m = r % d.M;
  ri.h = (r / d.M) % d.H;
  ri.b = r / (d.M * d.H);
  ri.kv = ri.h / (d.H / d.Hkv);
  if (d.starts) {
    ri.lv = d.starts[ri.b] + ri.m + 1;
    ri.len = d.starts[ri.b] + d.M;
  } else {
    ri.lv = d.lengths[ri.b];
    ri.len = ri.lv;
  }
  return ri;
}

template <typename KT>
__device__ inline const KT* key_ptr(const AttnDesc& d, const void* pool, int64_t b, int64_t kv, int64_t j) {
  const int64_t pg = d.pt[b * d.mp + j / d.P];
  return (const KT*)pool + pg * (d.Hkv * d.P * d.hd) + kv * d.P * d.hd + (j % d.P) * d.hd;
}

// rows of one (b, kv) group are ordered h-major: row index within the group g = (h - kv*rep) * M + m.
__device__ inline int64_t group_row(const AttnDesc& d, int64_t b, int64_t kv, int64_t gr) {
  const int64_t rep = d.H / d.Hkv;
  const int64_t hh = gr / d.M, m = gr % d.M;
  return (b * d.H + kv * rep + hh) * d.M + m;
}

// element offset of query row r = ((b * H) + h) * M + m
__device__ inline int64_t qoff(const AttnDesc& d, int64_t r) {
  const int64_t m = r % d.M, h = (r / d.M) % d.H, b = r / (d.M * d.H);
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
  const int64_t b = bkv / d.Hkv, kv = bkv % d.Hkv;
  const int64_t j0 = (int64_t)blockIdx.y * kKeyTile;
  const int64_t len = d.starts ? d.starts[b] + d.M : d.lengths[b];
  if (j0 >= len) return;
  // largest visible key of this row tile (causal: rows are h-major, so take the max m in the tile)
  int64_t vis = len;
  if (d.starts) {
    int64_t mmax = -1;
    for (int i = 0; i < kRowTile; ++i) {
      const int64_t gr = rt * kRowTile + i;
      if (gr < grows) mmax = max(mmax, gr % d.M);
    }
    vis = d.starts[b] + mmax + 1;
  }
  if (j0 >= vis) return;
  const int tid = threadIdx.x;
  // stage q rows and the key tile; max|q| per row, max|K| over cached keys
  for (int i = tid; i < kRowTile * d.hd; i += blockDim.x) {
    const int ri = i / d.hd, c = i % d.hd;
    const int64_t gr = rt * kRowTile + ri;
    sq[ri][c] = gr < grows ? d.q[qoff(d, group_row(d, b, kv, gr)) + c] : 0;
  }
  uint64_t mk = 0;
  for (int i = tid; i < kKeyTile * d.hd; i += blockDim.x) {
    const int ki = i / d.hd, c = i % d.hd;
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
    const int64_t lv = d.starts ? d.starts[b] + (gr % d.M) + 1 : len;
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
  const int64_t b = bkv / d.Hkv, kv = bkv % d.Hkv;
  const int64_t j0 = (int64_t)blockIdx.y * kKeyTile;
  const int64_t len = d.starts ? d.starts[b] + d.M : d.lengths[b];
  if (j0 >= len) return;
  const int tid = threadIdx.x;
  // max|V| over all cached keys (every key tile of the sequence is visited by row tile 0)
  uint64_t mv = 0;
  for (int i = tid; i < kKeyTile * d.hd; i += blockDim.x) {
    const int ki = i / d.hd, c = i % d.hd;
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
      const int64_t lv = d.starts ? d.starts[b] + (gr % d.M) + 1 : len;
      if (j < lv) { p = d.scores[group_row(d, b, kv, gr) * d.Lmax + j]; any = 1; }
    }
    sp[ri][ki] = p;
  }
  if (!__syncthreads_or(any)) return;
  for (int i = tid; i < kRowTile * d.hd; i += blockDim.x) {
    const int ri = i / d.hd, c = i % d.hd;
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
  const int64_t r = i / d.hd;
  d.out[qoff(d, r) + i % d.hd] = (int64_t)d.acc[i] >> d.frac;
  if (i % d.hd == 0) {
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
//   D1 scores : wave = 4 keys x 16 lanes (8 dims per lane, coalesced 512 B rows), rep dots per key, 16-lane
//               shuffle reduction; scores[(b,h)][j]; per-head max via atomicMax
//   D2 exp    : thread per key: e_j = 2^-(...) for each head (stored in place), Z by wave sums + atomicAdd
//   D3 PV     : WG per (b, kv, 256-key chunk): p_j = (e_j << f) / Z through a 2^64 / Z reciprocal with one
//               correction step (exact for e_j << f < 2^40), staged in LDS; lanes split head_dim; int64 partial
//               sums added into acc atomically
//   final     : the shared attn_final_kernel
// ---------------------------------------------------------------------------------------------------------
constexpr int kDecChunk = 256;
constexpr int kMaxRep = 8;

__device__ inline int64_t page_off(const AttnDesc& d, int64_t b, int64_t kv, int64_t j) {
  const int64_t pg = d.pt[b * d.mp + j / d.P];
  return pg * (d.Hkv * d.P * d.hd) + kv * d.P * d.hd + (j % d.P) * d.hd;
}

template <typename KT, int REP>
__global__ __launch_bounds__(256) void dec_scores_kernel(AttnDesc d) {
  const int64_t bkv = blockIdx.x, b = bkv / d.Hkv, kv = bkv % d.Hkv;
  const int64_t L = d.starts ? d.starts[b] + 1 : d.lengths[b];
  const int64_t j0 = (int64_t)blockIdx.y * kDecChunk;
  if (j0 >= L) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane >> 4, l16 = lane & 15;          // key within the 4-key group, lane within the key
  const bool dims = l16 * 8 < d.hd;
  // this lane's 8 dims of the group's REP query rows
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
  const int64_t jend = min(j0 + kDecChunk, L);
  for (int64_t jj = j0 + wave * 4; jj < jend; jj += 16) {
    const int64_t j = jj + sub;
    const bool live = j < jend;
    int64_t kvv[8];
    if (live && dims) {
      const KT* kp = (const KT*)d.K + page_off(d, b, kv, j) + l16 * 8;
#pragma unroll
      for (int c = 0; c < 8; ++c) kvv[c] = (int64_t)kp[c];
    } else {
#pragma unroll
      for (int c = 0; c < 8; ++c) kvv[c] = 0;
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) { const uint64_t a = imie_absu64(kvv[c]); mk = a > mk ? a : mk; }
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      uint64_t dot = 0;
#pragma unroll
      for (int c = 0; c < 8; ++c) dot += (uint64_t)q[r][c] * (uint64_t)kvv[c];
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
  mk = imie_wave_max_u64(mk);
  if (lane == 0) amax_u64(&d.maxk[bkv], mk);
#pragma unroll
  for (int r = 0; r < REP; ++r) {
    int64_t m = smax[r];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) { const int64_t w = __shfl_xor(m, o, 64); m = w > m ? w : m; }
    if (lane == 0 && m != INT64_MIN) amax_i64(&d.rowmax[b * d.H + kv * REP + r], m);
  }
}

__global__ __launch_bounds__(256) void dec_exp_kernel(AttnDesc d) {
  const int64_t bkv = blockIdx.x, b = bkv / d.Hkv, kv = bkv % d.Hkv;
  const int rep = (int)(d.H / d.Hkv);
  const int64_t L = d.starts ? d.starts[b] + 1 : d.lengths[b];
  const int64_t j = (int64_t)blockIdx.y * kDecChunk + threadIdx.x;
  if ((int64_t)blockIdx.y * kDecChunk >= L) return;
  const int lane = threadIdx.x & 63;
  for (int r = 0; r < rep; ++r) {
    const int64_t row = b * d.H + kv * rep + r;
    uint64_t e = 0;
    if (j < L) {
      int64_t dd = (int64_t)((uint64_t)d.rowmax[row] - (uint64_t)d.scores[row * d.Lmax + j]);
      if (dd > d.dclip) dd = d.dclip;
      e = (uint64_t)exp2_neg_fixed((int64_t)((uint64_t)dd * (uint64_t)d.log2e) >> d.frac, d.frac);
      d.scores[row * d.Lmax + j] = (int64_t)e;
    }
    uint64_t z = e;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) z += (uint64_t)__shfl_xor((int64_t)z, o, 64);
    if (lane == 0 && z) atomicAdd((unsigned long long*)&d.acc[d.B * d.H * d.M * d.hd + row], (unsigned long long)z);
  }
}

template <typename KT>
__global__ __launch_bounds__(256) void dec_pv_kernel(AttnDesc d) {
  __shared__ int64_t sp[kMaxRep][kDecChunk];
  __shared__ uint64_t red[4][kMaxRep][128];
  const int64_t bkv = blockIdx.x, b = bkv / d.Hkv, kv = bkv % d.Hkv;
  const int rep = (int)(d.H / d.Hkv);
  const int64_t L = d.starts ? d.starts[b] + 1 : d.lengths[b];
  const int64_t j0 = (int64_t)blockIdx.y * kDecChunk;
  if (j0 >= L) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint64_t* Zs = d.acc + d.B * d.H * d.M * d.hd;
  // p for this chunk (exact floor((e << f) / Z) via reciprocal + one correction), max|p| per head
  for (int r = 0; r < rep; ++r) {
    const int64_t row = b * d.H + kv * rep + r;
    const uint64_t Z = Zs[row];
    const uint64_t rz = Z > 1 ? (~(uint64_t)0) / Z : 0;
    const int64_t j = j0 + tid;
    int64_t p = 0;
    if (j < L && Z != 0) {
      const uint64_t num = (uint64_t)d.scores[row * d.Lmax + j] << d.frac;
      if (Z == 1) p = (int64_t)num;
      else {
        uint64_t qq = __umul64hi(num, rz);
        if (num - qq * Z >= Z) ++qq;
        p = (int64_t)qq;
      }
    }
    sp[r][tid] = p;
    uint64_t m = (uint64_t)p;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) { const uint64_t w = __shfl_xor(m, o, 64); m = w > m ? w : m; }
    if (lane == 0 && m) amax_u64(&d.maxp[row], m);
  }
  __syncthreads();
  // PV: wave w takes keys j0 + w, w + 4, ...; lane covers dims 2*lane, 2*lane+1
  uint64_t acc[kMaxRep][2];
#pragma unroll
  for (int r = 0; r < kMaxRep; ++r) acc[r][0] = acc[r][1] = 0;
  uint64_t mv = 0;
  const int c0 = 2 * lane;
  for (int i = wave; i < kDecChunk && j0 + i < L; i += 4) {
    const int64_t j = j0 + i;
    const KT* vp = (const KT*)d.V + page_off(d, b, kv, j);
    const int64_t v0 = c0 < d.hd ? (int64_t)vp[c0] : 0, v1 = c0 + 1 < d.hd ? (int64_t)vp[c0 + 1] : 0;
    const uint64_t a0 = imie_absu64(v0), a1 = imie_absu64(v1);
    mv = a0 > mv ? a0 : mv;
    mv = a1 > mv ? a1 : mv;
#pragma unroll
    for (int r = 0; r < kMaxRep; ++r) {
      if (r >= rep) break;
      const uint64_t pp = (uint64_t)sp[r][i];
      acc[r][0] += pp * (uint64_t)v0;
      acc[r][1] += pp * (uint64_t)v1;
    }
  }
  mv = imie_wave_max_u64(mv);
  if (lane == 0) amax_u64(&d.maxv[bkv], mv);
  for (int r = 0; r < rep; ++r) {
    if (c0 < 128) { red[wave][r][c0] = acc[r][0]; if (c0 + 1 < 128) red[wave][r][c0 + 1] = acc[r][1]; }
  }
  __syncthreads();
  for (int i = tid; i < rep * d.hd; i += blockDim.x) {
    const int r = i / (int)d.hd, c = i % (int)d.hd;
    const uint64_t v = red[0][r][c] + red[1][r][c] + red[2][r][c] + red[3][r][c];
    if (v) atomicAdd((unsigned long long*)&d.acc[(b * d.H + kv * rep + r) * d.hd + c], (unsigned long long)v);
  }
}

__global__ void dec_init_kernel(AttnDesc d) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t rows = d.B * d.H;
  if (i < rows * d.hd + rows) d.acc[i] = 0;          // PV accumulators then the Z sums
  if (i < rows) { d.rowmax[i] = INT64_MIN; d.maxp[i] = 0; }
  if (i < d.B * d.Hkv) { d.maxk[i] = 0; d.maxv[i] = 0; }
}

}  // namespace

size_t imie_attn_scratch_bytes(int64_t B, int64_t H, int64_t Hkv, int64_t M, int64_t hd, int64_t Lmax) {
  const int64_t rows = B * H * M;
  return (size_t)(rows * Lmax + rows * hd + rows + 3 * rows + 2 * B * Hkv) * 8 + 256;
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
  d.maxv = (uint64_t*)p;
}

int imie_attention_launch(AttnDesc d, hipStream_t st) {
  if (d.frac < 1 || d.frac > 29 || d.H % d.Hkv != 0 || d.hd > 128 || d.hd <= 0) return IMIE_EARG;
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
  if (d.M == 1 && (rp == 1 || rp == 2 || rp == 4 || rp == 8) && d.hd <= 128) {
    const int64_t nch = (d.Lmax + kDecChunk - 1) / kDecChunk;
    const dim3 gd((unsigned)(d.B * d.Hkv), (unsigned)nch);
    const int64_t ni = rows * d.hd + rows;
    hipLaunchKernelGGL(dec_init_kernel, dim3((unsigned)((ni + 255) / 256)), dim3(256), 0, st, d);
    IMIE_HIP(hipGetLastError());
    const int rep = (int)(d.H / d.Hkv);
#define IMIE_DEC_SCORES(KT_, R_) hipLaunchKernelGGL((dec_scores_kernel<KT_, R_>), gd, dim3(256), 0, st, d)
#define IMIE_DEC_SCORES_R(KT_)                                                                             \
    if (rep == 1) IMIE_DEC_SCORES(KT_, 1); else if (rep == 2) IMIE_DEC_SCORES(KT_, 2);                     \
    else if (rep <= 4 && rep % 4 == 0) IMIE_DEC_SCORES(KT_, 4); else IMIE_DEC_SCORES(KT_, 8)
    if (rep != 1 && rep != 2 && rep != 4 && rep != 8) return IMIE_EARG;
    if (d.kv32) { IMIE_DEC_SCORES_R(int32_t); } else { IMIE_DEC_SCORES_R(int64_t); }
#undef IMIE_DEC_SCORES_R
#undef IMIE_DEC_SCORES
    IMIE_HIP(hipGetLastError());
    hipLaunchKernelGGL(dec_exp_kernel, gd, dim3(256), 0, st, d);
    IMIE_HIP(hipGetLastError());
    if (d.kv32) hipLaunchKernelGGL(dec_pv_kernel<int32_t>, gd, dim3(256), 0, st, d);
    else hipLaunchKernelGGL(dec_pv_kernel<int64_t>, gd, dim3(256), 0, st, d);
    IMIE_HIP(hipGetLastError());
    hipLaunchKernelGGL(attn_final_kernel, dim3((unsigned)((rows * d.hd + 255) / 256)), dim3(256), 0, st, d);
    IMIE_HIP(hipGetLastError());
    imie_prof_mark(IMIE_K_ATTN, st, false);
    return IMIE_OK;
  }
  hipLaunchKernelGGL(attn_init_kernel, dim3((unsigned)((ninit + 255) / 256)), dim3(256), 0, st, d);
  IMIE_HIP(hipGetLastError());
  const dim3 g2((unsigned)(d.B * d.Hkv * nrt), (unsigned)nkt);
  if (d.kv32) hipLaunchKernelGGL(attn_scores_kernel<int32_t>, g2, dim3(256), 0, st, d);
  else hipLaunchKernelGGL(attn_scores_kernel<int64_t>, g2, dim3(256), 0, st, d);
  IMIE_HIP(hipGetLastError());
  hipLaunchKernelGGL(attn_softmax_kernel, dim3((unsigned)rows), dim3(256), 0, st, d);
  IMIE_HIP(hipGetLastError());
  if (d.kv32) hipLaunchKernelGGL(attn_pv_kernel<int32_t>, g2, dim3(256), 0, st, d);
  else hipLaunchKernelGGL(attn_pv_kernel<int64_t>, g2, dim3(256), 0, st, d);
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
