// north-mini-code Q4_K / Q6_K integer linear and the ragged grouped MoE FFN for gfx950.
//
// Semantics (reference: north-mini-code/src/nmc/qk_codec.py:28-206, cohere2.py:102-111, :168-188; producer
// north-mini-code/tools/nmc_qk_cuda.cu:92-237, :2184-2254):
//   y[t, o] = floor( sum_i W[o, i] * x[t, i] / 2^fw )   exactly (big-int in the oracle), W = dequantized block
//   Q4_K (144 B): W = dq*sc_j*q - dmq*m_j, sub-blocks of 32; Q6_K (210 B): W = dq*sc_j*(q6 - 32), sub-blocks of 16
//   dq = round_half_even(fp16 * 2^fw) from the fp16 bits in integer arithmetic (exact; no libm, no FP rounding).
// Evaluation: per sub-block j, sum_i W x = (dq*sc_j) * qdot_j - (dmq*m_j) * xsum_j with qdot_j = sum q*x in
// int64 (|x| < 2^52 keeps it exact; larger staged values take an int128 path), the products and the running sum in
// int128. A result that does not fit int64 (the oracle's astype would raise) sets status bit 2.
//
// Work: a workgroup = (weight group, 64-row tile); the x rows routed to that weight are staged block by block in
// LDS (16 rows per pass) and 4 threads per output row each own a quarter of them, so every weight block is read
// from HBM once per call no matter how many tokens use it.
#include "imie_common.h"
#include "imie_kernels.h"
#include <string.h>
#include <stdlib.h>
#include <algorithm>
#include <map>
#include <tuple>

namespace {

typedef __int128 i128;
constexpr int kRows = 64;        // output rows per workgroup
constexpr int kXRows = 16;       // staged x rows per pass (4 per thread)
// dq * sc * q must fit int64 for every finite fp16 scale (as the oracle's int64 weight arrays require)
constexpr int kMaxFw = 36;

struct QKWeight {
  uint8_t* p = nullptr;
  int64_t out_f = 0, nb = 0;
  int qtype = 0;
  size_t bytes = 0;
};
std::vector<QKWeight> g_qk;
int64_t g_qk_live = 0;

// profile counters (qk_cuda.py:24-34 metric order)
enum { PM_REG_CALLS, PM_REG_NS, PM_H2D_CALLS, PM_H2D_BYTES, PM_H2D_NS, PM_D2H_CALLS, PM_D2H_BYTES, PM_D2H_NS,
       PM_ALLOC_CALLS, PM_ALLOC_BYTES, PM_ALLOC_NS, PM_FREE_CALLS, PM_NATIVE_CALLS, PM_RESIDENT_CALLS,
       PM_GROUPED_CALLS, PM_MOE_CALLS, PM_MOE_BATCHED_CALLS, PM_MOE_BATCHED_DP4A_CALLS, PM_Q_CALLS, PM_Q_NS,
       PM_K_CALLS, PM_K_NS, PM_V_CALLS, PM_V_NS, PM_O_CALLS, PM_O_NS, PM_OTHER_CALLS, PM_OTHER_NS, PM_COUNT };
unsigned long long g_prof[PM_COUNT];
int g_prof_on = 0;
inline void prof(int k, unsigned long long v = 1) { if (g_prof_on) g_prof[k] += v; }

struct MoeWs {
  DevBuf items, pairs, x, y, g, u, d, out, gates, status, tok;
  int64_t grows = 0;
} g_mws;

// round(fp16 h * 2^fw) to the nearest integer, ties to even, without branches (lanes of different rows take
// different exponents): a normal h is (1024 + mant) 2^(e - 25), a subnormal mant 2^-24. A left shift (sh >= 0) is
// exact; a right shift by s rounds m >> s with the remainder against half; every shift of 12 or more gives 0 (m <
// 2^11), so s is clamped to 12, as the 32-bit remainder arithmetic needs.
__device__ inline int64_t fp16_fixed(uint32_t h, int fw) {
  const uint32_t e = (h >> 10) & 31, mant = h & 0x3FF;
  const uint32_t m = e == 0 ? mant : (mant | 0x400);
  const int sh = (e == 0 ? 1 : (int)e) - 25 + fw;
  const int64_t rp = (int64_t)m << (sh > 0 ? sh : 0);
  const uint32_t s = sh < 0 ? (uint32_t)(-sh < 12 ? -sh : 12) : 1u;
  const uint32_t q = m >> s, rem = m & ((1u << s) - 1u), half = 1u << (s - 1u);
  const uint32_t rn = q + ((rem > half || (rem == half && (q & 1u))) ? 1u : 0u);
  const int64_t r = sh >= 0 ? rp : (int64_t)rn;
  return ((h >> 15) & 1) ? -r : r;
}

// fp16_fixed with the right-shift rounding done by the float unit: m 2^sh for sh < 0 is exact in single precision
// (m < 2^11) and rint rounds it half to even like the integer rule (values below one half, where the integer rule
// clamps its shift, round to 0 either way); sh >= 0 is the exact left shift. Branch-free, about half the integer
// rule's instructions; exponent 31 is treated as finite exactly as there.
__device__ inline int64_t fp16_fixed_fast(uint32_t h, int fw) {
  const uint32_t e = (h >> 10) & 31, mant = h & 0x3FF;
  const uint32_t m = e == 0 ? mant : (mant | 0x400);
  const int sh = (e == 0 ? 1 : (int)e) - 25 + fw;
  const int64_t up = (int64_t)((uint64_t)m << (sh > 0 ? sh : 0));
  const int64_t dn = (int64_t)(uint32_t)__builtin_rintf(__builtin_ldexpf((float)m, sh < 0 ? sh : 0));
  const int64_t r = sh >= 0 ? up : dn;
  return ((h >> 15) & 1) ? -r : r;
}

__global__ void fp16_fixed_probe_kernel(const uint16_t* __restrict__ h, int64_t n, int fw, int64_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = fp16_fixed_fast(h[i], fw);
}

struct Item {               // one weight applied to `count` x rows
  const uint8_t* w;
  int64_t out_f, nb;
  int qtype;
  int first, count;         // into the pair arrays
};

// y[yi[p]][o] = floor(W[o] . x[xi[p]] / 2^fw) for the pairs of one item.
// run_gate (nullable): the launch runs only when *run_gate != 0 (the MFMA path found activations it cannot take)
// One (64-row tile bx, item by) of the exact int128 kernel; every thread of the workgroup calls it with the same
// (bx, by).
__device__ void qk_group_tile(const Item* __restrict__ items, const int* __restrict__ xi, const int* __restrict__ yi,
                              const int64_t* __restrict__ X, int64_t K, int64_t* __restrict__ Y, int64_t ldy, int fw,
                              int* __restrict__ status, int64_t bx, int64_t by) {
  __shared__ int64_t sx[kXRows][257];
  __shared__ int s_wide;
  const Item it = items[by];
  const int64_t o = bx * kRows + (threadIdx.x >> 2);
  if (bx * kRows >= it.out_f) return;
  const int slot = threadIdx.x & 3;
  const bool live = o < it.out_f;
  const int bs = it.qtype == 0 ? 144 : 210;
  const uint8_t* row = it.w + (live ? o : 0) * it.nb * bs;
  for (int c0 = 0; c0 < it.count; c0 += kXRows) {
    const int cn = min(kXRows, it.count - c0);
    i128 acc[4] = {0, 0, 0, 0};
    for (int64_t b = 0; b < it.nb; ++b) {
      __syncthreads();
      if (threadIdx.x == 0) s_wide = 0;
      __syncthreads();
      int wide = 0;
      for (int i = threadIdx.x; i < cn * 256; i += blockDim.x) {
        const int r = i >> 8, c = i & 255;
        const int64_t v = X[(int64_t)xi[it.first + c0 + r] * K + b * 256 + c];
        sx[r][c] = v;
        if (v >= ((int64_t)1 << 52) || v <= -((int64_t)1 << 52)) wide = 1;
      }
      if (wide) s_wide = 1;
      __syncthreads();
      const bool fast = s_wide == 0;
      const uint8_t* blk = row + b * bs;
      if (it.qtype == 0) {
        const int64_t dq = fp16_fixed_fast(blk[0] | (blk[1] << 8), fw), dmq = fp16_fixed_fast(blk[2] | (blk[3] << 8), fw);
        const uint8_t* sc = blk + 4;
        const uint8_t* qs = blk + 16;
#pragma unroll 1
        for (int j = 0; j < 8; ++j) {
          int s, m;
          if (j < 4) { s = sc[j] & 63; m = sc[j + 4] & 63; }
          else { s = (sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4); m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4); }
          const int64_t ds = dq * s, dm = dmq * m;
          const int g = j >> 1, hi = j & 1;
          uint8_t q[32];
#pragma unroll
          for (int l = 0; l < 32; ++l) q[l] = hi ? (qs[32 * g + l] >> 4) : (qs[32 * g + l] & 0xF);
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int r = slot + 4 * k;
            if (r >= cn) break;
            const int64_t* xv = &sx[r][32 * j];
            if (fast) {
              int64_t qd = 0, xs = 0;
#pragma unroll
              for (int l = 0; l < 32; ++l) { qd += (int64_t)q[l] * xv[l]; xs += xv[l]; }
              acc[k] += (i128)ds * qd - (i128)dm * xs;
            } else {
              i128 qd = 0, xs = 0;
              for (int l = 0; l < 32; ++l) { qd += (i128)q[l] * xv[l]; xs += xv[l]; }
              acc[k] += (i128)ds * qd - (i128)dm * xs;
            }
          }
        }
      } else {
        const uint8_t* ql = blk;
        const uint8_t* qh = blk + 128;
        const int8_t* sc = (const int8_t*)(blk + 192);
        const int64_t dq = fp16_fixed_fast(blk[208] | (blk[209] << 8), fw);
#pragma unroll 1
        for (int j = 0; j < 16; ++j) {
          // sub-block j covers positions 16 j .. 16 j + 15: half = j / 8, quarter qq = (j % 8) / 2, is = j % 2
          const int half = j >> 3, qq = (j & 7) >> 1, is = j & 1;
          const int qlo = 64 * half, qho = 32 * half;
          const int64_t ds = dq * sc[8 * half + is + 2 * qq];
          int8_t q[16];
#pragma unroll
          for (int l0 = 0; l0 < 16; ++l0) {
            const int l = 16 * is + l0;
            int v;
            if (qq == 0) v = (ql[qlo + l] & 0xF) | (((qh[qho + l] >> 0) & 3) << 4);
            else if (qq == 1) v = (ql[qlo + l + 32] & 0xF) | (((qh[qho + l] >> 2) & 3) << 4);
            else if (qq == 2) v = (ql[qlo + l] >> 4) | (((qh[qho + l] >> 4) & 3) << 4);
            else v = (ql[qlo + l + 32] >> 4) | (((qh[qho + l] >> 6) & 3) << 4);
            q[l0] = (int8_t)(v - 32);
          }
          const int pos0 = 128 * half + 32 * qq + 16 * is;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int r = slot + 4 * k;
            if (r >= cn) break;
            const int64_t* xv = &sx[r][pos0];
            if (fast) {
              int64_t qd = 0;
#pragma unroll
              for (int l = 0; l < 16; ++l) qd += (int64_t)q[l] * xv[l];
              acc[k] += (i128)ds * qd;
            } else {
              i128 qd = 0;
              for (int l = 0; l < 16; ++l) qd += (i128)q[l] * xv[l];
              acc[k] += (i128)ds * qd;
            }
          }
        }
      }
    }
    if (live) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int r = slot + 4 * k;
        if (r >= cn) break;
        const i128 y = acc[k] >> fw;
        if (y > (i128)INT64_MAX || y < (i128)INT64_MIN) atomicOr(status, IMIE_EOVF);
        Y[(int64_t)yi[it.first + c0 + r] * ldy + o] = (int64_t)y;
      }
    }
  }
}

__global__ __launch_bounds__(256) void qk_group_kernel(const Item* __restrict__ items, const int* __restrict__ xi,
                                                       const int* __restrict__ yi, const int64_t* __restrict__ X,
                                                       int64_t K, int64_t* __restrict__ Y, int64_t ldy, int fw,
                                                       int* __restrict__ status, const int* __restrict__ run_gate) {
  if (run_gate && *run_gate == 0) return;
  qk_group_tile(items, xi, yi, X, K, Y, ldy, fw, status, blockIdx.x, blockIdx.y);
}

// The exact kernel as the fallback of a fused MoE stage: a small grid that ends at once unless the prep flagged a
// wide activation row (*run_gate != 0); then its workgroups walk all (tile, item) pairs, ntx tiles per item.
constexpr int kGatedWgs = 128;
__global__ __launch_bounds__(256) void qk_group_gated_kernel(const Item* __restrict__ items, const int* __restrict__ xi,
                                                             const int* __restrict__ yi, const int64_t* __restrict__ X,
                                                             int64_t K, int64_t* __restrict__ Y, int64_t ldy, int fw,
                                                             int* __restrict__ status, const int* __restrict__ run_gate,
                                                             int64_t ntx, int64_t ne) {
  if (*run_gate == 0) return;
  for (int64_t t = blockIdx.x; t < ntx * ne; t += gridDim.x) {
    qk_group_tile(items, xi, yi, X, K, Y, ldy, fw, status, t % ntx, t / ntx);
    __syncthreads();                                  // the tile's shared buffers are free for the next one
  }
}

// nmc SiLU*up: g <- ((g * sigmoid(g)) >> fa) exactly, then gu = (g * u) >> fa exactly (cohere2.py:109-111,
// :183-185); sigmoid without the (1<<62)/log2e cap (north-mini-code/src/nmc/_bonsai/fixedpoint.py:148).
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
  if (k < 0) return 0;
  return poly >> (k < 63 ? k : 63);
}

// (silu(x) * u) >> fa in int128 with the int64 range checks (status bit 2)
__device__ inline int64_t qk_silu_elem(int64_t x, int64_t u, int fa, int64_t log2e, int64_t dclip, int* status) {
  const int64_t m = x > 0 ? x : 0;
  int64_t d0 = m, d1 = (int64_t)((uint64_t)m - (uint64_t)x);
  if (d0 > dclip) d0 = dclip;
  if (d1 > dclip) d1 = dclip;
  const int64_t e0 = exp2_neg_fixed((int64_t)((uint64_t)d0 * (uint64_t)log2e) >> fa, fa);
  const int64_t e1 = exp2_neg_fixed((int64_t)((uint64_t)d1 * (uint64_t)log2e) >> fa, fa);
  const int64_t z = e0 + e1;
  const int64_t sig = z == 0 ? 0 : (int64_t)(((uint64_t)e1 << fa) / (uint64_t)z);
  const i128 s = ((i128)x * sig) >> fa;
  if (s > (i128)INT64_MAX || s < (i128)INT64_MIN) atomicOr(status, IMIE_EOVF);
  const i128 gu = ((i128)(int64_t)s * u) >> fa;
  if (gu > (i128)INT64_MAX || gu < (i128)INT64_MIN) atomicOr(status, IMIE_EOVF);
  return (int64_t)gu;
}

__global__ void qk_silu_mul_kernel(const int64_t* __restrict__ g, const int64_t* __restrict__ u, int64_t n, int fa,
                                   int64_t log2e, int64_t dclip, int64_t* __restrict__ out, int* __restrict__ status,
                                   const int* __restrict__ run_gate = nullptr) {
  if (run_gate && *run_gate == 0) return;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    out[i] = qk_silu_elem(g[i], u[i], fa, log2e, dclip, status);
}

// The exact gate and up kernels and SiLU * up as the fallback of the fused gate/up stage, in one launch: a small
// grid that ends at once unless the prep flagged a wide activation row; then each workgroup takes (tile, item)
// pairs, computes the gate tile and the up tile and turns its own tile's elements into silu(gate) * up.
constexpr int kGatedWgs2 = 128;
__global__ __launch_bounds__(256) void qk_gateup_gated_kernel(const Item* __restrict__ ig, const Item* __restrict__ iu,
                                                              const int* __restrict__ xi, const int* __restrict__ yi,
                                                              const int64_t* __restrict__ X, int64_t K,
                                                              int64_t* __restrict__ gb, int64_t* __restrict__ ub,
                                                              int64_t ldy, int fw, int fa, int64_t log2e,
                                                              int64_t dclip, int* __restrict__ status,
                                                              const int* __restrict__ run_gate, int64_t ntx,
                                                              int64_t ne) {
  if (*run_gate == 0) return;
  for (int64_t t = blockIdx.x; t < ntx * ne; t += gridDim.x) {
    const int64_t bx = t % ntx, by = t / ntx;
    qk_group_tile(ig, xi, yi, X, K, gb, ldy, fw, status, bx, by);
    __syncthreads();
    qk_group_tile(iu, xi, yi, X, K, ub, ldy, fw, status, bx, by);
    __threadfence_block();
    __syncthreads();                                  // both tiles written (and the shared buffers free)
    const Item it = ig[by];
    const int64_t o0 = bx * kRows, no = it.out_f - o0 < kRows ? it.out_f - o0 : kRows;
    if (no > 0)
      for (int64_t e = threadIdx.x; e < (int64_t)it.count * no; e += blockDim.x) {
        const int64_t idx = (int64_t)yi[it.first + e / no] * ldy + o0 + e % no;
        gb[idx] = qk_silu_elem(gb[idx], ub[idx], fa, log2e, dclip, status);
      }
    __syncthreads();
  }
}

// out[t][o] = sum_j (dd[t*k + j][o] * gates[t*k + j]) >> fa (exact; cohere2.py:187 then astype int64)
// flags (optional): the fused MoE's two wide-row flags, cleared here, after their last reader, for the next call
__global__ void qk_combine_kernel(const int64_t* __restrict__ dd, int m, int k, int64_t d_model,
                                  const int64_t* __restrict__ gates, int fa, int64_t* __restrict__ out,
                                  int* __restrict__ status, int* __restrict__ flags = nullptr) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (flags && idx < 2) flags[idx] = 0;
  if (idx >= (int64_t)m * d_model) return;
  const int64_t t = idx / d_model, o = idx % d_model;
  i128 acc = 0;
  for (int j = 0; j < k; ++j) acc += ((i128)dd[(t * k + j) * d_model + o] * gates[t * k + j]) >> fa;
  if (acc > (i128)INT64_MAX || acc < (i128)INT64_MIN) atomicOr(status, IMIE_EOVF);
  out[idx] = (int64_t)acc;
}

// ---------------------------------------------------------------------------------------------------------
// int8-MFMA path (v_mfma_i32_16x16x32_i8, tokens in M, weight rows in N, one sub-block per K = 32 step):
//   prep  : the activation rows' balanced base-256 digit planes xd[l][row][K] (l < kQkLimbs), the sums of every
//           16 consecutive activations xs16[row][K / 16], and a flag when a row needs more than kQkLimbs limbs
//   Q4_K  : qdot_j = sum_l 256^l D_l with D_l = MFMA(digits_l(x), q) over sub-block j (32 positions, q in 0..15),
//           S1 = sum_j sc_j qdot_j, S2 = sum_j m_j xsum_j (int64: |x| <= 127 (256^5 - 1) / 255 keeps
//           |qdot| < 2^48, |S1| < 2^57, |S2| < 2^53), then acc += dq S1 - dmq S2 (int128) per 256-block
//   Q6_K  : the same with q6 - 32 as int8, sub-blocks of 16 (two MFMAs per 32 positions, each with the other
//           sub-block's K groups zeroed in A), no min term (|S1| < 2^59)
//   y = acc >> fw, refused (status bit 2) outside int64, as the VALU path.
// MFMA operands: A lane l = token l % 16, K group l / 16 (8 bytes); B lane l = weight row l % 16, K group l / 16;
// D lane l holds tokens 4 (l / 16) + r of row l % 16.
// ---------------------------------------------------------------------------------------------------------
constexpr int kQkLimbs = 5;

__global__ __launch_bounds__(256) void qk_prep_kernel(const int64_t* __restrict__ X, int64_t rows, int64_t K,
                                                      int8_t* __restrict__ xd, int64_t* __restrict__ xs16,
                                                      int* __restrict__ Lrow, int* __restrict__ wide) {
  __shared__ uint64_t s_mx[4];
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint64_t mx = 0;
  // eight consecutive activations per thread: their digits of each limb plane packed into one 64-bit store
  for (int64_t c0 = 8 * (int64_t)tid; c0 < K; c0 += 8 * 256) {
    if (c0 + 8 <= K) {
      int64_t v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = X[r * K + c0 + e];
      uint64_t pk[kQkLimbs];
#pragma unroll
      for (int l = 0; l < kQkLimbs; ++l) pk[l] = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint64_t a = imie_absu64(v[e]);
        mx = a > mx ? a : mx;
        int64_t x = v[e];
#pragma unroll
        for (int l = 0; l < kQkLimbs; ++l) {
          const int64_t dg = ((x + 128) & 255) - 128;
          x = (int64_t)((uint64_t)x - (uint64_t)dg) >> 8;
          pk[l] |= (uint64_t)(uint8_t)dg << (8 * e);
        }
      }
#pragma unroll
      for (int l = 0; l < kQkLimbs; ++l) *(uint64_t*)&xd[((int64_t)l * rows + r) * K + c0] = pk[l];
    } else {
      for (int64_t c = c0; c < K; ++c) {
        int64_t v = X[r * K + c];
        const uint64_t a = imie_absu64(v);
        mx = a > mx ? a : mx;
#pragma unroll
        for (int l = 0; l < kQkLimbs; ++l) {
          const int64_t dg = ((v + 128) & 255) - 128;
          v = (int64_t)((uint64_t)v - (uint64_t)dg) >> 8;
          xd[((int64_t)l * rows + r) * K + c] = (int8_t)dg;
        }
      }
    }
  }
  // sums of 16 consecutive activations (thread per group; callers whose kernels read no sums pass none)
  for (int64_t gq = tid; xs16 && gq < K / 16; gq += 256) {
    int64_t sm = 0;
#pragma unroll
    for (int e = 0; e < 16; ++e) sm = (int64_t)((uint64_t)sm + (uint64_t)X[r * K + 16 * gq + e]);
    xs16[r * (K / 16) + gq] = sm;
  }
  mx = imie_wave_max_u64_full(mx);
  if (lane == 0) s_mx[wave] = mx;
  __syncthreads();
  if (tid == 0) {
    uint64_t m = s_mx[0];
    for (int w = 1; w < 4; ++w) m = s_mx[w] > m ? s_mx[w] : m;
    const bool fits = m <= imie_balanced_cap(kQkLimbs);
    Lrow[r] = fits ? imie_limbs_needed(m) : kQkLimbs;
    if (!fits) atomicOr(wide, 1);
  }
}

__global__ void qk_flag_reset_kernel(int* f) { *f = 0; }
__global__ void qk_flags_reset_kernel(int* f, int n) { if ((int)threadIdx.x < n) f[threadIdx.x] = 0; }

__device__ inline v4i mfma32(int64_t a, int64_t b, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x32_i8((long)a, (long)b, c, 0, 0, 0);
}

template <int QT>
__global__ __launch_bounds__(256) void qk_mfma_kernel(const Item* __restrict__ items, const int* __restrict__ xi,
                                                      const int* __restrict__ yi, const int8_t* __restrict__ xd,
                                                      const int64_t* __restrict__ xs16, const int* __restrict__ Lrow,
                                                      int64_t rows, int64_t K, int64_t* __restrict__ Y, int64_t ldy,
                                                      int fw, int* __restrict__ status, const int* __restrict__ wide,
                                                      int dot4_max) {
  if (*wide) return;                                  // the VALU kernel takes this call
  const Item it = items[blockIdx.y];
  if (it.qtype != QT || it.count <= dot4_max) return; // small items: qk_dot4_kernel
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, kg = lane >> 4;
  const int64_t o = (int64_t)blockIdx.x * 64 + wave * 16 + n;
  if ((int64_t)blockIdx.x * 64 + wave * 16 >= it.out_f) return;
  const bool orow = o < it.out_f;
  constexpr int BS = QT == 0 ? 144 : 210;
  const uint8_t* wrow = it.w + (orow ? o : 0) * it.nb * BS;
  const int64_t K16 = K / 16;
  for (int c0 = 0; c0 < it.count; c0 += 16) {
    // A rows: token c0 + n of the item (zero past the item's count)
    const bool arow = c0 + n < it.count;
    const int64_t xr = arow ? xi[it.first + c0 + n] : 0;
    int La = arow ? Lrow[xr] : 1;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) { const int t = __shfl_xor(La, off, 64); La = t > La ? t : La; }
    const int L = La;                                 // limbs of this token tile (wave-uniform)
    // D rows: tokens c0 + 4 kg + q
    int64_t drow[4];
    bool dlive[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      dlive[q] = c0 + 4 * kg + q < it.count;
      drow[q] = dlive[q] ? xi[it.first + c0 + 4 * kg + q] : 0;
    }
    i128 acc[4] = {0, 0, 0, 0};
    for (int64_t b = 0; b < it.nb; ++b) {
      const uint8_t* blk = wrow + b * BS;
      int64_t S1[4] = {0, 0, 0, 0}, S2[4] = {0, 0, 0, 0};
      if (QT == 0) {
        const int64_t dq = fp16_fixed_fast(blk[0] | (blk[1] << 8), fw), dmq = fp16_fixed_fast(blk[2] | (blk[3] << 8), fw);
        const uint8_t* scb = blk + 4;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint2 qv = *(const uint2*)(blk + 16 + 32 * g + 8 * kg);
#pragma unroll
          for (int hi = 0; hi < 2; ++hi) {
            const int j = 2 * g + hi;
            const uint32_t b0 = hi ? (qv.x >> 4) & 0x0F0F0F0Fu : qv.x & 0x0F0F0F0Fu;
            const uint32_t b1 = hi ? (qv.y >> 4) & 0x0F0F0F0Fu : qv.y & 0x0F0F0F0Fu;
            const int64_t bq = (int64_t)(((uint64_t)b1 << 32) | b0);
            const int64_t pos = b * 256 + 32 * j + 8 * kg;
            int64_t qdot[4] = {0, 0, 0, 0};
#pragma unroll
            for (int l = 0; l < kQkLimbs; ++l) {
              if (l >= L) break;
              const int64_t av = arow ? *(const int64_t*)(xd + ((int64_t)l * rows + xr) * K + pos) : 0;
              const v4i d = mfma32(av, bq, v4i{0, 0, 0, 0});
#pragma unroll
              for (int q = 0; q < 4; ++q) qdot[q] += (int64_t)d[q] << (8 * l);
            }
            int sc, mn;
            if (j < 4) { sc = scb[j] & 63; mn = scb[j + 4] & 63; }
            else { sc = (scb[j + 4] & 0xF) | ((scb[j - 4] >> 6) << 4); mn = (scb[j + 4] >> 4) | ((scb[j] >> 6) << 4); }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int64_t xs = xs16[drow[q] * K16 + (b * 256 + 32 * j) / 16] + xs16[drow[q] * K16 + (b * 256 + 32 * j) / 16 + 1];
              S1[q] += (int64_t)sc * qdot[q];
              S2[q] += (int64_t)mn * xs;
            }
          }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[q] += (i128)dq * S1[q] - (i128)dmq * S2[q];
      } else {
        const uint8_t* ql = blk;
        const uint8_t* qh = blk + 128;
        const int8_t* scs = (const int8_t*)(blk + 192);
        const int64_t dq = fp16_fixed_fast(blk[208] | (blk[209] << 8), fw);
#pragma unroll
        for (int half = 0; half < 2; ++half)
#pragma unroll
          for (int qq = 0; qq < 4; ++qq) {
            // 32 positions 128 half + 32 qq + (0..31): lane K group kg takes 8 kg .. 8 kg + 7 (sub-block is = kg / 2)
            const uint2 lv = *(const uint2*)(ql + 64 * half + ((qq & 1) ? 32 : 0) + 8 * kg);
            const uint2 hv = *(const uint2*)(qh + 32 * half + 8 * kg);
            const int sl = qq >= 2 ? 4 : 0, sh = 2 * qq;
            uint32_t v0 = ((lv.x >> sl) & 0x0F0F0F0Fu) | (((hv.x >> sh) & 0x03030303u) << 4);
            uint32_t v1 = ((lv.y >> sl) & 0x0F0F0F0Fu) | (((hv.y >> sh) & 0x03030303u) << 4);
            v0 = ((v0 | 0x80808080u) - 0x20202020u) ^ 0x80808080u;   // bytewise q6 - 32 as int8
            v1 = ((v1 | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
            const int64_t bq = (int64_t)(((uint64_t)v1 << 32) | v0);
            const int64_t pos = b * 256 + 128 * half + 32 * qq + 8 * kg;
            int64_t qd0[4] = {0, 0, 0, 0}, qd1[4] = {0, 0, 0, 0};
#pragma unroll
            for (int l = 0; l < kQkLimbs; ++l) {
              if (l >= L) break;
              const int64_t av = arow ? *(const int64_t*)(xd + ((int64_t)l * rows + xr) * K + pos) : 0;
              const v4i d0 = mfma32(kg < 2 ? av : 0, bq, v4i{0, 0, 0, 0});
              const v4i d1 = mfma32(kg < 2 ? 0 : av, bq, v4i{0, 0, 0, 0});
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                qd0[q] += (int64_t)d0[q] << (8 * l);
                qd1[q] += (int64_t)d1[q] << (8 * l);
              }
            }
            const int s0 = scs[8 * half + 2 * qq], s1 = scs[8 * half + 2 * qq + 1];
#pragma unroll
            for (int q = 0; q < 4; ++q) S1[q] += (int64_t)s0 * qd0[q] + (int64_t)s1 * qd1[q];
          }
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[q] += (i128)dq * S1[q];
      }
    }
    if (orow) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (!dlive[q]) continue;
        const i128 y = acc[q] >> fw;
        if (y > (i128)INT64_MAX || y < (i128)INT64_MIN) atomicOr(status, IMIE_EOVF);
        Y[(int64_t)yi[it.first + c0 + 4 * kg + q] * ldy + o] = (int64_t)y;
      }
    }
  }
}

// v_dot4_i32_i8 path for items with few tokens (the MoE experts: ~4 tokens each), every token of the item once
// (no 16-row MFMA padding). Workgroup = (item, 64 weight rows); thread = (row, quarter q of each 256-block):
//   Q4_K: q covers qs bytes 32 q .. 32 q + 31, i.e. sub-blocks 2q (low nibbles) and 2q + 1 (high nibbles)
//   Q6_K: q = (half, pair of quarters qq): sub-blocks 8 half + 2 qq + is for qq in {2 (q & 1), 2 (q & 1) + 1}
// The weights are expanded to int8 once per block; per token and limb, 16 dot4s give the sub-block dot products.
// The 256-block's digits of up to 8 tokens are staged in LDS. Partial int128 sums of the 4 quarter-threads of a
// row are added by shuffles at the end (integer addition: order-free).
constexpr int kDotTok = 8;

__device__ inline i128 shfl_xor_i128(i128 v, int m) {
  const uint64_t lo = (uint64_t)v, hi = (uint64_t)((unsigned __int128)v >> 64);
  const uint64_t lo2 = (uint64_t)__shfl_xor((long long)lo, m, 64), hi2 = (uint64_t)__shfl_xor((long long)hi, m, 64);
  return (i128)(((unsigned __int128)hi2 << 64) | lo2);
}

template <int QT>
__global__ __launch_bounds__(256) void qk_dot4_kernel(const Item* __restrict__ items, const int* __restrict__ xi,
                                                      const int* __restrict__ yi, const int8_t* __restrict__ xd,
                                                      const int64_t* __restrict__ xs16, const int* __restrict__ Lrow,
                                                      int64_t rows, int64_t K, int64_t* __restrict__ Y, int64_t ldy,
                                                      int fw, int* __restrict__ status, const int* __restrict__ wide,
                                                      int maxcount) {
  __shared__ __align__(16) int8_t sx[kQkLimbs][kDotTok][256];
  __shared__ int64_t sxs[kDotTok][16];
  __shared__ int s_L;
  if (*wide) return;
  const Item it = items[blockIdx.y];
  if (it.qtype != QT || it.count > maxcount) return;
  const int tid = threadIdx.x, q = tid & 3;
  const int64_t o = (int64_t)blockIdx.x * 64 + (tid >> 2);
  if ((int64_t)blockIdx.x * 64 >= it.out_f) return;
  const bool orow = o < it.out_f;
  constexpr int BS = QT == 0 ? 144 : 210;
  const uint8_t* wrow = it.w + (orow ? o : 0) * it.nb * BS;
  const int64_t K16 = K / 16;
  for (int t0 = 0; t0 < it.count; t0 += kDotTok) {
    const int tn = min(kDotTok, it.count - t0);
    if (tid == 0) {
      int L = 1;
      for (int t = 0; t < tn; ++t) { const int lr = Lrow[xi[it.first + t0 + t]]; L = lr > L ? lr : L; }
      s_L = L;
    }
    __syncthreads();
    const int L = s_L;
    i128 acc[kDotTok];
#pragma unroll
    for (int t = 0; t < kDotTok; ++t) acc[t] = 0;
    for (int64_t b = 0; b < it.nb; ++b) {
      // stage the block's digits (L limbs x tn tokens x 256 bytes, 16 B per thread-step) and 16-sums
      for (int i = tid; i < L * tn * 16; i += 256) {
        const int l = i / (tn * 16), rem = i % (tn * 16), t = rem >> 4, c = rem & 15;
        const int64_t xr = xi[it.first + t0 + t];
        *(uint4*)&sx[l][t][16 * c] = *(const uint4*)(xd + ((int64_t)l * rows + xr) * K + b * 256 + 16 * c);
      }
      if (tid < tn * 16) {
        const int t = tid >> 4, c = tid & 15;
        sxs[t][c] = xs16[(int64_t)xi[it.first + t0 + t] * K16 + b * 16 + c];
      }
      __syncthreads();
      const uint8_t* blk = wrow + b * BS;
      if (QT == 0) {
        const int64_t dq = fp16_fixed_fast(blk[0] | (blk[1] << 8), fw), dmq = fp16_fixed_fast(blk[2] | (blk[3] << 8), fw);
        const uint8_t* scb = blk + 4;
        const uint4 qa = *(const uint4*)(blk + 16 + 32 * q), qb = *(const uint4*)(blk + 32 + 32 * q);
        const uint32_t qd[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        int wl[8], wh[8];
#pragma unroll
        for (int d = 0; d < 8; ++d) { wl[d] = (int)(qd[d] & 0x0F0F0F0Fu); wh[d] = (int)((qd[d] >> 4) & 0x0F0F0F0Fu); }
        int sc[2], mn[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int j = 2 * q + h;
          if (j < 4) { sc[h] = scb[j] & 63; mn[h] = scb[j + 4] & 63; }
          else { sc[h] = (scb[j + 4] & 0xF) | ((scb[j - 4] >> 6) << 4); mn[h] = (scb[j + 4] >> 4) | ((scb[j] >> 6) << 4); }
        }
#pragma unroll
        for (int t = 0; t < kDotTok; ++t) {
          if (t >= tn) break;
          int64_t qlo = 0, qhi = 0;
          for (int l = 0; l < L; ++l) {
            const int* xl = (const int*)&sx[l][t][64 * q];
            const int* xh = (const int*)&sx[l][t][64 * q + 32];
            int al = 0, ah = 0;
#pragma unroll
            for (int d = 0; d < 8; ++d) {
              al = __builtin_amdgcn_sdot4(xl[d], wl[d], al, false);
              ah = __builtin_amdgcn_sdot4(xh[d], wh[d], ah, false);
            }
            qlo += (int64_t)al << (8 * l);
            qhi += (int64_t)ah << (8 * l);
          }
          const int64_t S1 = (int64_t)sc[0] * qlo + (int64_t)sc[1] * qhi;
          const int64_t S2 = (int64_t)mn[0] * (sxs[t][4 * q] + sxs[t][4 * q + 1]) +
                             (int64_t)mn[1] * (sxs[t][4 * q + 2] + sxs[t][4 * q + 3]);
          acc[t] += (i128)dq * S1 - (i128)dmq * S2;
        }
      } else {
        const int half = q >> 1, qq0 = 2 * (q & 1);
        const uint8_t* ql = blk + 64 * half;
        const uint8_t* qh = blk + 128 + 32 * half;
        const int8_t* scs = (const int8_t*)(blk + 192);
        const int64_t dq = fp16_fixed_fast(blk[208] | (blk[209] << 8), fw);
        const uint4 l0 = *(const uint4*)ql, l1 = *(const uint4*)(ql + 16), l2 = *(const uint4*)(ql + 32),
                    l3 = *(const uint4*)(ql + 48);
        const uint4 h0 = *(const uint4*)qh, h1 = *(const uint4*)(qh + 16);
        const uint32_t lq[16] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w, l2.x, l2.y, l2.z, l2.w, l3.x, l3.y, l3.z, l3.w};
        const uint32_t hq[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
        const int sl = (q & 1) ? 4 : 0;
        int w[2][8];                                  // [qq - qq0][dword of the 32 positions]
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int qq = qq0 + u;
#pragma unroll
          for (int d = 0; d < 8; ++d) {
            uint32_t v = ((lq[((qq & 1) ? 8 : 0) + d] >> sl) & 0x0F0F0F0Fu) | (((hq[d] >> (2 * qq)) & 0x03030303u) << 4);
            v = ((v | 0x80808080u) - 0x20202020u) ^ 0x80808080u;   // bytewise q6 - 32 as int8
            w[u][d] = (int)v;
          }
        }
        int sc[2][2];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int is = 0; is < 2; ++is) sc[u][is] = scs[8 * half + 2 * (qq0 + u) + is];
#pragma unroll
        for (int t = 0; t < kDotTok; ++t) {
          if (t >= tn) break;
          int64_t qs4[2][2] = {{0, 0}, {0, 0}};
          for (int l = 0; l < L; ++l) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              const int* xp = (const int*)&sx[l][t][128 * half + 32 * (qq0 + u)];
              int a0 = 0, a1 = 0;
#pragma unroll
              for (int d = 0; d < 4; ++d) {
                a0 = __builtin_amdgcn_sdot4(xp[d], w[u][d], a0, false);
                a1 = __builtin_amdgcn_sdot4(xp[4 + d], w[u][4 + d], a1, false);
              }
              qs4[u][0] += (int64_t)a0 << (8 * l);
              qs4[u][1] += (int64_t)a1 << (8 * l);
            }
          }
          const int64_t S1 = (int64_t)sc[0][0] * qs4[0][0] + (int64_t)sc[0][1] * qs4[0][1] +
                             (int64_t)sc[1][0] * qs4[1][0] + (int64_t)sc[1][1] * qs4[1][1];
          acc[t] += (i128)dq * S1;
        }
      }
      __syncthreads();
    }
#pragma unroll
    for (int t = 0; t < kDotTok; ++t) {
      if (t >= tn) break;
      i128 v = acc[t];
      v += shfl_xor_i128(v, 1);
      v += shfl_xor_i128(v, 2);
      if (q == 0 && orow) {
        const i128 y = v >> fw;
        if (y > (i128)INT64_MAX || y < (i128)INT64_MIN) atomicOr(status, IMIE_EOVF);
        Y[(int64_t)yi[it.first + t0 + t] * ldy + o] = (int64_t)y;
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------------------------------
// Fused MoE expert kernels (the batched MoE of cohere2.py:168-188 with Q4_K gate/up and Q6_K down, the
// north-mini-code layout): one item per expert = its gate/up/down weights and the (token, pair) list routed to it.
//   moe_gateup : g = gate . h, u = up . h (the same activation operands feed both), then gu = (silu(g) * u) >> fa
//                in the epilogue (the exact arithmetic of qk_silu_mul_kernel), written per pair
//   moe_down   : d = down . gu per pair
// int8 MFMA v_mfma_i32_16x16x32_i8 with the MFMA M rows = (token t, digit limb l) = 4 t + l: four tokens of up to
// four balanced base-256 limbs per MFMA (a second MFMA takes limbs 4..7), weight rows in N, one sub-block (Q4_K:
// 32 positions; Q6_K: 16, the other half of the K groups zeroed in A) per K = 32 step. D lane (t, n) then holds
// the limb partial sums of token t for weight row n, recombined in place (no cross-lane traffic) into the
// sub-block dot q.x per limb; S1 = sum_j sc_j q.x_j and S2 = sum_j m_j xsum_j are summed per limb in int32 and
// recombined once per block into int64 (|x| < 127 (256^5-1)/255: |S1| < 2^57, |S2| < 2^53), and each 256-block
// adds dq S1 - dmq S2 into a 128-bit (hi, lo) accumulator with one 64 x 64 -> 128 multiply per term. MFMA sums are
// exact: |D| <= 32 * 128 * 32 < 2^31.
// gate/up: workgroup = (64 weight rows, item), wave = 16 rows. Up to eight tokens share one walk over the weights:
// with at most four limbs, two token groups of four are staged (32 digit rows, K in two halves, one barrier each)
// and every block's decode (scales, mins, nibbles) feeds both groups' MFMAs; otherwise one group of four at a time
// stages its rows over the whole K (limbs 0..3, then 4..7 in a second pass when there are more than four). The
// block loop has no barrier; the next block's weights are in flight while a block computes.
// down (K of a few blocks): workgroup = (64 weight rows, item); the block loop is software-pipelined, the next
// block's digits going to the other half of an LDS double buffer while a block computes. The buffer's second
// 16-row group holds tokens 4..7 (up to eight tokens of at most four limbs share each block's unpacked weights)
// or limbs 4..7 of up to four tokens.
// ---------------------------------------------------------------------------------------------------------
constexpr int kMoeTok = 4;         // tokens per MFMA row group (4 tokens x 4 limbs = 16 rows)
// LDS row stride of the staged digits: K + 16 bytes (K a multiple of 256). A lane of row r (of the 16 (token, limb)
// rows) and K group kg reads 8 bytes at r (K + 16) + 8 kg + 32 j, i.e. 8-byte slot 2 r + kg (mod 32): the 32 lanes
// of a half-wave hit 32 distinct slots (with a K-byte stride all 16 rows of a K group shared one slot: 16-way bank
// conflicts).
__host__ __device__ inline int64_t moe_kp(int64_t K) { return K + 16; }
// gate/up staging: 16 rows x (K + 16) (one token group) or 32 rows x (K / 2 + 16) (two groups, K in halves)
__host__ __device__ inline size_t moe_lds_bytes(int64_t K) { return (size_t)16 * (size_t)K + 512; }

struct MoeItem {
  const uint8_t* wg;        // gate (Q4_K), up (Q4_K), down (Q6_K) of the expert
  const uint8_t* wu;
  const uint8_t* wd;
  int first, count;         // into the pair arrays: ptok (activation row of h), ppair (gu / d row)
};

struct Acc128 {             // two's-complement 128-bit accumulator
  uint64_t lo;
  int64_t hi;
};

__device__ inline void acc_madd(Acc128& a, int64_t x, int64_t y) {
  const uint64_t pl = (uint64_t)x * (uint64_t)y;
  const int64_t ph = __mul64hi(x, y);
  a.lo += pl;
  a.hi += ph + (a.lo < pl ? 1 : 0);
}

// floor(acc / 2^fw) and whether it fits int64 (0 <= fw < 64)
__device__ inline int64_t acc_shift(Acc128 a, int fw, bool* fits) {
  const i128 v = (i128)(((unsigned __int128)(uint64_t)a.hi << 64) | a.lo);
  const i128 y = v >> fw;
  *fits = y <= (i128)INT64_MAX && y >= (i128)INT64_MIN;
  return (int64_t)y;
}

// exact nmc SiLU * up of one element (qk_silu_mul_kernel): false when an intermediate leaves int64
__device__ inline int64_t nmc_silu_mul(int64_t x, int64_t u, int fa, int64_t log2e, int64_t dclip, bool* ok) {
  const int64_t m = x > 0 ? x : 0;
  int64_t d0 = m, d1 = (int64_t)((uint64_t)m - (uint64_t)x);
  if (d0 > dclip) d0 = dclip;
  if (d1 > dclip) d1 = dclip;
  const int64_t e0 = exp2_neg_fixed((int64_t)((uint64_t)d0 * (uint64_t)log2e) >> fa, fa);
  const int64_t e1 = exp2_neg_fixed((int64_t)((uint64_t)d1 * (uint64_t)log2e) >> fa, fa);
  const int64_t z = e0 + e1;
  const int64_t sig = z == 0 ? 0 : (int64_t)(((uint64_t)e1 << fa) / (uint64_t)z);
  const i128 s = ((i128)x * sig) >> fa;
  bool good = s <= (i128)INT64_MAX && s >= (i128)INT64_MIN;
  const i128 gu = ((i128)(int64_t)s * u) >> fa;
  good = good && gu <= (i128)INT64_MAX && gu >= (i128)INT64_MIN;
  *ok = good;
  return (int64_t)gu;
}

// Per-block staging (the down kernel, whose K of a few blocks is walked with the next block's digits fetched while a
// block computes): up to 8 limbs x kMoeTok tokens x 256 bytes per block, rows of 272 bytes (moe_kp(256)), double
// buffered.
constexpr int kMoeLimbs = 8;
constexpr int kMoeRow = 272;
constexpr int kMoeBuf = kMoeLimbs * kMoeTok * kMoeRow;

// Staging of one block's digits (L limbs x kMoeTok tokens x 256 bytes) as a register fetch issued before the
// current block's compute and an LDS store after it. At most 8 x 4 x 16 = 512 uint4: two per thread. The thread's
// two (source row, LDS slot) pairs are fixed for a token group (MoePlan); a block only adds its offset.
struct MoePlan {
  const int8_t* src[2];     // digits of (limb, token) row at 16-byte chunk c, block 0
  int dst[2];               // LDS byte offset of [l][t][16 c]
  bool on[2];
};
__device__ inline MoePlan moe_plan(const int* rowsel, int tn, int L, const int8_t* __restrict__ xd, int64_t rows,
                                   int64_t K, int tid) {
  MoePlan p;
  const int n = L * tn * 16, nt = (int)blockDim.x;    // 256 or 512 threads: two or one chunks each
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int i = tid + nt * k;
    p.on[k] = i < n;
    const int l = p.on[k] ? i / (tn * 16) : 0, rem = i - l * (tn * 16), t = p.on[k] ? rem >> 4 : 0, c = rem & 15;
    p.src[k] = xd + ((int64_t)l * rows + rowsel[t]) * K + 16 * c;
    // row 16 gi + 4 (l mod 4) + (t mod 4): the second 16-row group holds limbs 4..7 (tn <= 4) or tokens 4..7 (L <= 4)
    const int gi = (l >= 4 || t >= kMoeTok) ? 1 : 0;
    p.dst[k] = (16 * gi + 4 * (l & 3) + (t & 3)) * kMoeRow + 16 * c;
  }
  return p;
}
struct MoeStage {
  uint4 v[2];
};
__device__ inline MoeStage moe_fetch(const MoePlan& p, int64_t b) {
  MoeStage r;
#pragma unroll
  for (int k = 0; k < 2; ++k) r.v[k] = p.on[k] ? *(const uint4*)(p.src[k] + b * 256) : uint4{0, 0, 0, 0};
  return r;
}
__device__ inline void moe_store(const MoeStage& r, const MoePlan& p, int8_t* buf) {
#pragma unroll
  for (int k = 0; k < 2; ++k)
    if (p.on[k]) *(uint4*)(buf + p.dst[k]) = r.v[k];
}

// both staging buffers to zero (threads tid of nt; the caller synchronizes before and after)
__device__ inline void moe_clear(int8_t* sx, int tid, int nt) {
  for (int i = tid; i < 2 * kMoeBuf / 16; i += nt) ((uint4*)sx)[i] = uint4{0, 0, 0, 0};
}

// Stage limbs 4 p .. 4 p + 3 of up to 8 tokens' activation rows, K positions kbeg .. kbeg + klen, into LDS row
// r = 16 grp + 4 l + t (token 4 grp + t, limb 4 p + l) at stride kp: 16 ngrp rows x klen / 16 chunks of 16 bytes, the
// loads of four chunks per thread issued before their stores. Rows of absent tokens (>= tn) or limbs (>= L) are
// written as zeros, so the MFMA A operands need no selects. The caller synchronizes before (buffer free) and after
// (rows visible).
__device__ inline void moe_stage(int8_t* sx, const int (&prow)[2 * kMoeTok], int tn, int L, int p, int ngrp,
                                 int64_t kbeg, int64_t klen, int64_t kp, const int8_t* __restrict__ xd, int64_t rows,
                                 int64_t K, int tid, int nt) {
  const int cpr = (int)(klen >> 4), total = 16 * ngrp * cpr;
  for (int i0 = tid; i0 < total; i0 += 4 * nt) {
    uint4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + u * nt;
      const int r = i / cpr, c = i - r * cpr, l = (r >> 2) & 3, tok = 4 * (r >> 4) + (r & 3);
      const bool on = i < total && tok < tn && 4 * p + l < L;
      int pr = prow[0];
#pragma unroll
      for (int q = 1; q < 2 * kMoeTok; ++q) pr = tok == q ? prow[q] : pr;
      v[u] = on ? *(const uint4*)(xd + ((int64_t)(4 * p + l) * rows + pr) * K + kbeg + 16 * c) : uint4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + u * nt;
      if (i < total) {
        const int r = i / cpr, c = i - r * cpr;
        *(uint4*)(sx + r * kp + 16 * c) = v[u];
      }
    }
  }
}

// The lane's A operand source: limb l (of the staged pass) of token t (row m = 4 t + l of the MFMA), K group kg.
struct MoeA {
  int off;                  // byte offset of [l][t][8 kg]
};
__device__ inline MoeA moe_a_lane(int lane, int64_t kp) {
  const int m = lane & 15, kg = lane >> 4, t = m >> 2, l = m & 3;
  MoeA r;
  r.off = (l * kMoeTok + t) * (int)kp + 8 * kg;
  return r;
}
// A operand at K position p0 (buf points at the block's first position)
__device__ inline int64_t moe_a(const int8_t* buf, const MoeA& a, int p0) {
  return *(const int64_t*)(buf + a.off + p0);
}

// sum_r T[r] << 8 (4 lg + r): a token's value from its per-limb partial sums (int32 per limb)
__device__ inline int64_t limb_sum(v4i d, int lg) {
  const int64_t v = (int64_t)d[0] + ((int64_t)d[1] << 8) + ((int64_t)d[2] << 16) + ((int64_t)d[3] << 24);
  return lg ? (int64_t)((uint64_t)v << 32) : v;
}

// Q4_K weights of one block for B lanes (row n, K group kg): the 16-byte header (d, dmin, 12 scale bytes) and the
// qs bytes 32 g + 8 kg .. + 7 for g = 0..3 (sub-blocks 2 g (low nibbles), 2 g + 1 (high nibbles))
struct Q4Lane {
  uint4 h;
  uint2 q[4];
};
// Loads of weight bytes through global-address-space pointers of native vector types. The item pointers come from
// memory, so plain loads through them are flat loads, which count against the LDS counter as well: every LDS wait
// in the block compute would then also wait for the next block's weights in flight.
typedef unsigned gv4u __attribute__((ext_vector_type(4)));
typedef unsigned gv2u __attribute__((ext_vector_type(2)));
template <typename T>
__device__ inline T gload(const uint8_t* p);
template <>
__device__ inline uint4 gload<uint4>(const uint8_t* p) {
  const gv4u v = *(__attribute__((address_space(1))) const gv4u*)p;
  return uint4{v.x, v.y, v.z, v.w};
}
template <>
__device__ inline uint2 gload<uint2>(const uint8_t* p) {
  const gv2u v = *(__attribute__((address_space(1))) const gv2u*)p;
  return uint2{v.x, v.y};
}
template <>
__device__ inline uint8_t gload<uint8_t>(const uint8_t* p) {
  return *(__attribute__((address_space(1))) const uint8_t*)p;
}
__device__ inline Q4Lane q4_lane_load(const uint8_t* blk, int kg) {
  Q4Lane r;
  r.h = gload<uint4>(blk);
#pragma unroll
  for (int g = 0; g < 4; ++g) r.q[g] = gload<uint2>(blk + 16 + 32 * g + 8 * kg);
  return r;
}

// One Q4_K block: acc += dq S1 - dmq S2 for the lane's (token, row). Per limb r, S1's part sum_j sc_j D_j[r] stays
// in int32 (|D| <= 32 * 128 * 15, 8 sub-blocks x 63: < 2^25) and S2's part sum_j m_j (sum of the sub-block's
// digits) is an MFMA accumulation with B = m_j in every byte (|.| <= 8 * 63 * 32 * 128 < 2^21).
template <int NG>
__device__ inline void q4_block_mfma(const Q4Lane& w, const int8_t* buf, int gstride, const MoeA& a, int lg, int fw,
                                     Acc128 (&acc)[NG], bool two) {
  const uint32_t hb = w.h.x;
  const int64_t dq = fp16_fixed_fast(hb & 0xFFFF, fw), dmq = fp16_fixed_fast(hb >> 16, fw);
  const uint32_t scw[3] = {w.h.y, w.h.z, w.h.w};
  auto scb = [&](int i) { return (int)((scw[i >> 2] >> (8 * (i & 3))) & 0xFF); };
  int sc[8], mn[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (j < 4) { sc[j] = scb(j) & 63; mn[j] = scb(j + 4) & 63; }
    else { sc[j] = (scb(j + 4) & 0xF) | ((scb(j - 4) >> 6) << 4); mn[j] = (scb(j + 4) >> 4) | ((scb(j) >> 6) << 4); }
  }
  // sub-block j's weights: the low / high nibbles of q bytes 32 (j / 2) + 8 kg ..; the min term's B operand has
  // m_j in every byte
  auto bq = [&](int j) {
    const uint2 qv = w.q[j >> 1];
    const uint32_t b0 = (j & 1) ? (qv.x >> 4) & 0x0F0F0F0Fu : qv.x & 0x0F0F0F0Fu;
    const uint32_t b1 = (j & 1) ? (qv.y >> 4) & 0x0F0F0F0Fu : qv.y & 0x0F0F0F0Fu;
    return (int64_t)(((uint64_t)b1 << 32) | b0);
  };
  auto bm = [&](int j) {
    const uint32_t mb = __builtin_amdgcn_perm(0u, (uint32_t)mn[j], 0u);   // byte 0 in all four bytes
    return (int64_t)(((uint64_t)mb << 32) | mb);
  };
  // the weight decode above is shared by the NG token groups (16 MFMA rows each, gstride bytes apart in LDS)
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) {
    if (gi > 0 && !two) break;                        // wave-uniform
    const int8_t* gb = buf + gi * gstride;
    v4i M = {0, 0, 0, 0}, T = {0, 0, 0, 0};
    // two halves of four sub-blocks: four independent MFMAs issued back to back, their results consumed after
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      v4i d[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int j = 4 * hh + jj;
        const int64_t av = moe_a(gb, a, 32 * j);
        d[jj] = mfma32(av, bq(j), v4i{0, 0, 0, 0});
        M = mfma32(av, bm(j), M);
      }
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int r = 0; r < 4; ++r) T[r] += __mul24(sc[4 * hh + jj], d[jj][r]);   // 24-bit: |sc| < 2^6, |D| < 2^17
    }
    acc_madd(acc[gi], dq, limb_sum(T, lg));
    acc_madd(acc[gi], -dmq, limb_sum(M, lg));
  }
}

// The token groups' activation rows (sel[first + t], absent tokens repeat the last one) and their limb counts
// (two load rounds, all issued at once); returns the largest
__device__ inline int moe_group_rows(const int* __restrict__ sel, const int* __restrict__ Lrow, int first, int tn,
                                     int (&prow)[2 * kMoeTok], int (&lr)[2 * kMoeTok]) {
#pragma unroll
  for (int i = 0; i < 2 * kMoeTok; ++i) prow[i] = sel[first + (i < tn ? i : tn - 1)];
  int L = 1;
#pragma unroll
  for (int i = 0; i < 2 * kMoeTok; ++i) { lr[i] = Lrow[prow[i]]; L = lr[i] > L ? lr[i] : L; }
  return L;
}

__global__ __launch_bounds__(256, 2) void moe_gateup_kernel(const MoeItem* __restrict__ items, const int* __restrict__ ptok,
                                                         const int* __restrict__ ppair, const int8_t* __restrict__ xd,
                                                         const int* __restrict__ Lrow, int64_t rows, int64_t K,
                                                         int64_t e_ffn, int fw, int fa, int64_t log2e, int64_t dclip,
                                                         int64_t* __restrict__ gu, int* __restrict__ status,
                                                         const int* __restrict__ wide) {
  extern __shared__ __align__(16) int8_t sx[];       // moe_lds_bytes(K)
  if (*wide) return;                                  // the VALU fallback takes this call
  const MoeItem it = items[blockIdx.y];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if ((int64_t)blockIdx.x * 64 >= e_ffn) return;
  const int n = lane & 15, kg = lane >> 4, t = lane >> 4;
  const int nb = (int)(K / 256);
  const int64_t o = (int64_t)blockIdx.x * 64 + wave * 16 + n;
  const bool orow = o < e_ffn;
  const uint8_t* grow = it.wg + (orow ? o : 0) * nb * 144;
  const uint8_t* urow = it.wu + (orow ? o : 0) * nb * 144;
  auto emit = [&](const Acc128& ag, const Acc128& au, int tok) {
    bool f1, f2, f3;
    const int64_t gy = acc_shift(ag, fw, &f1), uy = acc_shift(au, fw, &f2);
    const int64_t v = nmc_silu_mul(gy, uy, fa, log2e, dclip, &f3);
    if (!(f1 && f2 && f3)) atomicOr(status, IMIE_EOVF);
    gu[(int64_t)ppair[it.first + tok] * e_ffn + o] = v;
  };
  for (int t0 = 0; t0 < it.count; t0 += 2 * kMoeTok) {
    const int tn8 = min(2 * kMoeTok, it.count - t0);
    int prow[2 * kMoeTok], lr[2 * kMoeTok];
    const int L8 = moe_group_rows(ptok, Lrow, it.first + t0, tn8, prow, lr);
    // one weight slot per projection, the first requested before the staging: block b + 1 is requested as soon as
    // block b has consumed the slot (the other waves of the SIMD cover the latency)
    Q4Lane gw = q4_lane_load(grow, kg), uw = q4_lane_load(urow, kg);
    if (tn8 > kMoeTok && L8 <= 4 && (nb & 1) == 0) {
      // two token groups of four in one walk over the weights (the block decode shared): K staged in halves of
      // 32 rows x (K / 2 + 16)
      const int64_t kp = K / 2 + 16;
      const MoeA al = moe_a_lane(lane, kp);
      Acc128 ag[2] = {{0, 0}, {0, 0}}, au[2] = {{0, 0}, {0, 0}};
      for (int h = 0; h < 2; ++h) {
        __syncthreads();                              // the buffer is free
        moe_stage(sx, prow, tn8, L8, 0, 2, h * (K / 2), K / 2, kp, xd, rows, K, tid, blockDim.x);
        __syncthreads();
        for (int bb = 0; bb < nb / 2; ++bb) {
          const int b = h * (nb / 2) + bb, bn = b + 1 < nb ? b + 1 : b;
          const int8_t* buf = sx + 256 * bb;
          q4_block_mfma<2>(gw, buf, (int)(16 * kp), al, 0, fw, ag, true);
          gw = q4_lane_load(grow + bn * 144, kg);
          q4_block_mfma<2>(uw, buf, (int)(16 * kp), al, 0, fw, au, true);
          uw = q4_lane_load(urow + bn * 144, kg);
        }
      }
      if (orow) {
        emit(ag[0], au[0], t0 + t);
        if (kMoeTok + t < tn8) emit(ag[1], au[1], t0 + kMoeTok + t);
      }
      continue;
    }
    // one token group of four at a time; more than four limbs take two passes per group (limbs 0..3, 4..7)
    const int64_t kp = K + 16;
    const MoeA al = moe_a_lane(lane, kp);
    for (int s0 = 0; s0 < tn8; s0 += kMoeTok) {
      const int tn = min(kMoeTok, tn8 - s0);
      int pr4[2 * kMoeTok];
      int L = 1;
#pragma unroll
      for (int i = 0; i < 2 * kMoeTok; ++i) {
        const int q = s0 + (i < tn ? i : tn - 1);
        int v = prow[0], lv = lr[0];
#pragma unroll
        for (int z = 1; z < 2 * kMoeTok; ++z) { v = q == z ? prow[z] : v; lv = q == z ? lr[z] : lv; }
        pr4[i] = v;
        L = i < tn && lv > L ? lv : L;
      }
      const int np = L > 4 ? 2 : 1;
      Acc128 ag[1] = {{0, 0}}, au[1] = {{0, 0}};
      for (int p = 0; p < np; ++p) {
        __syncthreads();                              // the buffer is free
        moe_stage(sx, pr4, tn, L, p, 1, 0, K, kp, xd, rows, K, tid, blockDim.x);
        __syncthreads();
        for (int b = 0; b < nb; ++b) {
          // the next block of this walk: this group's next pass or the following group start again at block 0
          const int bn = b + 1 < nb ? b + 1 : 0;
          const int8_t* buf = sx + 256 * b;
          q4_block_mfma<1>(gw, buf, 0, al, p, fw, ag, false);
          gw = q4_lane_load(grow + bn * 144, kg);
          q4_block_mfma<1>(uw, buf, 0, al, p, fw, au, false);
          uw = q4_lane_load(urow + bn * 144, kg);
        }
      }
      if (orow && t < tn) emit(ag[0], au[0], t0 + s0 + t);
    }
  }
}

// Q6_K weights of one block for B lanes (row n, K group kg): per K step (half, qq) the ql bytes
// 64 half + 32 (qq & 1) + 8 kg .. + 7 and the qh bytes 32 half + 8 kg .. + 7 (bits 2 qq, 2 qq + 1); the 16
// int8 scales and d
struct Q6Lane {
  uint2 l[2][2];            // [half][qq & 1]
  uint2 h[2];               // [half]
  uint4 sc;
  uint32_t d;
};
__device__ inline Q6Lane q6_lane_load(const uint8_t* blk, int kg) {
  Q6Lane r;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
#pragma unroll
    for (int o = 0; o < 2; ++o) r.l[half][o] = gload<uint2>(blk + 64 * half + 32 * o + 8 * kg);
    r.h[half] = gload<uint2>(blk + 128 + 32 * half + 8 * kg);
  }
  r.sc = gload<uint4>(blk + 192);
  r.d = (uint32_t)gload<uint8_t>(blk + 208) | ((uint32_t)gload<uint8_t>(blk + 209) << 8);
  return r;
}

// One Q6_K block: acc += dq S1; per limb r, sum_j sc_j D_j[r] in int32 (|D| <= 32 * 128 * 32 = 2^17, 16
// sub-blocks x 128: < 2^28)
// The second group (gstride bytes further in LDS) is either limbs 4..7 of the same tokens (added into acc0 with
// lg1 = 1) or limbs 0..3 of four more tokens (acc1, lg1 = 0); the block's unpacked weights and scales serve both.
__device__ inline void q6_block_mfma(const Q6Lane& w, const int8_t* buf, int gstride, const MoeA& a, int kg, int fw,
                                     Acc128& acc0, Acc128& acc1, int lg1, bool two) {
  const int64_t dq = fp16_fixed_fast(w.d, fw);
  const uint32_t scw[4] = {w.sc.x, w.sc.y, w.sc.z, w.sc.w};
  auto scs = [&](int i) { return (int)(int8_t)((scw[i >> 2] >> (8 * (i & 3))) & 0xFF); };
  const bool klo = kg < 2;
  int64_t bq[2][4];
#pragma unroll
  for (int half = 0; half < 2; ++half)
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const uint2 lv = w.l[half][qq & 1], hv = w.h[half];
      const int sl = qq >= 2 ? 4 : 0, sh = 2 * qq;
      uint32_t v0 = ((lv.x >> sl) & 0x0F0F0F0Fu) | (((hv.x >> sh) & 0x03030303u) << 4);
      uint32_t v1 = ((lv.y >> sl) & 0x0F0F0F0Fu) | (((hv.y >> sh) & 0x03030303u) << 4);
      v0 = ((v0 | 0x80808080u) - 0x20202020u) ^ 0x80808080u;   // bytewise q6 - 32 as int8
      v1 = ((v1 | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
      bq[half][qq] = (int64_t)(((uint64_t)v1 << 32) | v0);
    }
#pragma unroll
  for (int gi = 0; gi < 2; ++gi) {
    if (gi == 1 && !two) break;                       // wave-uniform
    const int8_t* gb = buf + gi * gstride;
    v4i T = {0, 0, 0, 0};
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      // the 8 MFMAs of a half are independent: issued back to back, consumed afterwards
      v4i d[4][2];
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        // the K step spans sub-blocks 8 half + 2 qq (K groups 0, 1) and + 1 (K groups 2, 3)
        const int64_t av = moe_a(gb, a, 128 * half + 32 * qq);
        d[qq][0] = mfma32(klo ? av : 0, bq[half][qq], v4i{0, 0, 0, 0});
        d[qq][1] = mfma32(klo ? 0 : av, bq[half][qq], v4i{0, 0, 0, 0});
      }
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const int s0 = scs(8 * half + 2 * qq), s1 = scs(8 * half + 2 * qq + 1);
#pragma unroll
        for (int r = 0; r < 4; ++r) T[r] += __mul24(s0, d[qq][0][r]) + __mul24(s1, d[qq][1][r]);   // |s| < 2^8, |D| < 2^18
      }
    }
    if (gi == 0) acc_madd(acc0, dq, limb_sum(T, 0));
    else acc_madd(acc1, dq, limb_sum(T, lg1));
  }
}

__global__ __launch_bounds__(256) void moe_down_kernel(const MoeItem* __restrict__ items, const int* __restrict__ ppair,
                                                       const int8_t* __restrict__ xd, const int64_t* __restrict__ xs16,
                                                       const int* __restrict__ Lrow, int64_t rows, int64_t K,
                                                       int64_t d_model, int fw, int64_t* __restrict__ dout,
                                                       int* __restrict__ status, const int* __restrict__ wide) {
  __shared__ __align__(16) int8_t sx[2][kMoeBuf];
  __shared__ int s_rows[2 * kMoeTok];
  if (*wide) return;
  const MoeItem it = items[blockIdx.y];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if ((int64_t)blockIdx.x * 64 >= d_model) return;
  const int n = lane & 15, kg = lane >> 4, t = lane >> 4;
  const int64_t o = (int64_t)blockIdx.x * 64 + wave * 16 + n;
  const bool orow = o < d_model;
  const int64_t nb = K / 256;
  const uint8_t* drow = it.wd + (orow ? o : 0) * nb * 210;
  for (int t0 = 0; t0 < it.count;) {
    // up to eight tokens with at most four limbs (the second 16-row group holds tokens 4..7), else up to four
    // tokens (the second group holds limbs 4..7 when there are more than four)
    const int tn8 = min(2 * kMoeTok, it.count - t0);
    int L4 = 1, L8 = 1;
    for (int i = 0; i < tn8; ++i) {
      const int lr = Lrow[ppair[it.first + t0 + i]];
      L8 = lr > L8 ? lr : L8;
      if (i < kMoeTok) L4 = L8;
    }
    const bool tok2 = tn8 > kMoeTok && L8 <= 4;
    const int tn = tok2 ? tn8 : min(kMoeTok, tn8), L = tok2 ? L8 : L4;
    __syncthreads();                                  // the previous token group is done with the buffers
    moe_clear(&sx[0][0], tid, blockDim.x);
    if (tid < tn) s_rows[tid] = ppair[it.first + t0 + tid];
    __syncthreads();
    const MoeA al = moe_a_lane(lane, kMoeRow);
    Q6Lane w0 = q6_lane_load(drow, kg), w1 = w0;
    if (nb > 1) w1 = q6_lane_load(drow + 210, kg);
    const MoePlan pl = moe_plan(s_rows, tn, L, xd, rows, K, tid);
    moe_store(moe_fetch(pl, 0), pl, &sx[0][0]);
    __syncthreads();
    Acc128 ad{0, 0}, ad1{0, 0};
    Acc128& a2 = tok2 ? ad1 : ad;
    const int lg1 = tok2 ? 0 : 1;
    const bool two = tok2 || L > 4;
    constexpr int gstride = 4 * kMoeTok * kMoeRow;
    for (int64_t b = 0; b < nb; b += 2) {
      MoeStage nx{};
      if (b + 1 < nb) nx = moe_fetch(pl, b + 1);
      q6_block_mfma(w0, &sx[0][0], gstride, al, kg, fw, ad, a2, lg1, two);
      if (b + 2 < nb) w0 = q6_lane_load(drow + (b + 2) * 210, kg);
      if (b + 1 >= nb) break;
      moe_store(nx, pl, &sx[1][0]);
      __syncthreads();
      if (b + 2 < nb) nx = moe_fetch(pl, b + 2);
      q6_block_mfma(w1, &sx[1][0], gstride, al, kg, fw, ad, a2, lg1, two);
      if (b + 3 < nb) w1 = q6_lane_load(drow + (b + 3) * 210, kg);
      if (b + 2 >= nb) break;
      moe_store(nx, pl, &sx[0][0]);
      __syncthreads();
    }
    if (orow && t < tn) {
      bool f;
      const int64_t y = acc_shift(ad, fw, &f);
      if (!f) atomicOr(status, IMIE_EOVF);
      dout[(int64_t)ppair[it.first + t0 + t] * d_model + o] = y;
    }
    if (orow && tok2 && kMoeTok + t < tn) {
      bool f;
      const int64_t y = acc_shift(ad1, fw, &f);
      if (!f) atomicOr(status, IMIE_EOVF);
      dout[(int64_t)ppair[it.first + t0 + kMoeTok + t] * d_model + o] = y;
    }
    t0 += tn;
  }
}

// int8-MFMA path on/off (IMIE_QK_MFMA=0 forces the VALU kernel; tests compare both)
bool qk_mfma_enabled() {
  static const bool v = [] { const char* e = getenv("IMIE_QK_MFMA"); return !(e && atoi(e) == 0); }();
  return v;
}

// a Q4_K / Q6_K handle (int64 matrices registered by qk_register_i64 are qtype 2 and not accepted here)
const QKWeight* qk_get(int64_t h) {
  if (h < 0 || h >= (int64_t)g_qk.size() || !g_qk[(size_t)h].p || g_qk[(size_t)h].qtype > 1) return nullptr;
  return &g_qk[(size_t)h];
}

// Enqueue a set of items over device X (rows x K) into device Y (rows x ldy). pairs: host arrays. The int8-MFMA
// kernels run unless an activation row needs more than kQkLimbs limbs (or K is not a multiple of 256); then the
// exact VALU kernel does (both are enqueued, a device flag selects).
struct QkPrepWs {
  DevBuf xd, xs, lr, flag;
} g_qprep;

int run_items(const std::vector<Item>& items, const std::vector<int>& xi, const std::vector<int>& yi,
              const int64_t* X, int64_t K, int64_t* Y, int64_t ldy, int fw, int* status, hipStream_t st,
              DevBuf& ibuf, DevBuf& pbuf) {
  if (items.empty()) return IMIE_OK;
  const size_t np = xi.size();
  if (ibuf.ensure(items.size() * sizeof(Item)) || pbuf.ensure(np * 8)) return IMIE_EARG;
  IMIE_HIP(hipMemcpyAsync(ibuf.p, items.data(), items.size() * sizeof(Item), hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemcpyAsync(pbuf.p, xi.data(), np * 4, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemcpyAsync((int*)pbuf.p + np, yi.data(), np * 4, hipMemcpyHostToDevice, st));
  int64_t maxo = 0;
  for (auto& it : items) maxo = it.out_f > maxo ? it.out_f : maxo;
  int64_t rows = 0;
  for (int r : xi) rows = r + 1 > rows ? r + 1 : rows;
  const bool mfma_ok = K % 256 == 0 && qk_mfma_enabled();
  const int* gate = nullptr;
  imie_prof_mark(IMIE_K_QK, st, true);
  if (mfma_ok) {
    if (g_qprep.xd.ensure((size_t)(kQkLimbs * rows * K)) || g_qprep.xs.ensure((size_t)(rows * (K / 16)) * 8) ||
        g_qprep.lr.ensure((size_t)rows * 4) || g_qprep.flag.ensure(64))
      return IMIE_EARG;
    int* flag = (int*)g_qprep.flag.p;
    hipLaunchKernelGGL(qk_flag_reset_kernel, dim3(1), dim3(1), 0, st, flag);
    hipLaunchKernelGGL(qk_prep_kernel, dim3((unsigned)rows), dim3(256), 0, st, X, rows, K, (int8_t*)g_qprep.xd.p,
                       (int64_t*)g_qprep.xs.p, (int*)g_qprep.lr.p, flag);
    const dim3 grid((unsigned)((maxo + 63) / 64), (unsigned)items.size());
    constexpr int kDot4Max = 32;                      // items with at most this many tokens take the dot4 kernel
    bool q4s = false, q6s = false, q4b = false, q6b = false;
    for (auto& it : items) {
      const bool small = it.count <= kDot4Max;
      q4s = q4s || (it.qtype == 0 && small); q6s = q6s || (it.qtype == 1 && small);
      q4b = q4b || (it.qtype == 0 && !small); q6b = q6b || (it.qtype == 1 && !small);
    }
    const Item* ip = (const Item*)ibuf.p;
    const int *xip = (const int*)pbuf.p, *yip = (const int*)pbuf.p + np;
    const int8_t* xdp = (const int8_t*)g_qprep.xd.p;
    const int64_t* xsp = (const int64_t*)g_qprep.xs.p;
    const int* lrp = (const int*)g_qprep.lr.p;
    if (q4s) hipLaunchKernelGGL(qk_dot4_kernel<0>, grid, dim3(256), 0, st, ip, xip, yip, xdp, xsp, lrp, rows, K, Y, ldy, fw, status, flag, kDot4Max);
    if (q6s) hipLaunchKernelGGL(qk_dot4_kernel<1>, grid, dim3(256), 0, st, ip, xip, yip, xdp, xsp, lrp, rows, K, Y, ldy, fw, status, flag, kDot4Max);
    if (q4b) hipLaunchKernelGGL(qk_mfma_kernel<0>, grid, dim3(256), 0, st, ip, xip, yip, xdp, xsp, lrp, rows, K, Y, ldy, fw, status, flag, kDot4Max);
    if (q6b) hipLaunchKernelGGL(qk_mfma_kernel<1>, grid, dim3(256), 0, st, ip, xip, yip, xdp, xsp, lrp, rows, K, Y, ldy, fw, status, flag, kDot4Max);
    gate = flag;
  }
  hipLaunchKernelGGL(qk_group_kernel, dim3((unsigned)((maxo + kRows - 1) / kRows), (unsigned)items.size()),
                     dim3(256), 0, st, (const Item*)ibuf.p, (const int*)pbuf.p, (const int*)pbuf.p + np, X, K, Y,
                     ldy, fw, status, gate);
  imie_prof_mark(IMIE_K_QK, st, false);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

void silu_consts_nmc(int fa, int64_t* log2e, int64_t* dclip) {
  const int sh = 16 - fa;
  *log2e = sh >= 0 ? (94548 >> sh) : ((int64_t)94548 << -sh);
  *dclip = (((int64_t)fa + 2) << (2 * fa)) / *log2e;
}

int read_status_and(hipStream_t st, int* stat) {
  IMIE_HIP(hipMemcpyAsync(stat, g_mws.status.p, 4, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipStreamSynchronize(st));
  return IMIE_OK;
}

// Batched MoE: P = m*k pairs (token-major, pair p belongs to token p / k). Pairs sharing a weight run in one
// item, so each expert's gate/up/down are read once per call. This form runs each projection as its own item list
// (any quantisation types); moe_batched below takes the fused expert kernels when the layout allows.
int moe_batched_items(const long long* gate_h, const long long* up_h, const long long* down_h, int m, int k,
                      const int64_t* h_dev, const int64_t* gates_dev, int64_t d_model, int64_t e_ffn, int fa, int fw,
                      int64_t* out_dev, hipStream_t st) {
  const int64_t P = (int64_t)m * k;
  if (m <= 0 || k <= 0 || d_model <= 0 || e_ffn <= 0 || d_model % 256 || e_ffn % 256 || fa < 1 || fa > 28 || fw < 0 ||
      fw > 62)
    return IMIE_EARG;
  for (int64_t p = 0; p < P; ++p) {
    const QKWeight *g = qk_get(gate_h[p]), *u = qk_get(up_h[p]), *d = qk_get(down_h[p]);
    if (!g || !u || !d || g->out_f != e_ffn || g->nb * 256 != d_model || u->out_f != e_ffn || u->nb * 256 != d_model ||
        d->out_f != d_model || d->nb * 256 != e_ffn)
      return IMIE_EARG;
  }
  if (g_mws.g.ensure((size_t)(P * e_ffn) * 8) || g_mws.u.ensure((size_t)(P * e_ffn) * 8) ||
      g_mws.d.ensure((size_t)(P * d_model) * 8) || g_mws.status.ensure(64))
    return IMIE_EARG;
  int64_t *gb = (int64_t*)g_mws.g.p, *ub = (int64_t*)g_mws.u.p, *db = (int64_t*)g_mws.d.p;
  int* status = (int*)g_mws.status.p;
  // group pairs by weight handle
  auto build = [&](const long long* hs, bool x_per_pair, std::vector<Item>& items, std::vector<int>& xi,
                   std::vector<int>& yi) {
    std::map<long long, std::vector<int>> groups;
    for (int64_t p = 0; p < P; ++p) groups[hs[p]].push_back((int)p);
    for (auto& kv : groups) {
      const QKWeight* w = qk_get(kv.first);
      Item it{w->p, w->out_f, w->nb, w->qtype, (int)xi.size(), (int)kv.second.size()};
      for (int p : kv.second) { xi.push_back(x_per_pair ? p : p / k); yi.push_back(p); }
      items.push_back(it);
    }
  };
  std::vector<Item> ig, iu, idn;
  std::vector<int> xg, yg, xu, yu, xd, yd;
  build(gate_h, false, ig, xg, yg);
  build(up_h, false, iu, xu, yu);
  build(down_h, true, idn, xd, yd);
  static DevBuf ib1, pb1, ib2, pb2, ib3, pb3;
  int rc = run_items(ig, xg, yg, h_dev, d_model, gb, e_ffn, fw, status, st, ib1, pb1);
  if (!rc) rc = run_items(iu, xu, yu, h_dev, d_model, ub, e_ffn, fw, status, st, ib2, pb2);
  if (rc) return rc;
  int64_t log2e, dclip;
  silu_consts_nmc(fa, &log2e, &dclip);
  const int64_t n = P * e_ffn;
  hipLaunchKernelGGL(qk_silu_mul_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, gb, ub, n, fa, log2e,
                     dclip, gb, status);
  IMIE_HIP(hipGetLastError());
  rc = run_items(idn, xd, yd, gb, e_ffn, db, d_model, fw, status, st, ib3, pb3);
  if (rc) return rc;
  hipLaunchKernelGGL(qk_combine_kernel, dim3((unsigned)(((int64_t)m * d_model + 255) / 256)), dim3(256), 0, st, db,
                     m, k, d_model, gates_dev, fa, out_dev, status);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

// Batched MoE with the fused expert kernels (Q4_K gate/up, Q6_K down): one item per expert, its pairs listed
// once. Sequence: prep(h) -> gate/up + SiLU*up -> prep(gu) -> down -> combine. When an activation row needs more
// than kQkLimbs digit limbs, the prep sets a device flag: the fused kernels return at once and the exact VALU item
// kernels (enqueued behind them, gated by the same flag) compute that stage instead, with no host round trip.
int moe_batched(const long long* gate_h, const long long* up_h, const long long* down_h, int m, int k,
                const int64_t* h_dev, const int64_t* gates_dev, int64_t d_model, int64_t e_ffn, int fa, int fw,
                int64_t* out_dev, hipStream_t st) {
  const int64_t P = (int64_t)m * k;
  if (m <= 0 || k <= 0 || d_model <= 0 || e_ffn <= 0 || d_model % 256 || e_ffn % 256 || fa < 1 || fa > 28 || fw < 0 ||
      fw > 62)
    return IMIE_EARG;
  bool fused = fw <= kMaxFw && qk_mfma_enabled();
  for (int64_t p = 0; p < P && fused; ++p) {
    const QKWeight *g = qk_get(gate_h[p]), *u = qk_get(up_h[p]), *d = qk_get(down_h[p]);
    if (!g || !u || !d) return IMIE_EARG;
    fused = g->qtype == 0 && u->qtype == 0 && d->qtype == 1;
  }
  if (!fused)
    return moe_batched_items(gate_h, up_h, down_h, m, k, h_dev, gates_dev, d_model, e_ffn, fa, fw, out_dev, st);
  for (int64_t p = 0; p < P; ++p) {
    const QKWeight *g = qk_get(gate_h[p]), *u = qk_get(up_h[p]), *d = qk_get(down_h[p]);
    if (g->out_f != e_ffn || g->nb * 256 != d_model || u->out_f != e_ffn || u->nb * 256 != d_model ||
        d->out_f != d_model || d->nb * 256 != e_ffn)
      return IMIE_EARG;
  }
  if (g_mws.g.ensure((size_t)(P * e_ffn) * 8) || g_mws.u.ensure((size_t)(P * e_ffn) * 8) ||
      g_mws.d.ensure((size_t)(P * d_model) * 8) || g_mws.status.ensure(64))
    return IMIE_EARG;
  int64_t *gb = (int64_t*)g_mws.g.p, *ub = (int64_t*)g_mws.u.p, *db = (int64_t*)g_mws.d.p;
  int* status = (int*)g_mws.status.p;
  // experts = distinct (gate, up, down) handle triples; pairs listed expert by expert
  std::map<std::tuple<long long, long long, long long>, std::vector<int>> groups;
  for (int64_t p = 0; p < P; ++p) groups[std::make_tuple(gate_h[p], up_h[p], down_h[p])].push_back((int)p);
  const size_t ne = groups.size();
  std::vector<MoeItem> mi;
  std::vector<Item> ig, iu, idn;
  std::vector<int> ptok, ppair;
  mi.reserve(ne);
  for (auto& kv : groups) {
    const QKWeight* g = qk_get(std::get<0>(kv.first));
    const QKWeight* u = qk_get(std::get<1>(kv.first));
    const QKWeight* d = qk_get(std::get<2>(kv.first));
    const int first = (int)ptok.size(), count = (int)kv.second.size();
    mi.push_back(MoeItem{g->p, u->p, d->p, first, count});
    ig.push_back(Item{g->p, g->out_f, g->nb, g->qtype, first, count});
    iu.push_back(Item{u->p, u->out_f, u->nb, u->qtype, first, count});
    idn.push_back(Item{d->p, d->out_f, d->nb, d->qtype, first, count});
    for (int p : kv.second) { ptok.push_back(p / k); ppair.push_back(p); }
  }
  // one upload: [MoeItem x ne][Item gate x ne][Item up x ne][Item down x ne][ptok P][ppair P]
  static DevBuf meta;
  const size_t o_items = 0, o_ig = o_items + ne * sizeof(MoeItem), o_iu = o_ig + ne * sizeof(Item),
               o_id = o_iu + ne * sizeof(Item), o_pt = o_id + ne * sizeof(Item), o_pp = o_pt + (size_t)P * 4,
               total = o_pp + (size_t)P * 4;
  static std::vector<uint8_t> hb;                     // pageable staging: the async copy reads it before returning
  hb.resize(total);
  memcpy(hb.data() + o_items, mi.data(), ne * sizeof(MoeItem));
  memcpy(hb.data() + o_ig, ig.data(), ne * sizeof(Item));
  memcpy(hb.data() + o_iu, iu.data(), ne * sizeof(Item));
  memcpy(hb.data() + o_id, idn.data(), ne * sizeof(Item));
  memcpy(hb.data() + o_pt, ptok.data(), (size_t)P * 4);
  memcpy(hb.data() + o_pp, ppair.data(), (size_t)P * 4);
  if (meta.ensure(total)) return IMIE_EARG;
  IMIE_HIP(hipMemcpyAsync(meta.p, hb.data(), total, hipMemcpyHostToDevice, st));
  const uint8_t* mb = (const uint8_t*)meta.p;
  const MoeItem* d_items = (const MoeItem*)(mb + o_items);
  const Item *d_ig = (const Item*)(mb + o_ig), *d_iu = (const Item*)(mb + o_iu), *d_id = (const Item*)(mb + o_id);
  const int *d_pt = (const int*)(mb + o_pt), *d_pp = (const int*)(mb + o_pp);
  const int64_t prow = P > m ? P : m, pk = d_model > e_ffn ? d_model : e_ffn;
  if (g_qprep.xd.ensure((size_t)(kQkLimbs * prow * pk)) || g_qprep.xs.ensure((size_t)(prow * (pk / 16)) * 8) ||
      g_qprep.lr.ensure((size_t)prow * 4) || g_qprep.flag.ensure(64))
    return IMIE_EARG;
  int* flagA = (int*)g_qprep.flag.p;
  int* flagB = flagA + 1;
  int8_t* xdp = (int8_t*)g_qprep.xd.p;
  int64_t* xsp = (int64_t*)g_qprep.xs.p;
  int* lrp = (int*)g_qprep.lr.p;
  int64_t log2e, dclip;
  silu_consts_nmc(fa, &log2e, &dclip);
  imie_prof_mark(IMIE_K_QK, st, true);
  // the wide-row flags start clear: the previous call's combine kernel cleared them (a fresh or foreign value
  // only costs a run of the exact fallbacks, whose results equal the fused kernels')
  // the fused expert kernels read no 16-element sums (their min terms are MFMA accumulations)
  hipLaunchKernelGGL(qk_prep_kernel, dim3((unsigned)m), dim3(256), 0, st, h_dev, (int64_t)m, d_model, xdp, nullptr, lrp,
                     flagA);
  hipLaunchKernelGGL(moe_gateup_kernel, dim3((unsigned)((e_ffn + 63) / 64),
                     (unsigned)ne), dim3(256), moe_lds_bytes(d_model), st, d_items,
                     d_pt, d_pp, xdp, lrp, (int64_t)m, d_model, e_ffn, fw, fa, log2e, dclip, gb, status, flagA);
  // exact VALU fallback of the gate/up stage (runs only when the prep flagged a wide activation row)
  const int64_t ntg = (e_ffn + kRows - 1) / kRows;
  hipLaunchKernelGGL(qk_gateup_gated_kernel, dim3(kGatedWgs2), dim3(256), 0, st, d_ig, d_iu, d_pt, d_pp, h_dev,
                     d_model, gb, ub, e_ffn, fw, fa, log2e, dclip, status, flagA, ntg, (int64_t)ne);
  // down over the P rows of gu
  hipLaunchKernelGGL(qk_prep_kernel, dim3((unsigned)P), dim3(256), 0, st, gb, P, e_ffn, xdp, nullptr, lrp, flagB);
  hipLaunchKernelGGL(moe_down_kernel, dim3((unsigned)((d_model + 63) / 64), (unsigned)ne), dim3(256), 0, st, d_items,
                     d_pp, xdp, xsp, lrp, P, e_ffn, d_model, fw, db, status, flagB);
  hipLaunchKernelGGL(qk_group_gated_kernel, dim3(kGatedWgs), dim3(256), 0, st, d_id, d_pp, d_pp, gb, e_ffn, db,
                     d_model, fw, status, flagB, (int64_t)((d_model + kRows - 1) / kRows), (int64_t)ne);
  hipLaunchKernelGGL(qk_combine_kernel, dim3((unsigned)(((int64_t)m * d_model + 255) / 256)), dim3(256), 0, st, db,
                     m, k, d_model, gates_dev, fa, out_dev, status, flagA);
  imie_prof_mark(IMIE_K_QK, st, false);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

int host_linear(const std::vector<int64_t>& handles, const int64_t* x, int64_t T, int fw, int64_t* out_flat) {
  // all handles share the input width; outputs concatenated handle-major (each T x out_f)
  hipStream_t st = imie_stream();
  const QKWeight* w0 = qk_get(handles[0]);
  const int64_t K = w0->nb * 256;
  int64_t total = 0;
  for (auto h : handles) total += T * qk_get(h)->out_f;
  if (g_mws.x.ensure((size_t)(T * K) * 8) || g_mws.y.ensure((size_t)total * 8) || g_mws.status.ensure(64))
    return IMIE_EARG;
  IMIE_HIP(hipMemcpyAsync(g_mws.x.p, x, (size_t)(T * K) * 8, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemsetAsync(g_mws.status.p, 0, 4, st));
  prof(PM_H2D_CALLS); prof(PM_H2D_BYTES, (unsigned long long)(T * K * 8));
  int64_t off = 0;
  static DevBuf ib, pb;
  for (auto h : handles) {
    const QKWeight* w = qk_get(h);
    std::vector<Item> items{Item{w->p, w->out_f, w->nb, w->qtype, 0, (int)T}};
    std::vector<int> xi((size_t)T), yi((size_t)T);
    for (int64_t t = 0; t < T; ++t) { xi[(size_t)t] = (int)t; yi[(size_t)t] = (int)t; }
    int rc = run_items(items, xi, yi, (const int64_t*)g_mws.x.p, K, (int64_t*)g_mws.y.p + off, w->out_f, fw,
                       (int*)g_mws.status.p, st, ib, pb);
    if (rc) return rc;
    IMIE_HIP(hipStreamSynchronize(st));   // ib/pb are reused by the next handle
    off += T * w->out_f;
  }
  int stat = 0;
  if (read_status_and(st, &stat)) return IMIE_EARG;
  IMIE_HIP(hipMemcpy(out_flat, g_mws.y.p, (size_t)total * 8, hipMemcpyDeviceToHost));
  prof(PM_D2H_CALLS); prof(PM_D2H_BYTES, (unsigned long long)(total * 8));
  return stat ? IMIE_EOVF : IMIE_OK;
}

int64_t qk_register(const uint8_t* W, int64_t out_f, int64_t nb, int qtype) {
  if (!W || out_f <= 0 || nb <= 0 || (qtype != 0 && qtype != 1) || imie_device_ready() != 0) return -1;
  QKWeight w;
  w.out_f = out_f; w.nb = nb; w.qtype = qtype;
  w.bytes = (size_t)(out_f * nb) * (qtype == 0 ? 144 : 210);
  if (hipMalloc((void**)&w.p, w.bytes) != hipSuccess) return -1;
  if (hipMemcpy(w.p, W, w.bytes, hipMemcpyHostToDevice) != hipSuccess) { imie_free(w.p); return -1; }
  g_qk.push_back(w);
  ++g_qk_live;
  prof(PM_REG_CALLS); prof(PM_ALLOC_CALLS); prof(PM_ALLOC_BYTES, w.bytes);
  return (int64_t)g_qk.size() - 1;
}

}  // namespace

// ---- internal API for the resident attention bank (csrc/nmcbank.hip) --------------------------------------------
int imie_qk_info(int64_t h, int64_t* out_f, int64_t* nb, int* qtype, const uint8_t** p) {
  if (h < 0 || h >= (int64_t)g_qk.size() || !g_qk[(size_t)h].p) return IMIE_EARG;
  const QKWeight& w = g_qk[(size_t)h];
  if (out_f) *out_f = w.out_f;
  if (nb) *nb = w.nb;
  if (qtype) *qtype = w.qtype;
  if (p) *p = w.p;
  return IMIE_OK;
}

// int64 matrix [rows, cols] registered as qtype 2 (nb holds cols)
int64_t imie_qk_register_i64(const int64_t* W, int64_t rows, int64_t cols) {
  if (!W || rows <= 0 || cols <= 0 || imie_device_ready() != 0) return -1;
  QKWeight w;
  w.out_f = rows; w.nb = cols; w.qtype = 2;
  w.bytes = (size_t)(rows * cols) * 8;
  if (hipMalloc((void**)&w.p, w.bytes) != hipSuccess) return -1;
  if (hipMemcpy(w.p, W, w.bytes, hipMemcpyHostToDevice) != hipSuccess) { imie_free(w.p); return -1; }
  g_qk.push_back(w);
  ++g_qk_live;
  prof(PM_REG_CALLS); prof(PM_ALLOC_CALLS); prof(PM_ALLOC_BYTES, w.bytes);
  return (int64_t)g_qk.size() - 1;
}

// y[t, :] = (W . x[t, :]) >> fw for T device rows into device out (T x out_f); status gets IMIE_EOVF where the
// oracle's int64 conversion would raise
int imie_qk_linear_dev(int64_t h, const int64_t* x, int64_t T, int fw, int64_t* out, int* status, hipStream_t st) {
  const QKWeight* w = qk_get(h);
  if (!w || !x || !out || !status || T <= 0) return IMIE_EARG;
  std::vector<Item> items{Item{w->p, w->out_f, w->nb, w->qtype, 0, (int)T}};
  std::vector<int> xi((size_t)T), yi((size_t)T);
  for (int64_t t = 0; t < T; ++t) { xi[(size_t)t] = (int)t; yi[(size_t)t] = (int)t; }
  static DevBuf ib[4], pb[4];
  static int slot = 0;
  slot = (slot + 1) & 3;                              // distinct item buffers for back-to-back launches
  return run_items(items, xi, yi, x, w->nb * 256, out, w->out_f, fw, status, st, ib[slot], pb[slot]);
}

// one token's MoE over k selected experts (host handle arrays), gates on the device; synchronous; 0, or IMIE_EOVF
// where the oracle's int64 conversions would raise
int imie_qk_moe_dev(const long long* gate_h, const long long* up_h, const long long* down_h, int k,
                    const int64_t* h_dev, const int64_t* gates_dev, int64_t d_model, int64_t e_ffn, int fa, int fw,
                    int64_t* out_dev, hipStream_t st) {
  if (g_mws.status.ensure(64)) return IMIE_EARG;
  IMIE_HIP(hipMemsetAsync(g_mws.status.p, 0, 4, st));
  int rc = moe_batched(gate_h, up_h, down_h, 1, k, h_dev, gates_dev, d_model, e_ffn, fa, fw, out_dev, st);
  if (rc) return rc;
  int stat = 0;
  if (read_status_and(st, &stat)) return IMIE_EARG;
  return stat ? IMIE_EOVF : IMIE_OK;
}

extern "C" {

// fp16 -> fixed point as the Q4_K / Q6_K kernels compute it (fp16_fixed_fast), over n host values; synchronous.
// Test hook (no reference counterpart): the exhaustive check against the oracle's integer rule.
int imie_fp16_fixed_probe(const uint16_t* h, int64_t n, int fw, int64_t* out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!h || !out || n <= 0 || fw < 0 || fw > 62 || imie_device_ready() != 0) return IMIE_EARG;
  hipStream_t st = imie_stream();
  static DevBuf a, b;                                 // grow-only staging, like the other host-pointer entry points
  if (a.ensure((size_t)n * 2) || b.ensure((size_t)n * 8)) return IMIE_EARG;
  IMIE_HIP(hipMemcpyAsync(a.p, h, (size_t)n * 2, hipMemcpyHostToDevice, st));
  hipLaunchKernelGGL(fp16_fixed_probe_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, (const uint16_t*)a.p,
                     n, fw, (int64_t*)b.p);
  IMIE_HIP(hipGetLastError());
  IMIE_HIP(hipMemcpyAsync(out, b.p, (size_t)n * 8, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipStreamSynchronize(st));
  return IMIE_OK;
}

// nmc_qk_cuda.cu:755 `qk_cuda_abi_version`; the reference bridge requires 5 (qk_cuda.py:22, 83-92).
int qk_cuda_abi_version(void) { return 5; }

// nmc_qk_cuda.cu `qk_cuda_available`: 0 iff usable.
int qk_cuda_available(void) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  return imie_device_ready();
}

// nmc_qk_cuda.cu:720 `qk_linear_cuda` (qk_cuda.py:230-244): per-call weight upload, y [T, out_f].
int qk_linear_cuda(const uint8_t* W, const int64_t* x, long long T, long long out_f, long long n_blocks, int fw,
                   int qtype, int64_t* out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  prof(PM_NATIVE_CALLS);
  if (!W || !x || !out || T < 0 || out_f <= 0 || n_blocks <= 0 || fw < 0 || fw > kMaxFw) return IMIE_EARG;
  if (T == 0) return IMIE_OK;
  const int64_t h = qk_register(W, out_f, n_blocks, qtype);
  if (h < 0) return IMIE_EARG;
  const int rc = host_linear({h}, x, T, fw, out);
  imie_free(g_qk[(size_t)h].p);
  g_qk[(size_t)h].p = nullptr;
  --g_qk_live;
  if (h == (int64_t)g_qk.size() - 1) g_qk.pop_back();
  return rc;
}

// nmc_qk_cuda.cu:1046 `qk_register_weight` (qk_cuda.py:252-270): raw Q4_K (0) / Q6_K (1) bytes -> handle.
long long qk_register_weight(const uint8_t* W, long long out_f, long long n_blocks, int qtype) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  return qk_register(W, out_f, n_blocks, qtype);
}

// nmc_qk_cuda.cu:1040 `qk_resident_reserve`: registry metadata only.
int qk_resident_reserve(long long count) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (count < 0) return IMIE_EARG;
  g_qk.reserve((size_t)count);
  return IMIE_OK;
}

// nmc_qk_cuda.cu:1252 `qk_apply_resident` (qk_cuda.py:387-397).
int qk_apply_resident(long long h, const int64_t* x, long long T, int fw, int64_t* out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  prof(PM_RESIDENT_CALLS);
  if (!qk_get(h) || !x || !out || T < 0 || fw < 0 || fw > kMaxFw) return IMIE_EARG;
  if (T == 0) return IMIE_OK;
  return host_linear({(int64_t)h}, x, T, fw, out);
}

// nmc_qk_cuda.cu:1284 `qk_apply_resident_grouped` (qk_cuda.py:405-442): same-input projections, one H2D and
// one D2H; outputs concatenated handle-major. phase_ids only feed the Q/K/V/O counters.
int qk_apply_resident_grouped(const long long* handles, const int* phase_ids, int count, const int64_t* x,
                              long long rows, int fw, long long total, int64_t* out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  prof(PM_GROUPED_CALLS);
  if (!handles || !x || !out || count <= 0 || count > 16 || rows <= 0 || fw < 0 || fw > kMaxFw) return IMIE_EARG;
  std::vector<int64_t> hs;
  int64_t K = -1, want = 0;
  for (int i = 0; i < count; ++i) {
    const QKWeight* w = qk_get(handles[i]);
    if (!w || (K >= 0 && w->nb * 256 != K)) return IMIE_EARG;
    K = w->nb * 256;
    want += rows * w->out_f;
    hs.push_back(handles[i]);
    if (phase_ids) {
      const int ph = phase_ids[i];
      prof(ph == 1 ? PM_Q_CALLS : ph == 2 ? PM_K_CALLS : ph == 3 ? PM_V_CALLS : ph == 4 ? PM_O_CALLS : PM_OTHER_CALLS);
    }
  }
  if (want != total) return IMIE_EARG;
  return host_linear(hs, x, rows, fw, out);
}

// DP4A entries (nmc_qk_cuda.cu:1932, :2003): on gfx950 the same exact kernel serves every limb count, so these
// return the apply_resident result after the reference's argument checks (Ln in [1, 8], matching qtype).
int qk_apply_resident_q6k_dp4a(long long h, const int64_t* x, long long T, int fw, int Ln, int64_t* out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  const QKWeight* w = qk_get(h);
  if (!w || w->qtype != 1 || Ln < 1 || Ln > 8) return IMIE_EARG;
  return qk_apply_resident(h, x, T, fw, out);
}
int qk_apply_resident_q4k_dp4a(long long h, const int64_t* x, long long T, int fw, int Ln, int64_t* out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  const QKWeight* w = qk_get(h);
  if (!w || w->qtype != 0 || Ln < 1 || Ln > 8) return IMIE_EARG;
  return qk_apply_resident(h, x, T, fw, out);
}

// nmc_qk_cuda.cu:2203-2254 `qk_moe_ffn_batched` (qk_cuda.py:1073-1101): host h [m, d_model], gates [m*k],
// handles flattened token-major; out [m, d_model]. rc 2 where the oracle's int64 conversions would raise.
int qk_moe_ffn_batched(const long long* gate_h, const long long* up_h, const long long* down_h, int m, int k,
                       const int64_t* h, const int64_t* gates, long long d_model, long long e_ffn, int fa, int fw,
                       int64_t* out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  prof(PM_MOE_BATCHED_CALLS);
  if (!gate_h || !up_h || !down_h || !h || !gates || !out || m <= 0 || k <= 0) return IMIE_EARG;
  hipStream_t st = imie_stream();
  const int64_t P = (int64_t)m * k;
  if (g_mws.x.ensure((size_t)(m * d_model) * 8) || g_mws.gates.ensure((size_t)P * 8) ||
      g_mws.out.ensure((size_t)(m * d_model) * 8) || g_mws.status.ensure(64))
    return IMIE_EARG;
  IMIE_HIP(hipMemcpyAsync(g_mws.x.p, h, (size_t)(m * d_model) * 8, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemcpyAsync(g_mws.gates.p, gates, (size_t)P * 8, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemsetAsync(g_mws.status.p, 0, 4, st));
  int rc = moe_batched(gate_h, up_h, down_h, m, k, (const int64_t*)g_mws.x.p, (const int64_t*)g_mws.gates.p,
                       d_model, e_ffn, fa, fw, (int64_t*)g_mws.out.p, st);
  if (rc) return rc;
  int stat = 0;
  if (read_status_and(st, &stat)) return IMIE_EARG;
  if (stat) return IMIE_EOVF;
  IMIE_HIP(hipMemcpy(out, g_mws.out.p, (size_t)(m * d_model) * 8, hipMemcpyDeviceToHost));
  return IMIE_OK;
}

// Guarded-limb batched entry (nmc_qk_cuda.cu:2261): exact for every activation here, never rc 2 for the limb
// envelope; overflow of the int64 results still returns 2 (the caller then runs the int128 entry, which agrees).
int qk_moe_ffn_batched_dp4a(const long long* gate_h, const long long* up_h, const long long* down_h, int m, int k,
                            const int64_t* h, const int64_t* gates, long long d_model, long long e_ffn, int fa, int fw,
                            int64_t* out) {
  prof(PM_MOE_BATCHED_DP4A_CALLS);
  return qk_moe_ffn_batched(gate_h, up_h, down_h, m, k, h, gates, d_model, e_ffn, fa, fw, out);
}

// nmc_qk_cuda.cu:1816 `qk_moe_ffn` (qk_cuda.py:1104-1124): one token, n_e selected experts, out [d_model].
int qk_moe_ffn(const long long* gate_h, const long long* up_h, const long long* down_h, int n_e, const int64_t* h,
               const int64_t* gates, long long d_model, long long e_ffn, int fa, int fw, int64_t* out) {
  prof(PM_MOE_CALLS);
  return qk_moe_ffn_batched(gate_h, up_h, down_h, 1, n_e, h, gates, d_model, e_ffn, fa, fw, out);
}
int qk_moe_ffn_dp4a(const long long* gate_h, const long long* up_h, const long long* down_h, int n_e, const int64_t* h,
                    const int64_t* gates, long long d_model, long long e_ffn, int fa, int fw, int64_t* out) {
  return qk_moe_ffn(gate_h, up_h, down_h, n_e, h, gates, d_model, e_ffn, fa, fw, out);
}

// Device-pointer batched MoE (no reference counterpart): h_dev [m, d_model], gates_dev [m*k], out_dev [m, d_model];
// status_dev receives bit 2 on an int64 envelope miss. Asynchronous on `stream`.
int imie_moe_ffn_batched_dev(const long long* gate_h, const long long* up_h, const long long* down_h, int m, int k,
                             const int64_t* h_dev, const int64_t* gates_dev, long long d_model, long long e_ffn,
                             int fa, int fw, int64_t* out_dev, void* stream) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!gate_h || !up_h || !down_h || !h_dev || !gates_dev || !out_dev) return IMIE_EARG;
  if (g_mws.status.ensure(64)) return IMIE_EARG;
  return moe_batched(gate_h, up_h, down_h, m, k, h_dev, gates_dev, d_model, e_ffn, fa, fw, out_dev,
                     (hipStream_t)stream);
}

int imie_moe_status(int clear, void* stream) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (g_mws.status.ensure(64)) return -1;
  hipStream_t st = (hipStream_t)stream;
  if (clear) return hipMemsetAsync(g_mws.status.p, 0, 4, st) == hipSuccess ? 0 : -1;
  int stat = 0;
  if (hipMemcpyAsync(&stat, g_mws.status.p, 4, hipMemcpyDeviceToHost, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess)
    return -1;
  return stat;
}

void qk_free_all(void) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  (void)hipDeviceSynchronize();
  for (auto& w : g_qk) if (w.p) { imie_free(w.p); prof(PM_FREE_CALLS); }
  g_qk.clear();
  g_qk_live = 0;
}

long long qk_resident_count(void) { return (long long)g_qk_live; }
long long qk_resident_capacity(void) { return (long long)g_qk.capacity(); }
long long qk_moe_workspace_allocations(void) { return 0; }
unsigned long long qk_moe_workspace_bytes(void) {
  return (unsigned long long)(g_mws.g.cap + g_mws.u.cap + g_mws.d.cap + g_mws.x.cap + g_mws.out.cap);
}
void qk_moe_workspace_release(void) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  (void)hipDeviceSynchronize();
  g_mws.g.release(); g_mws.u.release(); g_mws.d.release(); g_mws.x.release(); g_mws.out.release();
}

void qk_profile_reset(void) { memset(g_prof, 0, sizeof(g_prof)); }
void qk_profile_set_enabled(int enabled) { g_prof_on = enabled ? 1 : 0; }
// Copies min(capacity, PM_COUNT) counters; returns the number of counters the library keeps.
int qk_profile_snapshot(unsigned long long* out, int capacity) {
  if (out) for (int i = 0; i < capacity && i < PM_COUNT; ++i) out[i] = g_prof[i];
  return PM_COUNT;
}

}  // extern "C"
