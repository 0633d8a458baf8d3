// Q1_0 activation "prep": the balanced base-256 digit table of x that the MFMA matvec consumes, computed by one
// full wave per (token t, 512-wide slab). Shared by the stand-alone prep kernel and by the producers that fuse it
// into their epilogue (RMSNorm, SiLU * up), so a matvec can start from a table written by the kernel before it.
//
// Lane layout: g = lane >> 4 (block of the slab), s = lane & 7, dh = (lane >> 3) & 1; the lane's 8 positions are
// block * 128 + 32 d + 8 c + s for d in {2 dh, 2 dh + 1}, c = 0..3. Outputs per (t, slab): the limb count L (from
// the slab's max|x|), per-block totals, and xq[t][l][block][s] (uint4: dword d packs the digits of positions
// 32 d + 8 c + s as bytes c).
#pragma once
#include "imie_common.h"

namespace imie_q1 {

constexpr int kSlabBlocks = 4;     // 128-blocks per slab (= K 512 per wave step)
constexpr int kMaxLimbs = 8;
constexpr int kMaxSegs = 3;        // weights sharing one activation in a single matvec launch
constexpr int kGemmMinT = 8;       // from this many tokens the Q1 linear runs as an MFMA GEMM (own digit layout)

struct Q1PrepOut {                 // where a prep writes its table (sized for T tokens of nb blocks)
  uint32_t* xq;
  int64_t* totals;
  int* lslab;
  int64_t nb, nbp, nslabs;
};

struct GemmPrepOut {               // the GEMM digit table (T >= kGemmMinT): xg[limb][block][Tp][s], tg, lt
  uint4* xg;
  int64_t* tg;
  int* lt;
  int64_t nb, nbp, nslabs, Tp;
};
constexpr int kGemmNarrowLimbs = 3;  // the GEMM's narrow kernels read 3 limbs; the prep zero-fills up to that

struct Q1Zero {                    // outputs a producer clears before a K-split matvec adds into them
  int64_t* p[kMaxSegs];
  int64_t n[kMaxSegs];
  int cnt;
};

// Matvec prologue (single-token decode): the matvec workgroups derive their slab range's digit table from the
// producer's inputs themselves instead of reading a table a separate kernel wrote.
enum { kProNone = 0, kProCopy = 1, kProSiluMul = 2, kProNorm = 3 };
struct Q1Pro {
  const int64_t* x;                // activations (kProCopy), gate (kProSiluMul), the row to normalise (kProNorm)
  const int64_t* x2;               // kProSiluMul: up
  const int64_t* gain;             // kProNorm: gain (cols)
  const uint64_t* gmax;            // kProNorm: max |gain| (one device word, written by an earlier kernel)
  int64_t cols;                    // length of x (= the matvec's K)
  int64_t eps, log2e, dclip;       // kProNorm: eps; kProSiluMul: log2(e) and the exponent clip
  int frac;                        // the producer's fixed-point fraction bits
  int* status;                     // kProNorm: refusal bit 4
  Q1Zero zero;                     // outputs of a later K-split matvec, cleared by these workgroups
};

__device__ inline int64_t prep_pos(int lane, int64_t sl, int q) {
  const int g = lane >> 4, s = lane & 7, dh = (lane >> 3) & 1;
  const int d = 2 * dh + (q >> 2), c = q & 3;
  return (sl * kSlabBlocks + g) * 128 + 32 * d + 8 * c + s;
}

// v[q] = x at prep_pos(lane, sl, q) (0 for blocks >= nb); every lane of the wave participates.
__device__ inline void prep_slab(int64_t v[8], const Q1PrepOut& po, int64_t t, int64_t sl) {
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, s = lane & 7, dh = (lane >> 3) & 1;
  const int64_t blk = sl * kSlabBlocks + g;
  uint64_t mx = 0;
  int64_t part = 0;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const uint64_t a = imie_absu64(v[q]);
    mx = a > mx ? a : mx;
    part = (int64_t)((uint64_t)part + (uint64_t)v[q]);
  }
  mx = imie_wave_max_u64_full(mx);
  const int L = imie_limbs_needed(mx);
  // block total: sum over the 16 lanes of group g (one DPP row)
  part = (int64_t)imie_row_sum_u64_full((uint64_t)part);
  if ((lane & 15) == 0) po.totals[t * po.nbp + blk] = part;
  if (lane == 0) po.lslab[t * po.nslabs + sl] = L;
  for (int l = 0; l < L; ++l) {
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int64_t dig = ((v[q] + 128) & 255) - 128;          // balanced digit in [-128, 127]
      v[q] = (int64_t)(((uint64_t)v[q] - (uint64_t)dig)) >> 8;  // exact: v - dig is a multiple of 256
      const uint32_t byte = (uint32_t)(dig & 0xFF) << (8 * (q & 3));
      if (q < 4) w0 |= byte; else w1 |= byte;
    }
    uint32_t* dst = po.xq + ((((t * kMaxLimbs + l) * po.nbp + blk) * 8 + s) * 4);
    *(uint2*)(dst + 2 * dh) = uint2{w0, w1};
  }
}

// prep_slab into LDS: the slab's limb count, block totals and digits for a workgroup-local table laid out as the
// global one of a single token (dst[l * 32 + block * 8 + s], eight limbs); every lane of the wave participates.
__device__ inline void prep_slab_lds(int64_t v[8], uint4* dst, int* L_out, int64_t* tot_out) {
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, s = lane & 7, dh = (lane >> 3) & 1;
  uint64_t mx = 0;
  int64_t part = 0;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const uint64_t a = imie_absu64(v[q]);
    mx = a > mx ? a : mx;
    part = (int64_t)((uint64_t)part + (uint64_t)v[q]);
  }
  mx = imie_wave_max_u64_full(mx);
  const int L = imie_limbs_needed(mx);
  part = (int64_t)imie_row_sum_u64_full((uint64_t)part);
  if ((lane & 15) == 0) tot_out[g] = part;
  if (lane == 0) *L_out = L;
  for (int l = 0; l < L; ++l) {
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int64_t dig = ((v[q] + 128) & 255) - 128;
      v[q] = (int64_t)(((uint64_t)v[q] - (uint64_t)dig)) >> 8;
      const uint32_t byte = (uint32_t)(dig & 0xFF) << (8 * (q & 3));
      if (q < 4) w0 |= byte; else w1 |= byte;
    }
    *(uint2*)((uint32_t*)(dst + l * 32 + g * 8 + s) + 2 * dh) = uint2{w0, w1};
  }
}

// workgroup `wg` of `nwg` clears its share of the zero list (threads tid of nthreads)
__device__ inline void zero_share(const Q1Zero& z, int64_t wg, int64_t nwg, int tid, int nthreads) {
  for (int i = 0; i < z.cnt; ++i)
    for (int64_t e = wg * nthreads + tid; e < z.n[i]; e += nwg * nthreads) z.p[i][e] = 0;
}

// GEMM table entries of token t, slab sl from v[q] = x at prep_pos(lane, sl, q) (0 beyond the row): the slab's
// limb count (its max|x| over the 64 lanes), per-block totals, and balanced base-256 digits for every limb up to
// max(L, kGemmNarrowLimbs) (zeros above L). One full wave.
__device__ inline void prep_gemm_slab(int64_t v[8], const GemmPrepOut& gp, int64_t t, int64_t sl) {
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, s = lane & 7, dh = (lane >> 3) & 1;
  const int64_t blk = sl * kSlabBlocks + g;
  uint64_t mx = 0;
  int64_t part = 0;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const uint64_t a = imie_absu64(v[q]);
    mx = a > mx ? a : mx;
    part = (int64_t)((uint64_t)part + (uint64_t)v[q]);
  }
  mx = imie_wave_max_u64_full(mx);
  const int L = imie_limbs_needed(mx);
  part = (int64_t)imie_row_sum_u64_full((uint64_t)part);   // block total: the 16 lanes of group g (one DPP row)
  if ((lane & 15) == 0) gp.tg[blk * gp.Tp + t] = part;
  if (lane == 0) gp.lt[t * gp.nslabs + sl] = L;
  const int Lw = L > kGemmNarrowLimbs ? L : kGemmNarrowLimbs;
  for (int l = 0; l < Lw; ++l) {
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int64_t dig = ((v[q] + 128) & 255) - 128;
      v[q] = (int64_t)(((uint64_t)v[q] - (uint64_t)dig)) >> 8;
      const uint32_t byte = (uint32_t)(dig & 0xFF) << (8 * (q & 3));
      if (q < 4) w0 |= byte; else w1 |= byte;
    }
    uint32_t* dst = (uint32_t*)(gp.xg + ((l * gp.nbp + blk) * gp.Tp + t) * 8 + s);
    dst[2 * dh] = w0;
    dst[2 * dh + 1] = w1;
  }
}

}  // namespace imie_q1
