// Packed Q1_0 linear for gfx950.
//
//   out[t, o] = sum_b ( S[t, o, b] * scale[o, b] ) >> frac        (mod 2^64, floor per 128-block)
//   S[t, o, b] = sum_{i in block b} sign[o, i] * x[t, i] = 2 * pos - total,  pos = sum_{bit=1} x
//
// Reference semantics: bonsai/src/trinote/infer_int/reference_bonsai.py:149-219 (q1_linear_ref) and the C
// producer bonsai/tools/bonsai_q1_kernel.c:85-106. Bit i of byte j of a block is weight 8j+i.
//
// Matvec design (T < 8): int8 MFMA v_mfma_i32_16x16x64_i8 over 16-row tiles and 512-column slabs:
//   * B operand = one bit position s of the weight bytes of 16 output rows as 0/1 bytes
//       B_s dword = (word >> s) & 0x01010101                            (2 VALU per 4 dwords of weights)
//   * A operand = balanced base-256 digits ("limbs") of x from the prepared digit table, rows = (block g of the
//     slab, limb r of a group of four); the 8 bit positions accumulate into one tile, so up to four limbs
//     cost 8 MFMAs per slab and tile.
//   * Slabs whose digits fit one limb (|x| <= 127, e.g. int8 activations) use rows = (block g, bit position
//     mod 4) instead, with mask-only B bytes (0 or 2^s; 0x80 reads as -128): 8 MFMAs, no shifts.
//   * Epilogue per (row, block): pos = sum_r D[r] << 8r, 2*pos - total, * scale, floor shift, add (wrapping
//     int64, as the reference's C producer).
// MFMA int32 accumulation is exact: each D entry is at most 8 * 16 * 128 = 2^14 in magnitude.
// Prefill (T >= 8) uses the tiled GEMM further down.
#include "imie_common.h"
#include <vector>
#include "imie_kernels.h"
#include "imie_q1prep.h"
#include "imie_fixed.h"
#include "imie_silu.h"
#include <string.h>
#include <type_traits>
#include <stdlib.h>

namespace {

using namespace imie_q1;
constexpr int kTileRows = 16;      // output rows per MFMA tile

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
  uint4* signs = nullptr;          // prefill copy: +-1 int8 per weight in MFMA operand order (made on first use)
  int scale64 = 0;
  int64_t maxsc = 0;               // max |scale| (host-side bounds for the GEMM epilogue)
  uint64_t rsum[8] = {};           // [r - 1]: max over rows and over r equal block ranges of sum |scale|
  size_t bytes = 0;
  bool live = false;
};

std::vector<Q1Weight>& registry() {
  static std::vector<Q1Weight> r;
  return r;
}
uint64_t g_resident_bytes = 0;

struct Workspace {
  DevBuf x, out;
  Q1Ws w;
} g_ws;

}  // namespace

// Host repack: natural (N, nb, 16) bits + (N, nb) scales -> tiled layout. Exposed for CPU tests.
static DevBuf g_gemm_ops;   // executed GEMM int8 MFMA ops while profiling (gemm_opcount_kernel)

// Executed int8 MFMA ops of the GEMM launches recorded while profiling (synchronizes); reset != 0 clears.
extern "C" int imie_profile_gemm_ops(unsigned long long* ops, int reset) {
  if (!ops) return IMIE_EARG;
  *ops = 0;
  if (g_gemm_ops.ensure(64)) return IMIE_EARG;
  IMIE_HIP(hipDeviceSynchronize());
  IMIE_HIP(hipMemcpy(ops, g_gemm_ops.p, 8, hipMemcpyDeviceToHost));
  if (reset) IMIE_HIP(hipMemset(g_gemm_ops.p, 0, 8));
  return IMIE_OK;
}

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

// Stand-alone activation prep (see imie_q1prep.h): grid (nslabs, T), one wave per (token, slab); the
// workgroups also clear the zero list for a following K-split matvec.
__global__ __launch_bounds__(64) void q1_prep_kernel(const int64_t* __restrict__ x, int64_t K, Q1PrepOut po,
                                                      Q1Zero zero) {
  const int lane = threadIdx.x;
  const int64_t sl = blockIdx.x, t = blockIdx.y;
  zero_share(zero, t * po.nslabs + sl, (int64_t)gridDim.y * po.nslabs, lane, 64);
  int64_t v[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int64_t pos = prep_pos(lane, sl, q);
    v[q] = (pos < po.nb * 128) ? x[t * K + pos] : 0;
  }
  prep_slab(v, po, t, sl);
}

// ------------------------------------------------------------------------------------------------------
// MFMA matvec / small-T linear.
//   * MFMA rows m = 4*blk + limb (limbs in groups of four): A lane (m, g) holds the balanced digits of limb
//     4*lg + (m & 3) of block g for one bit position s (non-zero iff m >> 2 == g), B lane (n, g) the bit s of
//     block g's 16 weight bytes of output row n as 0/1 bytes ((w >> s) & 0x01010101). The 8 MFMAs of one slab
//     (s = 0..7) accumulate into one tile: lane (g, n) then holds D[r] = sum over block g's 128 weights of
//     digit_r(x) * bit for output row n, and pos = sum_r D[r] << 8 (4 lg + r) (|D| <= 2^14, no cross-lane
//     traffic). Up to four limbs share the same 8 MFMAs.
//   * Each wave streams its own R tiles over a slab range with double-buffered 16 B/lane loads; the digit
//     table of the slab range (up to Lcap limbs) is staged once per workgroup in LDS.
//   * grid.y splits K: with ksplit > 1 the waves add their int64 partials into a zeroed output with 64-bit
//     atomics (integer addition: order-free and exact).
// ------------------------------------------------------------------------------------------------------
// RMSNorm prologue statistics (single row, cols <= kProNormCols): every workgroup reduces the whole row's 128-bit
// sum of squares itself and derives rms = isqrt(ssq // cols + eps) (fixedpoint.py:31-71). Waves whose |x| are all
// below 2^26 sum 52-bit squares in one 64-bit word per lane (one wave reduction); others carry four 32-bit limbs.
// Refusals decided here (block (0, 0) flags the status, every workgroup returns false): ssq of 2^128 or more, or
// rms == 0. The envelope max|n| * max|gain| <= INT64_MAX is checked per element where n is formed.
constexpr int kProNormCols = 4096;
template <int NT>
__device__ inline void pro_norm_row_load(const Q1Pro& p, int64_t (&v)[kProNormCols / NT]) {
#pragma unroll
  for (int k = 0; k < kProNormCols / NT; ++k) {
    const int64_t c = threadIdx.x + NT * k;
    v[k] = p.x[c < p.cols ? c : 0];                   // unconditional loads (no per-element branch); masked at use
  }
}
// v: the row as loaded by pro_norm_row_load (issued before the weights, so the wait for it is not a wait for them)
template <int NT>
__device__ bool pro_norm_stats(const Q1Pro& p, uint64_t* s_red, int64_t* s_x, uint64_t& rms,
                               int64_t (&v)[kProNormCols / NT]) {
  using namespace imie_fx;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int kPer = kProNormCols / NT;
#pragma unroll
  for (int k = 0; k < kPer; ++k) v[k] = tid + NT * k < p.cols ? v[k] : 0;
  uint64_t amax = 0;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const uint64_t a = imie_absu64(v[k]);
    amax = a > amax ? a : amax;
    s_x[tid + NT * k] = v[k];                       // the row on chip for the element phase (after the barrier)
  }
  uint64_t lm[4];
  if (!__any(amax >> 26 ? 1 : 0)) {
    // at most 16 squares below 2^52 per lane, 64 lanes: the wave's sum stays below 2^62
    uint64_t sq = 0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const uint32_t a = (uint32_t)imie_absu64(v[k]);
      sq += (uint64_t)a * a;
    }
    sq = imie_wave_sum_u64_full(sq);
    lm[0] = sq & 0xFFFFFFFFull; lm[1] = sq >> 32; lm[2] = 0; lm[3] = 0;
  } else {
    uint64_t hi = 0, lo = 0;
    int bad = 0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const uint64_t a = imie_absu64(v[k]);
      const u128 sq = (u128)a * a;
      const uint64_t sl = (uint64_t)sq, sh = (uint64_t)(sq >> 64);
      const uint64_t nl = lo + sl;
      const uint64_t cy = nl < lo ? 1 : 0;
      const uint64_t nh = hi + sh;
      bad |= (nh < hi ? 1 : 0) | (nh + cy < nh ? 1 : 0);
      hi = nh + cy;
      lo = nl;
    }
    u128_limbs(hi, lo, bad, lm);
#pragma unroll
    for (int i = 0; i < 4; ++i) lm[i] = imie_wave_sum_u64_full(lm[i]);
  }
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) s_red[wave * 4 + i] = lm[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint64_t t = 0;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) t += s_red[4 * w + i];
    lm[i] = t;
  }
  uint64_t hi, lo;
  int bad;
  u128_fold(lm, hi, lo, bad);
  rms = 0;
  if (!bad) {
    const u128 mean = div_u128_cols(((u128)hi << 64) | lo, (uint32_t)p.cols);
    if (mean <= ~(u128)0 - (u128)(uint64_t)p.eps) rms = isqrt_u128_fast(mean + (u128)(uint64_t)p.eps);
  }
  if (rms == 0 && tid == 0 && blockIdx.x == 0 && blockIdx.y == 0) atomicOr(p.status, IMIE_ERMS);
  return rms != 0;
}

struct Q1Segs {                    // up to kMaxSegs weights (same n_blocks) applied to the same activations
  const uint4* bits[kMaxSegs];
  const void* scale[kMaxSegs];
  int64_t N[kMaxSegs], ntiles[kMaxSegs];
  int64_t* out[kMaxSegs];
  int64_t gbegin[kMaxSegs + 1];    // first tile group of each segment (groups of R tiles)
  int cnt;
};

// PRO != kProNone (one token, R = 1, PF > 0, Lcap = 8): no digit table is read; the workgroup derives its slab
// range's table from the producer's inputs (pro) into LDS -- element values thread-per-element into s_y, then one
// wave per slab turns them into digits, limb counts and block totals -- while its weights are in flight.
// PERS (one token, one weight, one K range, two-slab pipeline): a grid of about two rounds of resident waves; each
// wave walks tile groups gi, gi + W, gi + 2W, ... (W waves in the grid), so the digit staging is paid once per
// workgroup and the pipeline runs on across group boundaries (the next group's first slab is in flight while the
// current group's last slab computes).
template <bool S64, int R, int TT, int PF = 0, int PRO = kProNone, int NT = 256, bool PERS = false>
__global__ __launch_bounds__(NT) void q1_gemv_mfma_kernel(
    Q1Segs sg, const uint4* __restrict__ xq, const int64_t* __restrict__ totals, const int* __restrict__ lslab,
    int64_t nslabs, int64_t nbp, int T, int frac, int64_t spk, int Lcap, int atomic_out, Q1Pro pro) {
  static_assert(PRO == kProNone || (R == 1 && TT == 1 && PF > 0) || (PERS && PRO == kProCopy),
                "prologue: one token, one tile, prefetched range (or the persistent kernel's copy prologue)");
  static_assert(PRO != kProNone || NT == 256, "NT: workgroup size of the prologue variants");
  static_assert(!PERS || (TT == 1 && PF == 0 && (PRO == kProNone || PRO == kProCopy) && NT == 256),
                "persistent: one token, pipelined slabs, at most 8 slabs staged by a copy prologue");
  extern __shared__ __align__(16) unsigned char smem[];
  uint4* stage = (uint4*)smem;                                   // [TT][spk][Lcap][32]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform: keeps the segment scalar
  const int64_t s0 = (int64_t)blockIdx.y * spk;
  const int64_t s1 = min(nslabs, s0 + spk);
  const int64_t nsl = s1 - s0;

  // this wave's tile group -> (segment, first tile)
  const int64_t gi_raw = (int64_t)blockIdx.x * (NT / 64) + wave;
  const bool live = gi_raw < sg.gbegin[sg.cnt];
  const int64_t gi = live ? gi_raw : sg.gbegin[sg.cnt] - 1;
  int seg = 0;
#pragma unroll
  for (int z = 1; z < kMaxSegs; ++z)
    if (z < sg.cnt && gi >= sg.gbegin[z]) seg = z;
  const uint4* __restrict__ bitsT = sg.bits[seg];
  const void* __restrict__ scaleT = sg.scale[seg];
  const int64_t N = sg.N[seg], ntiles = sg.ntiles[seg];
  int64_t* __restrict__ out = sg.out[seg];
  const int64_t tile0 = (gi - sg.gbegin[seg]) * R;
  const int g = lane >> 4;       // block within the slab
  const int n = lane & 15;       // output row within the tile
  const bool aact = (n >> 2) == g;   // A row n (block n / 4) meets this lane's K group g

  uint64_t acc[TT][R];
#pragma unroll
  for (int t = 0; t < TT; ++t)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[t][r] = 0;

  // PF > 0: the wave's whole slab range (at most PF slabs) is requested at once, before the digit staging
  // (decode-sized matvecs: every weight byte in flight in one round); PF == 0: two-slab software pipeline
  constexpr int NB = PF > 2 ? PF : 2;
  uint4 wb[NB][R];
  using ScT = typename std::conditional<S64, int64_t, int32_t>::type;   // widened at use: no wait at the load
  ScT sc[NB][R];
  int Lv[NB][TT];
  int64_t tv[NB][TT];
  auto load_t = [&](int buf, int64_t tb, int64_t sl) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t tl = tb + r < ntiles ? tb + r : tb;
      const int64_t idx = (tl * nslabs + sl) * 64 + lane;
      const v4i wv = __builtin_nontemporal_load(&((const v4i*)bitsT)[idx]);
      wb[buf][r] = uint4{(uint32_t)wv.x, (uint32_t)wv.y, (uint32_t)wv.z, (uint32_t)wv.w};
      sc[buf][r] = __builtin_nontemporal_load(&((const ScT*)scaleT)[idx]);
    }
    // the slab's digit count and block total travel with its weights (one prefetch, one wait)
#pragma unroll
    for (int t = 0; t < TT; ++t)
      if (PRO == kProNone && t < T) {
        Lv[buf][t] = lslab[t * nslabs + sl];
        tv[buf][t] = totals[(int64_t)t * nbp + sl * kSlabBlocks + g];
      }
  };
  auto load = [&](int buf, int64_t sl) { load_t(buf, tile0, sl); };
  // persistent mode: unit u = (group gi_raw + (u / nsl) W, slab s0 + u % nsl)
  const int64_t W = (int64_t)gridDim.x * (NT / 64);
  auto load_unit = [&](int buf, int64_t u) { load_t(buf, (gi_raw + (u / nsl) * W) * R, s0 + u % nsl); };
  // A operands of (token t, limb group lg): the 8 bit positions' digit rows, loaded once and shared by the R
  // tiles; from LDS (staged limbs), the global table (limbs beyond Lcap), or the 8-entry zero slot for lanes
  // whose row is not their block or whose limb is beyond the slab's count
  const uint4* zslot = stage + (int64_t)TT * spk * Lcap * 32;
  // PRO: slab limb counts, block totals and the element values after the zero slot
  int* sL = (int*)(stage + (int64_t)TT * spk * Lcap * 32 + 8);
  int64_t* stot = (int64_t*)(sL + 8);
  // element values (PRO), aliasing the table: each wave reads its slab's values before writing digits over them
  int64_t* s_y = (int64_t*)stage;
  const int arow_l = n & 3;
  auto compute = [&](int buf, int64_t sl) {
    uint64_t pos[TT][R];
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
      for (int r = 0; r < R; ++r) pos[t][r] = 0;
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      if (t >= T) break;
      const int L = PRO != kProNone ? sL[sl - s0] : Lv[buf][t];
      if (L == 1) {
        // one limb (e.g. int8 activations): rows = (block, bit position mod 4) with mask-only B operands
        // (bytes 0 / 2^s, 0x80 reading as -128); 128 * pos = sum d0[q] << (7 - q) + sum d1[q] << (3 - q)
        const int as = n & 3;
        uint4 a0 = uint4{0, 0, 0, 0}, a1 = uint4{0, 0, 0, 0};
        if (Lcap < 4) {
          const uint4* src = xq + ((int64_t)t * kMaxLimbs * nbp + sl * kSlabBlocks + g) * 8 + as;
          a0 = aact ? src[0] : uint4{0, 0, 0, 0};
          a1 = aact ? src[4] : uint4{0, 0, 0, 0};
        }
        v4i areg[8];
        if (Lcap >= 4) {
          // from LDS: each register reads either the lane's digits or the zero slot (a per-lane address select
          // instead of four data selects per register)
          const uint4* src = aact ? stage + ((t * spk + (sl - s0)) * Lcap) * 32 + g * 8 + as : zslot;
#pragma unroll
          for (int sh = 0; sh < 4; ++sh) {
            const uint4* p0 = as == sh ? src : zslot;
            const uint4* p1 = as == sh ? src + (aact ? 4 : 0) : zslot;
            const uint4 u0 = *p0, u1 = *p1;
            areg[sh] = v4i{(int)u0.x, (int)u0.y, (int)u0.z, (int)u0.w};
            areg[sh + 4] = v4i{(int)u1.x, (int)u1.y, (int)u1.z, (int)u1.w};
          }
        } else {
#pragma unroll
          for (int sh = 0; sh < 4; ++sh) {
            areg[sh] = as == sh ? v4i{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w} : v4i{0, 0, 0, 0};
            areg[sh + 4] = as == sh ? v4i{(int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w} : v4i{0, 0, 0, 0};
          }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const uint4 w = wb[buf][r];
          v4i d0 = {0, 0, 0, 0}, d1 = {0, 0, 0, 0};
#pragma unroll
          for (int sh = 0; sh < 8; ++sh) {
            const uint32_t m = 0x01010101u << sh;
            const v4i b = v4i{(int)(w.x & m), (int)(w.y & m), (int)(w.z & m), (int)(w.w & m)};
            if (sh < 4) d0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(areg[sh], b, d0, 0, 0, 0);
            else d1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(areg[sh], b, d1, 0, 0, 0);
          }
          const int p128 = (d0[0] << 7) + (d0[1] << 6) + (d0[2] << 5) + (d0[3] << 4) + (d1[0] << 3) +
                           (d1[1] << 2) + (d1[2] << 1) - d1[3];
          pos[t][r] += (uint64_t)(int64_t)(p128 >> 7);
        }
        continue;
      }
#pragma unroll
      for (int lg = 0; lg < 2; ++lg) {
        if (4 * lg >= L) break;                       // wave-uniform
        const int l = 4 * lg + arow_l;
        const bool on = aact && l < L;
        v4i A[8];
        if (4 * lg + 4 <= Lcap) {
          const uint4* src = on ? stage + ((t * spk + (sl - s0)) * Lcap + l) * 32 + g * 8 : zslot;
#pragma unroll
          for (int sh = 0; sh < 8; ++sh) {
            const uint4 a = src[sh];
            A[sh] = v4i{(int)a.x, (int)a.y, (int)a.z, (int)a.w};
          }
        } else {
          const uint4* src = xq + ((int64_t)t * kMaxLimbs * nbp + (int64_t)l * nbp + sl * kSlabBlocks + g) * 8;
#pragma unroll
          for (int sh = 0; sh < 8; ++sh) {
            const uint4 a = src[sh];
            A[sh] = on ? v4i{(int)a.x, (int)a.y, (int)a.z, (int)a.w} : v4i{0, 0, 0, 0};
          }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const uint4 w = wb[buf][r];
          v4i D0 = {0, 0, 0, 0}, D1 = {0, 0, 0, 0};   // even / odd bit positions: two independent chains
#pragma unroll
          for (int sh = 0; sh < 8; ++sh) {
            uint32_t k = sh;
            asm volatile("" : "+s"(k));   // keep each bit-plane expansion next to its MFMA (no hoisting)
            const v4i b = v4i{(int)((w.x >> k) & 0x01010101u), (int)((w.y >> k) & 0x01010101u),
                              (int)((w.z >> k) & 0x01010101u), (int)((w.w >> k) & 0x01010101u)};
            if (sh & 1) D1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[sh], b, D1, 0, 0, 0);
            else D0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[sh], b, D0, 0, 0, 0);
          }
#pragma unroll
          for (int q = 0; q < 4; ++q) pos[t][r] += (uint64_t)(int64_t)(D0[q] + D1[q]) << (8 * (4 * lg + q));
        }
      }
    }
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      if (t >= T) break;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int64_t tot = PRO != kProNone ? stot[(sl - s0) * 4 + g] : tv[buf][t];
        const uint64_t S = 2u * pos[t][r] - (uint64_t)tot;
        const int64_t prod = (int64_t)(S * (uint64_t)(int64_t)sc[buf][r]);
        acc[t][r] += (uint64_t)imie_floor_shift(prod, frac);
      }
    }
  };

  // this wave's first weight slab (PF: all of its slabs) is requested before the shared digit staging, so the
  // latencies overlap; with a prologue, after the prologue's own inputs: the memory counter is in order, so the
  // prologue's wait for its inputs would otherwise wait for every weight load too
  auto issue_weights = [&]() {
    if (PF > 0) {
#pragma unroll
      for (int j = 0; j < PF; ++j)
        if (live && j < nsl) load(j, s0 + j);
    } else if (live) {
      if (PERS) load_unit(0, 0);
      else load(0, s0);
    }
  };
  if (PRO == kProNone) issue_weights();
  if (PRO != kProNone) {
    __shared__ uint64_t s_red[4 * (NT / 64)];
    // the range's inputs, element c0 + threadIdx.x + NT k for threadIdx.x + NT k < 512 nsl, all requested before any
    // use (a loop over a run-time count would wait for each load in turn)
    constexpr int PSL = PERS ? 8 : PF;                   // slabs a prologue stages (persistent: all, K <= 4096)
    constexpr int KY = PSL * 512 / NT > 1 ? PSL * 512 / NT : 1;
    const int64_t nel = nsl * 512;
    const int64_t c0 = s0 * 512;
    int64_t ya[KY], yb[KY];
#pragma unroll
    for (int k = 0; k < KY; ++k) {
      const int64_t c = c0 + threadIdx.x + NT * k;
      const int64_t cc = (threadIdx.x + NT * k < nel && c < pro.cols) ? c : 0;
      ya[k] = PRO == kProNorm ? 0 : pro.x[cc];
      yb[k] = PRO == kProSiluMul ? pro.x2[cc] : (PRO == kProNorm ? pro.gain[cc] : 0);
    }
    int64_t rowv[kProNormCols / NT];
    if (PRO == kProNorm) pro_norm_row_load<NT>(pro, rowv);
    const uint64_t gmax = PRO == kProNorm ? *pro.gmax : 0;
    issue_weights();
    zero_share(pro.zero, (int64_t)blockIdx.y * gridDim.x + blockIdx.x, (int64_t)gridDim.x * gridDim.y, threadIdx.x,
               NT);
    uint64_t rms = 0;
    if (PRO == kProNorm) {
      __shared__ int64_t s_x[kProNormCols];
      if (!pro_norm_stats<NT>(pro, s_red, s_x, rms, rowv)) return;   // the same verdict in every workgroup
#pragma unroll
      for (int k = 0; k < KY; ++k) {                          // this range's x from the row staged in LDS
        const int64_t c = c0 + threadIdx.x + NT * k;
        ya[k] = s_x[(threadIdx.x + NT * k < nel && c < pro.cols) ? c : 0];
      }
    }
    // kProNorm: n = floor((x << f) / rms) in double precision where exact, then y = (n * gain) >> f. A wave whose
    // elements all meet the bounds of the short path (|x| << f < 2^53, rms < 2^51; |n|, |gain| < 2^31 for the
    // 32 x 32 -> 64 product) runs it branch-free; any other wave takes the general routine per element (with the
    // integer division and its reciprocal). Then the envelope per element: |n| * max|gain| beyond INT64_MAX, or an
    // n outside int64, flags the refusal (the oracle's check over the row's maxima).
    uint64_t nmax = 0;
    bool nfit = true;
    if (PRO == kProNorm) {
      const double rms_d = (double)rms, rinv_d = 1.0 / rms_d;
      // |n| <= |x| * 2^f / rms + 1, so |x| < 2^(30 - f) * rms, i.e. (|x| >> (30 - f)) < rms, keeps |n| below 2^31
      bool fast = pro.frac >= 1 && pro.frac <= 29 && (rms >> 51) == 0;
#pragma unroll
      for (int k = 0; k < KY; ++k) {
        const uint64_t ax = imie_absu64(ya[k]), ag = imie_absu64(yb[k]);
        fast = fast && (ax >> (53 - pro.frac)) == 0 && (ax >> (30 - pro.frac)) < rms && (ag >> 31) == 0;
      }
      if (!__any(fast ? 0 : 1)) {
#pragma unroll
        for (int k = 0; k < KY; ++k) {
          const int64_t c = c0 + threadIdx.x + NT * k;
          if (threadIdx.x + NT * k >= nel) break;
          const int64_t nv = imie_fx::norm_elem_f64_fast(ya[k], pro.frac, rms_d, rinv_d);
          const uint64_t an = imie_absu64(nv);
          nmax = an > nmax ? an : nmax;
          const int64_t prod = (int64_t)(int32_t)nv * (int64_t)(int32_t)yb[k];
          s_y[threadIdx.x + NT * k] = c < pro.cols ? (prod >> pro.frac) : 0;
        }
      } else {
        const uint64_t rinv = imie_fx::recip_u64(rms);
#pragma unroll
        for (int k = 0; k < KY; ++k) {
          const int64_t c = c0 + threadIdx.x + NT * k;
          if (threadIdx.x + NT * k >= nel) break;
          int64_t y = 0;
          if (c < pro.cols) {
            int64_t nv;
            if (!imie_fx::norm_elem_f64(ya[k], pro.frac, rms, rms_d, rinv_d, &nv)) {
              bool f;
              nv = imie_fx::norm_elem(ya[k], pro.frac, rms, rinv, &f);
              nfit = nfit && f;
            }
            const uint64_t an = imie_absu64(nv);
            nmax = an > nmax ? an : nmax;
            y = imie_floor_shift((int64_t)((uint64_t)nv * (uint64_t)yb[k]), pro.frac);
          }
          s_y[threadIdx.x + NT * k] = y;
        }
      }
    } else {
#pragma unroll
      for (int k = 0; k < KY; ++k) {
        const int64_t c = c0 + threadIdx.x + NT * k;
        if (threadIdx.x + NT * k >= nel) break;
        int64_t y = 0;
        if (c < pro.cols)
          y = PRO == kProCopy ? ya[k] : imie_silu::silu_mul_fast(ya[k], yb[k], pro.frac, pro.log2e, pro.dclip);
        s_y[threadIdx.x + NT * k] = y;
      }
    }
    if (PRO == kProNorm && (!nfit || (unsigned __int128)nmax * gmax > (unsigned __int128)INT64_MAX))
      atomicOr(pro.status, IMIE_ERMS);
    if (threadIdx.x < 8) stage[(int64_t)spk * Lcap * 32 + threadIdx.x] = uint4{0, 0, 0, 0};
    __syncthreads();
    for (int64_t j = wave; j < nsl; j += NT / 64) {
      int64_t v[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) v[q] = s_y[j * 512 + prep_pos(lane, 0, q)];
      prep_slab_lds(v, stage + j * Lcap * 32, &sL[j], &stot[j * 4]);
    }
    __syncthreads();
  } else {
  // stage the digit operands of this slab range (the same x for every wave of the workgroup)
  for (int t = 0; t < T; ++t)
    for (int64_t j = 0; j < nsl; ++j) {
      const int L = min(lslab[t * nslabs + s0 + j], Lcap);
      uint4* dst = stage + ((t * spk + j) * Lcap) * 32;
      for (int i = threadIdx.x; i < L * 32; i += blockDim.x) {
        const int l = i >> 5, e = i & 31;
        dst[i] = xq[(((int64_t)t * kMaxLimbs + l) * nbp + (s0 + j) * kSlabBlocks) * 8 + e];
      }
    }
  if (threadIdx.x < 8) stage[(int64_t)TT * spk * Lcap * 32 + threadIdx.x] = uint4{0, 0, 0, 0};
  __syncthreads();
  }

  if (!live) return;

  if (PERS) {
    // a group's row totals are complete after its last slab: reduce the 4 blocks of each row and store them
    auto flush = [&](int64_t tb) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        uint64_t v = acc[0][r];
        v += (uint64_t)__shfl_xor((int64_t)v, 16, 64);
        v += (uint64_t)__shfl_xor((int64_t)v, 32, 64);
        const int64_t row = (tb + r) * kTileRows + n;
        if (g == 0 && tb + r < ntiles && row < N) {
          if (atomic_out == 2) out[row] = (int64_t)((uint64_t)out[row] + v);
          else out[row] = (int64_t)v;
        }
        acc[0][r] = 0;
      }
    };
    const int64_t ngroups = sg.gbegin[1];
    const int64_t nu = ((ngroups - 1 - gi_raw) / W + 1) * nsl;   // live: gi_raw < ngroups
    auto step = [&](int buf, int64_t u) {
      compute(buf, s0 + u % nsl);
      if ((u + 1) % nsl == 0) flush((gi_raw + (u / nsl) * W) * R);
    };
    int64_t u = 0;
    for (; u + 1 < nu; u += 2) {
      load_unit(1, u + 1);
      step(0, u);
      if (u + 2 < nu) load_unit(0, u + 2);
      step(1, u + 1);
    }
    if (u < nu) step(0, u);
    return;
  }
  if (PF > 0) {
#pragma unroll
    for (int j = 0; j < PF; ++j)
      if (j < nsl) compute(j, s0 + j);
  } else {
    // software pipeline over the slab range: prefetch slab j+1 while computing slab j
    int64_t sl = s0;
    for (; sl + 1 < s1; sl += 2) {
      load(1, sl + 1);
      compute(0, sl);
      if (sl + 2 < s1) load(0, sl + 2);
      compute(1, sl + 1);
    }
    if (sl < s1) compute(0, sl);
  }

  // sum the 4 blocks of each row (lane groups g) and write / accumulate row totals
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    if (t >= T) break;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      uint64_t v = acc[t][r];
      v += (uint64_t)__shfl_xor((int64_t)v, 16, 64);
      v += (uint64_t)__shfl_xor((int64_t)v, 32, 64);
      const int64_t row = (tile0 + r) * kTileRows + n;
      if (g == 0 && tile0 + r < ntiles && row < N) {
        if (atomic_out == 1) atomicAdd((unsigned long long*)&out[(int64_t)t * N + row], (unsigned long long)v);
        else if (atomic_out == 2) out[(int64_t)t * N + row] = (int64_t)((uint64_t)out[(int64_t)t * N + row] + v);
        else out[(int64_t)t * N + row] = (int64_t)v;
      }
    }
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
// GEMM path (T >= kGemmMinT tokens; prefill): int8 MFMA with TOKENS in the MFMA M dimension.
//   * K step = 64 positions of one block: the 4 MFMA K-groups are the shifts s = 4h + g (h = half of the
//     block), 16 positions each. B lane (output n, group g) = (block bits dword d >> s) & 0x01010101: bytes
//     {0, 1} for positions 32d + 8c + s, the order the digit table uses for A (token m, group g).
//   * Per block and limb l: D = sum over the block of bit * digit_l (2 MFMAs); pos = sum_l D_l << 8l; then the
//     exact per-(token, output, block) epilogue S = 2 pos - total, += (S * scale) >> frac (wrapping int64).
//   * Workgroup tile 64 tokens x 128 outputs, 2 x 2 waves of 32 x 64 (2 x 4 MFMA tiles). Workgroups of one token
//     tile are mapped to one XCD (blockIdx % 8) so that XCD's L2 keeps the tile's digits.
//   * Two kernels split the blocks by the workgroup's limb count on the block's slab (max over its 64 tokens):
//     "narrow" (<= 3 limbs, |x| <= 2^23: pos and S exact in int32; digits staged through double-buffered LDS,
//     next block's loads in flight during the MFMAs) and "wide" (> 3 limbs: int64 pos / S, per-token limb
//     masking), which adds its blocks into the narrow kernel's output. Every block is taken by exactly one.
// Digit table layout for the GEMM: xg[l][block][Tp][s] (uint4), totals tg[block][Tp], limbs lt[t][slab]; the
// prep writes zero digits for limbs L_t <= l < 3 so narrow tiles need no per-token masking.
// ------------------------------------------------------------------------------------------------------
constexpr int kNarrowLimbs = kGemmNarrowLimbs;
constexpr int kGemmMaxSlabs = 64;  // K <= 32768

// one wave per (token, slab), four slabs per workgroup
__global__ __launch_bounds__(256) void q1_prep_gemm_kernel(const int64_t* __restrict__ x, int64_t K, GemmPrepOut gp) {
  const int lane = threadIdx.x & 63;
  const int64_t sl = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6), t = blockIdx.y;
  if (sl >= gp.nslabs) return;                        // whole wave
  int64_t v[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int64_t pos = prep_pos(lane, sl, q);
    v[q] = (pos < gp.nb * 128) ? x[t * K + pos] : 0;
  }
  prep_gemm_slab(v, gp, t, sl);
}

struct GemmArgs {
  const uint4* signs;              // q1_gemm_pm_kernel: [o][block][8] uint4 of +-1 bytes
  const uint4* bitsT;
  const void* scaleT;
  const uint4* xg;
  const int64_t* tg;
  const int* lt;
  int64_t T, Tp, N, nb, nbp, nslabs, ntt, nto;
  int64_t ntiles16;                // 16 * tiles: rows of the tiled scale layout
  int frac, accumulate;
  int kfold;                       // > 0: high-dword epilogue (narrow kernel), folded every kfold blocks
  int rlen;                        // q1_gemm_ps_kernel<.., 2>: first block of the second int32 partial sum
  int ksplit;                      // narrow kernel: blocks split over gridDim.y ranges, outputs added atomically
  int64_t* out;
  int* wide_any;                   // set by q1_gemm_pm_kernel per 64-token tile: some slab needs > 3 limbs (the
                                   // wide kernel's workgroups of other tiles end at once); nullptr: not known
};

// block bits of this lane's NT outputs (every K-group reads the same 16 bytes) and their scales
template <bool S64, int NT>
__device__ inline void gemm_load_b(const GemmArgs& a, int64_t o0, int m, int64_t b, uint4 w[NT], int64_t sc[NT]) {
  const int64_t sl = b >> 2;
#pragma unroll
  for (int jj = 0; jj < NT; ++jj) {
    const int64_t o = o0 + 16 * jj + m;
    w[jj] = uint4{0, 0, 0, 0};
    sc[jj] = 0;
    if (o < a.N) {
      const int64_t idx = ((o >> 4) * a.nslabs + sl) * 64 + 16 * (b & 3) + m;
      const v4i wv = *((const v4i*)a.bitsT + idx);
      w[jj] = uint4{(uint32_t)wv.x, (uint32_t)wv.y, (uint32_t)wv.z, (uint32_t)wv.w};
      sc[jj] = S64 ? ((const int64_t*)a.scaleT)[idx] : (int64_t)((const int32_t*)a.scaleT)[idx];
    }
  }
}

__device__ inline v4i expand_bits(const uint4 w, int sh) {
  return v4i{(int)((w.x >> sh) & 0x01010101u), (int)((w.y >> sh) & 0x01010101u), (int)((w.z >> sh) & 0x01010101u),
             (int)((w.w >> sh) & 0x01010101u)};
}

__device__ inline void gemm_tile(const GemmArgs& a, int wave, int64_t& t0w, int64_t& o0w, int64_t& t0g, bool& live,
                                 int64_t wg = -1) {
  if (wg < 0) wg = blockIdx.x;
  int64_t tt, ot;
  if (a.ntt >= 8) {
    // >= 8 token tiles: each XCD (blockIdx % 8) walks whole token tiles, so its L2 keeps those tiles' digits
    const int64_t xcd = wg & 7, j = wg >> 3, tpx = (a.ntt + 7) / 8;
    tt = xcd + 8 * (j / a.nto);
    ot = j % a.nto;
    live = tt < a.ntt && (j / a.nto) < tpx;
  } else {
    // few token tiles (batched decode): spread the output tiles over every XCD
    tt = wg / a.nto;
    ot = wg % a.nto;
    live = tt < a.ntt;
  }
  t0g = tt * 64;
  t0w = t0g + (wave >> 1) * 32;
  o0w = ot * 128 + (wave & 1) * 64;
}

// per-slab limb maximum over the workgroup's 64 tokens into s_lw
__device__ inline void gemm_slab_limbs(const GemmArgs& a, int64_t t0g, int* s_lw) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t t = t0g + lane;
  for (int64_t sl = wave; sl < a.nslabs; sl += 4) {
    int L = t < a.T ? a.lt[t * a.nslabs + sl] : 0;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) { const int w2 = __shfl_xor(L, o, 64); L = w2 > L ? w2 : L; }
    if (lane == 0) s_lw[sl] = L;
  }
  __syncthreads();
}

// NBUF = 2: double-buffered LDS operands, one barrier per block (62 KB of LDS: 2 workgroups per CU); NBUF = 1:
// one buffer and two barriers per block (31 KB: more workgroups per CU to overlap one another's waits)
// FE (int32 scales with |scale| < 2^(frac-1), frac <= 31): per element and block, p = S * (scale << (32 - frac))
// + H with H = A * 2^32, so the high dword of p is A + floor(S * scale / 2^frac) exactly; clearing p's low dword
// gives the next H (one v_mad_i64_i32 and one clear). A is folded into the int64 sum every kfold blocks, chosen
// on the host so |A| + max|q| stays below 2^31 (|S| < 2^30 on <= 3 limbs).
template <bool S64, int NBUF, bool FE>
__global__ __launch_bounds__(256) void q1_gemm_narrow_kernel(GemmArgs a) {
  constexpr int MT = 2, NT = 4;
  __shared__ int s_lw[kGemmMaxSlabs];
  // [buffer][limb][token][shift], tokens padded to 9 x 16 B: the 16 lanes of a quarter-wave read tokens
  // m = 0..15 at a 144 B stride, which covers all 64 LDS banks once (a 128 B stride would hit 2 of them)
  __shared__ v4i sA[NBUF][kNarrowLimbs][64][9];
  __shared__ uint4 sB[NBUF][128];                     // block bits of the 128 outputs
  typedef typename std::conditional<S64, int64_t, int32_t>::type ST;
  __shared__ ST sS[NBUF][128];                        // their scales (int32 unless the weight keeps int64)
  __shared__ int64_t sT[NBUF][64];                    // block totals of the 64 tokens
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int64_t t0, o0, t0g;
  bool live;
  gemm_tile(a, wave, t0, o0, t0g, live);
  if (!live) return;
  gemm_slab_limbs(a, t0g, s_lw);
  const int m = lane & 15, g = lane >> 4;
  const int tb = (wave >> 1) * 32;                    // this wave's first token within the workgroup tile
  const int ob = (wave & 1) * 64;                     // this wave's first output within the workgroup tile
  const int64_t o0g = o0 - ob;
  // cooperative stage: thread -> token tid >> 2, shifts 2 (tid & 3) + {0, 1} of every limb; threads < 128 also
  // one output's bits + scale, threads < 64 one token's total
  const int st_tok = tid >> 2, st_s = 2 * (tid & 3);
  v4i pa[kNarrowLimbs][2];
  uint4 pb = uint4{0, 0, 0, 0};
  ST ps = 0;
  int64_t pt = 0;
  auto stage_load = [&](int64_t b) {
    const int lwb = s_lw[b >> 2];
#pragma unroll
    for (int l = 0; l < kNarrowLimbs; ++l)
#pragma unroll
      for (int u = 0; u < 2; ++u)
        pa[l][u] = (lwb <= kNarrowLimbs && l < lwb)
                       ? *((const v4i*)a.xg + (uint32_t)((((uint32_t)l * (uint32_t)a.nbp + (uint32_t)b) *
                                                             (uint32_t)a.Tp + (uint32_t)(t0g + st_tok)) * 8u +
                                                            (uint32_t)(st_s + u)))
                       : v4i{0, 0, 0, 0};
    if (tid < 128) {
      const int64_t o = o0g + tid;
      pb = uint4{0, 0, 0, 0};
      ps = 0;
      if (o < a.N) {
        const int64_t idx = ((o >> 4) * a.nslabs + (b >> 2)) * 64 + 16 * (b & 3) + (o & 15);
        const v4i wv = *((const v4i*)a.bitsT + idx);
        pb = uint4{(uint32_t)wv.x, (uint32_t)wv.y, (uint32_t)wv.z, (uint32_t)wv.w};
        ps = ((const ST*)a.scaleT)[idx];
      }
    }
    if (tid < 64) pt = t0g + tid < a.T ? a.tg[b * a.Tp + t0g + tid] : 0;
  };
  auto stage_store = [&](int buf) {
#pragma unroll
    for (int l = 0; l < kNarrowLimbs; ++l)
#pragma unroll
      for (int u = 0; u < 2; ++u) sA[buf][l][st_tok][st_s + u] = pa[l][u];
    if (tid < 128) { sB[buf][tid] = pb; sS[buf][tid] = ps; }
    if (tid < 64) sT[buf][tid] = 0 - pt;             // negated block totals: S = (D << 1) + sT, one v_lshl_add
  };
  int64_t acc[MT][NT][4];
  int64_t accH[FE ? MT : 1][FE ? NT : 1][4];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int jj = 0; jj < NT; ++jj)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        acc[i][jj][r] = 0;
        if (FE) accH[FE ? i : 0][FE ? jj : 0][r] = 0;
      }
  int fcount = 0;
  auto fold = [&]() {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int jj = 0; jj < NT; ++jj)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          acc[i][jj][r] = (int64_t)((uint64_t)acc[i][jj][r] + (uint64_t)(accH[FE ? i : 0][FE ? jj : 0][r] >> 32));
          accH[FE ? i : 0][FE ? jj : 0][r] = 0;
        }
  };
  // this workgroup's block range (the whole K unless the launch splits it for a small token count)
  const int64_t b0 = (int64_t)blockIdx.y * a.nb / a.ksplit, b1 = ((int64_t)blockIdx.y + 1) * a.nb / a.ksplit;
  if (b0 >= b1) return;
  stage_load(b0);
  stage_store(NBUF == 2 ? (int)(b0 & 1) : 0);
  __syncthreads();
  for (int64_t b = b0; b < b1; ++b) {
    const int buf = NBUF == 2 ? (int)(b & 1) : 0;
    const bool more = b + 1 < b1;
    if (more) stage_load(b + 1);                      // next block's operands in flight during this block
    const int lw = s_lw[b >> 2];
    if (lw <= kNarrowLimbs) {
      v4i bx[NT][2];
#pragma unroll
      for (int jj = 0; jj < NT; ++jj) {
        const uint4 w = sB[buf][ob + 16 * jj + m];
        bx[jj][0] = expand_bits(w, g);
        bx[jj][1] = expand_bits(w, 4 + g);
      }
      // pos = sum_l D_l 256^l by Horner from the top limb: acc = (acc << 8) + MFMA(limb l); one shift per
      // element per limb, exact in int32 (every partial is bounded by |pos| <= 2^30)
      v4i D[MT][NT];
      {
        // top limb from a zero accumulator (no shift), then Horner down to limb 0
        const int l = lw - 1;
        v4i av[MT][2];
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int h = 0; h < 2; ++h) av[i][h] = sA[buf][l][tb + 16 * i + m][4 * h + g];
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int jj = 0; jj < NT; ++jj) {
            const v4i c = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i][0], bx[jj][0], v4i{0, 0, 0, 0}, 0, 0, 0);
            D[i][jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i][1], bx[jj][1], c, 0, 0, 0);
          }
      }
      for (int l = lw - 2; l >= 0; --l) {
        v4i av[MT][2];
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int h = 0; h < 2; ++h) av[i][h] = sA[buf][l][tb + 16 * i + m][4 * h + g];
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int jj = 0; jj < NT; ++jj) {
            v4i c = D[i][jj];
            c = v4i{(int)((uint32_t)c[0] << 8), (int)((uint32_t)c[1] << 8), (int)((uint32_t)c[2] << 8),
                    (int)((uint32_t)c[3] << 8)};
            c = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i][0], bx[jj][0], c, 0, 0, 0);
            D[i][jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i][1], bx[jj][1], c, 0, 0, 0);
          }
      }
      if (FE) {
        int32_t scp[NT];
#pragma unroll
        for (int jj = 0; jj < NT; ++jj) scp[jj] = (int32_t)((uint32_t)sS[buf][ob + 16 * jj + m] << (32 - a.frac));
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint32_t ntot = (uint32_t)sT[buf][tb + 16 * i + 4 * g + r];
#pragma unroll
            for (int jj = 0; jj < NT; ++jj) {
              const int32_t S = (int32_t)(((uint32_t)D[i][jj][r] << 1) + ntot);
              const int64_t p = (int64_t)S * (int64_t)scp[jj] + accH[FE ? i : 0][FE ? jj : 0][r];
              accH[FE ? i : 0][FE ? jj : 0][r] = p & (int64_t)0xFFFFFFFF00000000ll;
            }
          }
        if (++fcount == a.kfold) { fold(); fcount = 0; }
      } else {
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint32_t ntot = (uint32_t)sT[buf][tb + 16 * i + 4 * g + r];
#pragma unroll
            for (int jj = 0; jj < NT; ++jj) {
              const int32_t S = (int32_t)(((uint32_t)D[i][jj][r] << 1) + ntot);
              const ST sc = sS[buf][ob + 16 * jj + m];
              const int64_t prod = S64 ? (int64_t)((uint64_t)(int64_t)S * (uint64_t)(int64_t)sc)
                                       : (int64_t)S * (int64_t)(int32_t)sc;   // one v_mad_i64_i32
              acc[i][jj][r] = (int64_t)((uint64_t)acc[i][jj][r] + (uint64_t)imie_floor_shift(prod, a.frac));
            }
          }
      }
    }
    if (NBUF == 2) {
      if (more) stage_store(buf ^ 1);
      __syncthreads();
    } else {
      __syncthreads();                                // every wave is done with this block's operands
      if (more) stage_store(0);
      __syncthreads();
    }
  }
  if (FE) fold();
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int jj = 0; jj < NT; ++jj) {
      const int64_t o = o0 + 16 * jj + m;
      if (o >= a.N) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t t = t0 + 16 * i + 4 * g + r;
        if (t >= a.T) continue;
        int64_t* dst = a.out + t * a.N + o;
        if (a.ksplit > 1)                             // sums mod 2^64 commute: the result is order independent
          atomicAdd((unsigned long long*)dst, (unsigned long long)acc[i][jj][r]);
        else
          *dst = a.accumulate ? (int64_t)((uint64_t)*dst + (uint64_t)acc[i][jj][r]) : acc[i][jj][r];
      }
    }
}

// ------------------------------------------------------------------------------------------------------
// Prefill GEMM over a +-1 sign copy of the weight (T >= kPmMinT tokens, int32 scales with the high-dword
// epilogue). With the 288 GB of HBM a second copy of 1 byte per weight is affordable for prefill, and it takes
// the per-block work off the VALU: no bit expansion, and S = sum(sign * x) comes straight out of the MFMA (no
// 2 * pos - total correction). Operands are staged with buffer loads at per-thread offsets fixed for the whole
// loop and a uniform per-block offset, so the loop carries no address arithmetic.
// Sign layout: signs[(o * nb + b) * 8 + c] (uint4): byte k of chunk c is +1 when bit c of byte k of the block's
// 16 bit-bytes is set, else -1; chunk c = 4 h + g is the B operand of lane group g in K half h, the same chunk
// index the digit table uses for the A operand, so both sides of the MFMA see the same K order.
// ------------------------------------------------------------------------------------------------------
constexpr int64_t kPmMinT = 256;

__global__ __launch_bounds__(256) void q1_signs_kernel(const uint4* __restrict__ bitsT, int64_t N, int64_t nb,
                                                       int64_t nslabs, uint4* __restrict__ signs) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= N * nb) return;
  const int64_t o = i / nb, b = i - (i / nb) * nb;
  const uint4 w = bitsT[((o >> 4) * nslabs + (b >> 2)) * 64 + 16 * (b & 3) + (o & 15)];
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    uint32_t v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = 0xFFFFFFFFu ^ (((ww[q] >> c) & 0x01010101u) * 0xFEu);   // 1 -> 0x01, 0 -> 0xFF
    signs[i * 8 + c] = uint4{v[0], v[1], v[2], v[3]};
  }
}

__device__ inline __amdgpu_buffer_rsrc_t pm_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// 16 B per lane from global straight into LDS at lds + 16 * lane (buffer_load_dwordx4 ... lds; M0 = lds)
__device__ inline void pm_dma(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

// Tile 128 tokens x 128 outputs, 8 waves (4 token quarters x 2 output halves, each 32 x 64 as in the narrow
// kernel). Operands of block b + 1 are copied from global memory straight into the other half of a
// double-buffered LDS ring while block b computes (no staging registers, one barrier per block). Rows (tokens,
// outputs) are 8 chunks of 16 B with chunk c stored at slot c ^ ((row >> 1) & 7): the 16 lanes that read one
// chunk of 16 consecutive rows hit 16 distinct bank groups, and since every wave's rows start at a multiple of
// 16 the swizzle term depends on the lane only, so each operand read is one ds_read_b128 at a constant offset.
constexpr int kPmTok = 128;

// ACC: the launch adds into its outputs (a residual); the epilogue then reads each 16 x 16 tile's 4 outputs before
// writing them (a read after a store the compiler cannot tell apart waits for that store, one round trip per
// element). Without ACC the epilogue only stores, and the rest of the kernel compiles as before.
template <bool ACC>
__global__ __launch_bounds__(512) void q1_gemm_pm_kernel(GemmArgs a, uint32_t xg_bytes, uint32_t sg_bytes,
                                                         uint32_t sc_bytes) {
  constexpr int MT = 2, NT = 4;
  // per-slab limb maxima of the two 64-token halves: a half whose slab needs more than 3 limbs leaves that slab to
  // q1_gemm_wide_kernel, which decides on the same 64-token tiles
  __shared__ int s_lw[2][kGemmMaxSlabs];
  // the two halves of the ring are separate arrays: reads of one half then carry no wait on copies into the other
  __shared__ v4i sA0[kNarrowLimbs][kPmTok * 8], sA1[kNarrowLimbs][kPmTok * 8];   // 2 x 48 KB
  __shared__ v4i sB0[128 * 8], sB1[128 * 8];                                      // 2 x 16 KB
  __shared__ int32_t sS0[128], sS1[128];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t ntt = (a.T + kPmTok - 1) / kPmTok, wg = blockIdx.x;
  int64_t tt, ot;
  bool live;
  if (ntt >= 8) {                                     // each XCD walks whole token tiles (their digits stay in L2)
    const int64_t xcd = wg & 7, j = wg >> 3, tpx = (ntt + 7) / 8;
    tt = xcd + 8 * (j / a.nto);
    ot = j % a.nto;
    live = tt < ntt && (j / a.nto) < tpx;
  } else {
    tt = wg / a.nto;
    ot = wg % a.nto;
    live = tt < ntt;
  }
  if (!live) return;
  const int64_t t0g = tt * kPmTok, o0g = ot * 128;
  for (int64_t q = wave; q < 2 * a.nslabs; q += 8) {  // (half, slab) limb maxima over 64 tokens each
    const int hh = (int)(q & 1);
    const int64_t sl = q >> 1, t = t0g + 64 * hh + lane;
    int L = t < a.T ? a.lt[t * a.nslabs + sl] : 0;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) { const int w2 = __shfl_xor(L, o, 64); L = w2 > L ? w2 : L; }
    if (lane == 0) s_lw[hh][sl] = L;
  }
  const int m = lane & 15, g = lane >> 4;
  const int tb = (wave >> 1) * 32, ob = (wave & 1) * 64;
  const __amdgpu_buffer_rsrc_t rA = pm_rsrc(a.xg, xg_bytes), rB = pm_rsrc(a.signs, sg_bytes),
                               rS = pm_rsrc(a.scaleT, sc_bytes);
  // DMA roles: A = 3 limbs x 16 row groups of 8 tokens = 48 copies of 1 KB, 6 per wave; B = 16 row groups of 8
  // outputs, 2 per wave. Lane L of a copy fills slot L & 7 of row (L >> 3) of the group.
  const int drow = lane >> 3, dslot = lane & 7;
  uint32_t voA[6], voB[2];
#pragma unroll
  for (int q = 0; q < 6; ++q) {
    const int rg = (wave * 6 + q) & 15, t = rg * 8 + drow;
    voA[q] = (uint32_t)(t0g + t) * 128u + (uint32_t)(dslot ^ ((t >> 1) & 7)) * 16u;
  }
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int r = (wave * 2 + q) * 8 + drow;
    const int64_t o = o0g + r < a.N ? o0g + r : a.N - 1;                     // clamp: padding columns unused
    voB[q] = (uint32_t)o * (uint32_t)a.nb * 128u + (uint32_t)(dslot ^ ((r >> 1) & 7)) * 16u;
  }
  const int64_t so_ = o0g + (tid & 127) < a.ntiles16 ? o0g + (tid & 127) : a.ntiles16 - 1;
  const uint32_t voS = (uint32_t)(((so_ >> 4) * a.nslabs * 64 + (so_ & 15)) * 4);
  const uint32_t limb_stride = (uint32_t)a.nbp * (uint32_t)a.Tp * 128u, blk_stride = (uint32_t)a.Tp * 128u;
  auto issue = [&](int64_t b, v4i (*dA)[kPmTok * 8], v4i* dB) {
    const int l0 = s_lw[0][b >> 2], l1 = s_lw[1][b >> 2];
    const int a0 = l0 <= kNarrowLimbs ? l0 : 0, a1 = l1 <= kNarrowLimbs ? l1 : 0;
    const int lwb = a0 > a1 ? a0 : a1;                // limbs needed by the halves this kernel computes
#pragma unroll
    for (int q = 0; q < 6; ++q) {
      const int qi = wave * 6 + q, l = qi >> 4, rg = qi & 15;
      if (l < lwb)
        pm_dma(rA, &dA[l][rg * 64], voA[q], (uint32_t)l * limb_stride + (uint32_t)b * blk_stride);
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) pm_dma(rB, &dB[(wave * 2 + q) * 64], voB[q], (uint32_t)b * 128u);
  };
  auto load_scale = [&](int64_t b) -> int32_t {
    return (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rS, (int)voS, (int)((((b >> 2) * 64) + 16 * (b & 3)) * 4), 0);
  };
  int64_t acc[MT][NT][4];
  int32_t part[MT][NT][4];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int jj = 0; jj < NT; ++jj)
#pragma unroll
      for (int r = 0; r < 4; ++r) { acc[i][jj][r] = 0; part[i][jj][r] = 0; }
  // per-lane physical chunk of K half h (the swizzle term (row >> 1) & 7 is (m >> 1) & 7 for every read row)
  const int pc0 = (0 + g) ^ ((m >> 1) & 7), pc1 = (4 + g) ^ ((m >> 1) & 7);
  __syncthreads();                                    // s_lw
  if (ot == 0 && tid < 2 && t0g + 64 * tid < a.T) {   // one workgroup per token tile records its halves' flags
    int any = 0;
    for (int64_t sl = 0; sl < a.nslabs; ++sl) any |= s_lw[tid][sl] > kNarrowLimbs ? 1 : 0;
    a.wide_any[tt * 2 + tid] = any;
  }
  issue(0, sA0, sB0);
  if (tid < 128) sS0[tid] = load_scale(0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  int fcount = 0;
  // one block from (cA, cB, cS) while block b + 1 is copied into (nA, nB, nS)
  auto step = [&](int64_t b, const v4i (*cA)[kPmTok * 8], const v4i* cB, const int32_t* cS, v4i (*nA)[kPmTok * 8],
                  v4i* nB, int32_t* nS) {
    const bool more = b + 1 < a.nb;
    int32_t ps = 0;
    if (more) {
      issue(b + 1, nA, nB);
      if (tid < 128) ps = load_scale(b + 1);
    }
    const int lw = s_lw[wave >> 2][b >> 2];             // this wave's 64-token half
    if (lw <= kNarrowLimbs) {
      v4i bx[NT][2];
#pragma unroll
      for (int jj = 0; jj < NT; ++jj) {
        const int r = ob + 16 * jj + m;
        bx[jj][0] = cB[r * 8 + pc0];
        bx[jj][1] = cB[r * 8 + pc1];
      }
      int32_t scp[NT];
#pragma unroll
      for (int jj = 0; jj < NT; ++jj) scp[jj] = (int32_t)((uint32_t)cS[ob + 16 * jj + m] << (32 - a.frac));
      if (lw == kNarrowLimbs) {
        // the common case, chain-major: every (token tile, output tile) chain runs its three limbs (and the
        // shifts between them) on its own, so one chain's VALU work overlaps the other chains' MFMAs
        v4i av[kNarrowLimbs][MT][2];
#pragma unroll
        for (int l = 0; l < kNarrowLimbs; ++l)
#pragma unroll
          for (int i = 0; i < MT; ++i) {
            const int r = tb + 16 * i + m;
            av[l][i][0] = cA[l][r * 8 + pc0];
            av[l][i][1] = cA[l][r * 8 + pc1];
          }
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int jj = 0; jj < NT; ++jj) {
            v4i c = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[2][i][0], bx[jj][0], v4i{0, 0, 0, 0}, 0, 0, 0);
            c = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[2][i][1], bx[jj][1], c, 0, 0, 0);
#pragma unroll
            for (int l = 1; l >= 0; --l) {
              c = v4i{(int)((uint32_t)c[0] << 8), (int)((uint32_t)c[1] << 8), (int)((uint32_t)c[2] << 8),
                      (int)((uint32_t)c[3] << 8)};
              c = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[l][i][0], bx[jj][0], c, 0, 0, 0);
              c = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[l][i][1], bx[jj][1], c, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)   // high dword of S * (scale << (32 - frac)) = floor(S * scale / 2^frac)
              part[i][jj][r] = (int32_t)((uint32_t)part[i][jj][r] + (uint32_t)__mulhi(c[r], scp[jj]));
          }
      } else {
        v4i D[MT][NT];
        {
          const int l = lw - 1;
          v4i av[MT][2];
#pragma unroll
          for (int i = 0; i < MT; ++i) {
            const int r = tb + 16 * i + m;
            av[i][0] = cA[l][r * 8 + pc0];
            av[i][1] = cA[l][r * 8 + pc1];
          }
#pragma unroll
          for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int jj = 0; jj < NT; ++jj) {
              const v4i c = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i][0], bx[jj][0], v4i{0, 0, 0, 0}, 0, 0, 0);
              D[i][jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i][1], bx[jj][1], c, 0, 0, 0);
            }
        }
        for (int l = lw - 2; l >= 0; --l) {
          v4i av[MT][2];
#pragma unroll
          for (int i = 0; i < MT; ++i) {
            const int r = tb + 16 * i + m;
            av[i][0] = cA[l][r * 8 + pc0];
            av[i][1] = cA[l][r * 8 + pc1];
          }
#pragma unroll
          for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int jj = 0; jj < NT; ++jj) {
              v4i c = D[i][jj];
              c = v4i{(int)((uint32_t)c[0] << 8), (int)((uint32_t)c[1] << 8), (int)((uint32_t)c[2] << 8),
                      (int)((uint32_t)c[3] << 8)};
              c = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i][0], bx[jj][0], c, 0, 0, 0);
              D[i][jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i][1], bx[jj][1], c, 0, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int jj = 0; jj < NT; ++jj)
              part[i][jj][r] = (int32_t)((uint32_t)part[i][jj][r] + (uint32_t)__mulhi(D[i][jj][r], scp[jj]));
      }
      if (++fcount == a.kfold) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int jj = 0; jj < NT; ++jj)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              acc[i][jj][r] = (int64_t)((uint64_t)acc[i][jj][r] + (uint64_t)(int64_t)part[i][jj][r]);
              part[i][jj][r] = 0;
            }
        fcount = 0;
      }
    }
    if (more && tid < 128) nS[tid] = ps;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's copies of block b + 1 have landed
    __syncthreads();                                  // ... and every wave's; block b's half is free again
  };
  for (int64_t b = 0; b < a.nb; b += 2) {
    step(b, sA0, sB0, sS0, sA1, sB1, sS1);
    if (b + 1 < a.nb) step(b + 1, sA1, sB1, sS1, sA0, sB0, sS0);
  }
  const int64_t t0 = t0g + tb, o0 = o0g + ob;
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int jj = 0; jj < NT; ++jj) {
      const int64_t o = o0 + 16 * jj + m;
      if (o >= a.N) continue;
      int64_t prev[4] = {0, 0, 0, 0};
      if constexpr (ACC) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t t = t0 + 16 * i + 4 * g + r;
          prev[r] = t < a.T ? a.out[t * a.N + o] : 0;
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t t = t0 + 16 * i + 4 * g + r;
        if (t >= a.T) continue;
        const int64_t v = (int64_t)((uint64_t)acc[i][jj][r] + (uint64_t)(int64_t)part[i][jj][r]);
        a.out[t * a.N + o] = (int64_t)((uint64_t)prev[r] + (uint64_t)v);
      }
    }
}

// blocks whose slab needs more than kNarrowLimbs limbs on the tile's tokens; adds into out
// One wave's 16 MT x 16 NT sub-tile at (t0, o0): the blocks whose slab needs more than kNarrowLimbs limbs over
// the wave's 64-token tile (s_lw[slab] from gemm_slab_limbs), exact in int64 with any limb count, added into out
// (ATOMIC: with 64-bit atomic adds, for callers that stored the narrow blocks' sums to the same outputs).
template <bool S64, int MT, int NT, bool ATOMIC>
__device__ inline void gemm_wide_wave(const GemmArgs& a, int64_t t0, int64_t o0, const int* s_lw, int64_t bbeg = 0,
                                      int64_t bend = -1) {
  const int lane = threadIdx.x & 63;
  const int m = lane & 15, g = lane >> 4;
  int64_t ta[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) ta[i] = t0 + 16 * i + m;
  int64_t acc[MT][NT][4];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int jj = 0; jj < NT; ++jj)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][jj][r] = 0;
  if (bend < 0) bend = a.nb;
  for (int64_t b = bbeg; b < bend; ++b) {
    const int lwg = s_lw[b >> 2];
    if (lwg <= kNarrowLimbs) continue;
    const int64_t sl = b >> 2;
    int la[MT];
    int lw = 0;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      la[i] = ta[i] < a.T ? a.lt[ta[i] * a.nslabs + sl] : 0;
      lw = la[i] > lw ? la[i] : lw;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) { const int w2 = __shfl_xor(lw, o, 64); lw = w2 > lw ? w2 : lw; }
    lw = __builtin_amdgcn_readfirstlane(lw);
    uint4 w[NT];
    int64_t sc[NT];
    gemm_load_b<S64, NT>(a, o0, m, b, w, sc);
    v4i bx[NT][2];
#pragma unroll
    for (int jj = 0; jj < NT; ++jj) {
      bx[jj][0] = expand_bits(w[jj], g);
      bx[jj][1] = expand_bits(w[jj], 4 + g);
    }
    uint64_t pos[MT][NT][4];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int jj = 0; jj < NT; ++jj)
#pragma unroll
        for (int r = 0; r < 4; ++r) pos[i][jj][r] = 0;
    for (int l = 0; l < lw; ++l) {
      v4i av[MT][2];
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          av[i][h] = (l < la[i]) ? *((const v4i*)a.xg + ((l * a.nbp + b) * a.Tp + ta[i]) * 8 + 4 * h + g)
                                 : v4i{0, 0, 0, 0};
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int jj = 0; jj < NT; ++jj) {
          v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i][0], bx[jj][0], v4i{0, 0, 0, 0}, 0, 0, 0);
          d = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i][1], bx[jj][1], d, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r) pos[i][jj][r] += (uint64_t)(int64_t)d[r] << (8 * l);
        }
    }
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t t = t0 + 16 * i + 4 * g + r;
        const uint64_t tot = t < a.T ? (uint64_t)a.tg[b * a.Tp + t] : 0;
#pragma unroll
        for (int jj = 0; jj < NT; ++jj) {
          const uint64_t S = 2u * pos[i][jj][r] - tot;
          const int64_t prod = (int64_t)(S * (uint64_t)sc[jj]);
          acc[i][jj][r] = (int64_t)((uint64_t)acc[i][jj][r] + (uint64_t)imie_floor_shift(prod, a.frac));
        }
      }
  }
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int jj = 0; jj < NT; ++jj) {
      const int64_t o = o0 + 16 * jj + m;
      if (o >= a.N) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t t = t0 + 16 * i + 4 * g + r;
        if (t >= a.T) continue;
        int64_t* dst = a.out + t * a.N + o;
        if (ATOMIC) atomicAdd((unsigned long long*)dst, (unsigned long long)acc[i][jj][r]);
        else *dst = (int64_t)((uint64_t)*dst + (uint64_t)acc[i][jj][r]);
      }
    }
}


template <bool S64>
__device__ inline void gemm_wide_tile(const GemmArgs& a, int64_t wg, int* s_lw) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int64_t t0, o0, t0g;
  bool live;
  gemm_tile(a, wave, t0, o0, t0g, live, wg);
  if (!live) return;
  if (a.wide_any && a.wide_any[t0g >> 6] == 0) return;
  gemm_slab_limbs(a, t0g, s_lw);
  bool any = false;
  for (int64_t sl = 0; sl < a.nslabs; ++sl) any = any || s_lw[sl] > kNarrowLimbs;
  if (!any) return;
  gemm_wide_wave<S64, 2, 4, false>(a, t0, o0, s_lw);
}

// One workgroup per (64-token, 128-output) tile; with the tile flags written by the sign-copy kernel
// (a.wide_any) the workgroups of tiles no slab of which is wide end after one flag read.
template <bool S64>
__global__ __launch_bounds__(256) void q1_gemm_wide_kernel(GemmArgs a) {
  __shared__ int s_lw[kGemmMaxSlabs];
  gemm_wide_tile<S64>(a, blockIdx.x, s_lw);
}

// ------------------------------------------------------------------------------------------------------
// Prefill GEMM over the sign copy, several weights per launch (q1_gemm_ps_kernel). The same operands, LDS ring
// and swizzle as q1_gemm_pm_kernel, with three changes:
// * Int32 partial sums without folds. Each block's floor(S * scale / 2^frac) is added into an int32 partial; the
//   host proves, from the weight's row sums of |scale| and |S| < 2^30 (3 limbs), that the sum over the partial's
//   block range stays below 2^31 in magnitude, so the partial is exact after sign extension whatever it wrapped
//   through on the way (NP = 2: the second half of the blocks in a second partial). No int64 accumulators: a
//   32 x 64 sub-tile per wave (8 waves, two per SIMD) holds 8 independent MFMA chains, and each A operand row read
//   from LDS serves 4 output groups and each B row 2 token groups (a 32 x 32 sub-tile, 16 waves at 128 VGPRs,
//   reads twice the LDS bytes per MFMA).
// * The copies of block b + 1 are issued in three parts, one before each limb's MFMAs of block b, so the copy
//   traffic is spread over the block instead of queueing in front of it.
// * Slabs needing more than 3 limbs over a 64-token half (rare: activations beyond 2^23) are computed by the same
//   workgroup after its sums are stored (gemm_wide_wave, 64-bit atomic adds), so no second launch runs.
// One launch covers up to kMaxSegs weights of the same n_blocks (q / k / v, gate / up): their output tiles are
// concatenated, so the small k / v projections share the grid with q instead of each filling part of the chip.
// ------------------------------------------------------------------------------------------------------
constexpr int kPsBt = 4, kPsBo = 8;                  // q1_gemm_ps_kernel block of token x output tiles per XCD round
struct PsArgs {
  GemmArgs s[kMaxSegs];
  int64_t tend[kMaxSegs];          // cumulative output tiles through segment i
  uint32_t sg_bytes[kMaxSegs], sc_bytes[kMaxSegs];
  uint32_t xg_bytes;
  int cnt;
  int map;                         // 1: blocked tile order (see the kernel)
};

// ACC: some segment adds into its outputs (the segment's accumulate flag); see q1_gemm_pm_kernel
template <int MT, int NT, int NP, bool ACC = false>
__global__ __launch_bounds__(4096 / (MT * NT)) void q1_gemm_ps_kernel(PsArgs P) {
  constexpr int NW = 64 / (MT * NT);             // waves of 16 MT x 16 NT covering the 128 x 128 tile
  constexpr int WO = 128 / (16 * NT);            // waves along the outputs
  constexpr int QA = 48 / NW, QB = 16 / NW;      // 1 KB copies per wave and block: A (3 limbs x 16 row groups), B
  static_assert(NW == 8 || NW == 16, "8 or 16 waves");
  __shared__ int s_lw[2][kGemmMaxSlabs];
  __shared__ v4i sA0[kNarrowLimbs][kPmTok * 8], sA1[kNarrowLimbs][kPmTok * 8];   // 2 x 48 KB
  __shared__ v4i sB0[128 * 8], sB1[128 * 8];                                      // 2 x 16 KB
  __shared__ int32_t sS0[128], sS1[128];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t T = P.s[0].T, ntt = (T + kPmTok - 1) / kPmTok, nto = P.tend[P.cnt - 1], wg = blockIdx.x;
  int64_t tt, ot;
  bool live;
  if (P.map) {
    // blocks of kPsBt token tiles x kPsBo output tiles, one block per XCD round (the XCD's 32 CUs run one
    // workgroup each): every sign tile of the block is fetched for kPsBt workgroups and every digit tile for kPsBo
    // through the XCD's L2, instead of the sign tiles of 32 output tiles once each
    const int64_t xcd = wg & 7, j = wg >> 3, G = (j / (kPsBt * kPsBo)) * 8 + xcd, r = j % (kPsBt * kPsBo);
    const int64_t ntb = (ntt + kPsBt - 1) / kPsBt;
    tt = (G % ntb) * kPsBt + r / kPsBo;
    ot = (G / ntb) * kPsBo + r % kPsBo;
    live = tt < ntt && ot < nto;
  } else if (ntt >= 8) {                              // each XCD walks whole token tiles (their digits stay in L2)
    const int64_t xcd = wg & 7, j = wg >> 3, tpx = (ntt + 7) / 8;
    tt = xcd + 8 * (j / nto);
    ot = j % nto;
    live = tt < ntt && (j / nto) < tpx;
  } else {
    tt = wg / nto;
    ot = wg % nto;
    live = tt < ntt;
  }
  if (!live) return;
  const int seg = (ot >= P.tend[0] ? 1 : 0) + (P.cnt > 2 && ot >= P.tend[1] ? 1 : 0);
  const GemmArgs a = seg == 0 ? P.s[0] : (seg == 1 ? P.s[1] : P.s[2]);
  const uint32_t sg_bytes = seg == 0 ? P.sg_bytes[0] : (seg == 1 ? P.sg_bytes[1] : P.sg_bytes[2]);
  const uint32_t sc_bytes = seg == 0 ? P.sc_bytes[0] : (seg == 1 ? P.sc_bytes[1] : P.sc_bytes[2]);
  if (seg) ot -= P.tend[seg - 1];
  const int64_t t0g = tt * kPmTok, o0g = ot * 128;
  for (int64_t q = wave; q < 2 * a.nslabs; q += NW) {  // (half, slab) limb maxima over 64 tokens each
    const int hh = (int)(q & 1);
    const int64_t sl = q >> 1, t = t0g + 64 * hh + lane;
    int L = t < T ? a.lt[t * a.nslabs + sl] : 0;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) { const int w2 = __shfl_xor(L, o, 64); L = w2 > L ? w2 : L; }
    if (lane == 0) s_lw[hh][sl] = L;
  }
  const int m = lane & 15, g = lane >> 4;
  const int tb = (wave / WO) * 16 * MT, ob = (wave % WO) * 16 * NT, half = tb >> 6;
  const __amdgpu_buffer_rsrc_t rA = pm_rsrc(a.xg, P.xg_bytes), rB = pm_rsrc(a.signs, sg_bytes),
                               rS = pm_rsrc(a.scaleT, sc_bytes);
  // copy roles: lane L of a 1 KB copy fills slot L & 7 of row L >> 3 of an 8-row group
  const int drow = lane >> 3, dslot = lane & 7;
  uint32_t voA[QA], voB[QB];
#pragma unroll
  for (int q = 0; q < QA; ++q) {
    const int rg = (wave * QA + q) & 15, t = rg * 8 + drow;
    voA[q] = (uint32_t)(t0g + t) * 128u + (uint32_t)(dslot ^ ((t >> 1) & 7)) * 16u;
  }
#pragma unroll
  for (int q = 0; q < QB; ++q) {
    const int r = (wave * QB + q) * 8 + drow;
    const int64_t o = o0g + r < a.N ? o0g + r : a.N - 1;                     // clamp: padding columns unused
    voB[q] = (uint32_t)o * (uint32_t)a.nb * 128u + (uint32_t)(dslot ^ ((r >> 1) & 7)) * 16u;
  }
  const int64_t so_ = o0g + (tid & 127) < a.ntiles16 ? o0g + (tid & 127) : a.ntiles16 - 1;
  const uint32_t voS = (uint32_t)(((so_ >> 4) * a.nslabs * 64 + (so_ & 15)) * 4);
  const uint32_t limb_stride = (uint32_t)a.nbp * (uint32_t)a.Tp * 128u, blk_stride = (uint32_t)a.Tp * 128u;
  // part ph (0..2) of block b's copies, or all of them (ph < 0); all three limbs are copied (the table holds zero
  // digits above a token's limb count)
  auto issue = [&](int64_t b, v4i (*dA)[kPmTok * 8], v4i* dB, int ph) {
#pragma unroll
    for (int q = 0; q < QA; ++q) {
      if (ph >= 0 && q / (QA / 3) != ph) continue;
      const int qi = wave * QA + q, l = qi >> 4, rg = qi & 15;
      pm_dma(rA, &dA[l][rg * 64], voA[q], (uint32_t)l * limb_stride + (uint32_t)b * blk_stride);
    }
    if (ph < 0 || ph == 2)
#pragma unroll
      for (int q = 0; q < QB; ++q) pm_dma(rB, &dB[(wave * QB + q) * 64], voB[q], (uint32_t)b * 128u);
  };
  auto load_scale = [&](int64_t b) -> int32_t {
    return (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rS, (int)voS, (int)((((b >> 2) * 64) + 16 * (b & 3)) * 4), 0);
  };
  // NP int32 partial sums (NP = 2: blocks from a.rlen on go to `part` after `sav` took the first range)
  int32_t part[MT][NT][4], sav[MT][NT][NP == 2 ? 4 : 1];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int jj = 0; jj < NT; ++jj) {
#pragma unroll
      for (int r = 0; r < 4; ++r) part[i][jj][r] = 0;
#pragma unroll
      for (int r = 0; r < (NP == 2 ? 4 : 1); ++r) sav[i][jj][r] = 0;
    }
  const int64_t t0 = t0g + tb, o0 = o0g + ob;
  // per-lane physical chunk of K half h (the swizzle term (row >> 1) & 7 is (m >> 1) & 7 for every read row)
  const int pc0 = (0 + g) ^ ((m >> 1) & 7), pc1 = (4 + g) ^ ((m >> 1) & 7);
  __syncthreads();                                    // s_lw
  bool wide0 = false, wide1 = false;
  for (int64_t sl = 0; sl < a.nslabs; ++sl) {
    wide0 = wide0 || s_lw[0][sl] > kNarrowLimbs;
    wide1 = wide1 || s_lw[1][sl] > kNarrowLimbs;
  }
  issue(0, sA0, sB0, -1);
  if (tid < 128) sS0[tid] = load_scale(0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  // block b from (cA, cB, cS) while block b + 1 is copied into (nA, nB, nS)
  auto step = [&](int64_t b, const v4i (*cA)[kPmTok * 8], const v4i* cB, const int32_t* cS, v4i (*nA)[kPmTok * 8],
                  v4i* nB, int32_t* nS) {
    const bool more = b + 1 < a.nb;
    int32_t ps = 0;
    if (more && tid < 128) ps = load_scale(b + 1);
    if constexpr (NP == 2) {
      if (b == a.rlen) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int jj = 0; jj < NT; ++jj)
#pragma unroll
            for (int q = 0; q < 4; ++q) { sav[i][jj][q] = part[i][jj][q]; part[i][jj][q] = 0; }
      }
    }
    const int lw = s_lw[half][b >> 2];               // this wave's 64-token half
    if (lw <= kNarrowLimbs) {
      v4i bx[NT][2];
#pragma unroll
      for (int jj = 0; jj < NT; ++jj) {
        const int r = ob + 16 * jj + m;
        bx[jj][0] = cB[r * 8 + pc0];
        bx[jj][1] = cB[r * 8 + pc1];
      }
      int32_t scp[NT];
#pragma unroll
      for (int jj = 0; jj < NT; ++jj) scp[jj] = (int32_t)((uint32_t)cS[ob + 16 * jj + m] << (32 - a.frac));
      // limbs outermost: S = ((D2 * 256) + D1) * 256 + D0 per chain, each limb's operands read once
      v4i c[MT][NT];
      __builtin_amdgcn_s_setprio(1);               // favour this wave's MFMA issue over the others' epilogues
#pragma unroll
      for (int l = kNarrowLimbs - 1; l >= 0; --l) {
        if (more) issue(b + 1, nA, nB, kNarrowLimbs - 1 - l);
        v4i av[MT][2];
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          const int r = tb + 16 * i + m;
          av[i][0] = cA[l][r * 8 + pc0];
          av[i][1] = cA[l][r * 8 + pc1];
        }
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int jj = 0; jj < NT; ++jj) {
            v4i x = l == kNarrowLimbs - 1 ? v4i{0, 0, 0, 0}
                                          : v4i{(int)((uint32_t)c[i][jj][0] << 8), (int)((uint32_t)c[i][jj][1] << 8),
                                                (int)((uint32_t)c[i][jj][2] << 8), (int)((uint32_t)c[i][jj][3] << 8)};
            x = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i][0], bx[jj][0], x, 0, 0, 0);
            c[i][jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i][1], bx[jj][1], x, 0, 0, 0);
          }
      }
      // high dword of S * (scale << (32 - frac)) = floor(S * scale / 2^frac)
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int jj = 0; jj < NT; ++jj)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            part[i][jj][q] = (int32_t)((uint32_t)part[i][jj][q] + (uint32_t)__mulhi(c[i][jj][q], scp[jj]));
      __builtin_amdgcn_s_setprio(0);
    } else if (more) {
      issue(b + 1, nA, nB, -1);
    }
    if (more && tid < 128) nS[tid] = ps;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's copies of block b + 1 have landed
    __syncthreads();                                  // ... and every wave's; block b's half is free again
  };
  for (int64_t b = 0; b < a.nb; b += 2) {
    step(b, sA0, sB0, sS0, sA1, sB1, sS1);
    if (b + 1 < a.nb) step(b + 1, sA1, sB1, sS1, sA0, sB0, sS0);
  }
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int jj = 0; jj < NT; ++jj) {
      const int64_t o = o0 + 16 * jj + m;
      if (o >= a.N) continue;
      int64_t prev[4] = {0, 0, 0, 0};
      if constexpr (ACC) {
        if (a.accumulate) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int64_t t = t0 + 16 * i + 4 * g + q;
            prev[q] = t < T ? a.out[t * a.N + o] : 0;
          }
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t t = t0 + 16 * i + 4 * g + q;
        if (t >= T) continue;
        int64_t v = (int64_t)part[i][jj][q];
        if constexpr (NP == 2) v += (int64_t)sav[i][jj][q];
        a.out[t * a.N + o] = (int64_t)((uint64_t)prev[q] + (uint64_t)v);
      }
    }
  if (wide0 || wide1) {                               // uniform over the workgroup
    __threadfence();
    if (half ? wide1 : wide0) gemm_wide_wave<false, MT, NT, true>(a, t0, o0, s_lw[half]);
  }
}

// ------------------------------------------------------------------------------------------------------
// Batched-decode GEMM (kGemmMinT <= T <= 64 tokens, one token tile). The weights are streamed once and a launch
// moves only a few MB, so the kernel is built around having the bytes in flight early:
// * Workgroup = 128 outputs x 16 MT tokens over a K range of at most kBtMaxBlk blocks (the whole K, or a few
//   ranges added with 64-bit atomics when the output count alone cannot fill the chip); 4 MT waves, wave = 32
//   outputs (2 MFMA tiles) x one 16-token group, so a SIMD holds MT waves to overlap one another's LDS and MFMA
//   latencies.
// * At entry the workgroup copies ALL of its range's weight bits and scales into LDS (buffer_load ... lds, no
//   registers): the whole matrix is requested in the first microseconds instead of a few blocks at a time. The
//   digit rows of each block (3 limbs x 16 MT tokens, L2-resident) and its negated totals go through a ring of RA
//   slots, RA - 1 blocks ahead. The copies are inline asm, so the compiler adds no waits of its own; each block
//   waits with s_waitcnt vmcnt for the copies issued after it, then a bare s_barrier (no release fence, which would
//   drain the ring).
// * Per block the narrow kernel's arithmetic: pos by Horner over the limbs (int32 exact, |pos| <= 2^30), S = 2 pos
//   - total, q = floor(S * scale / 2^frac) as the high dword of S * (scale << (32 - frac)) (int32 scales below
//   2^(frac - 1)); q summed in an int32 partial folded into int64 every kf blocks, kf from the weight's largest
//   |scale| (kf ((2^30 max|scale|) >> frac) + kf < 2^31).
// * A slab needing more than 3 limbs over the T tokens is skipped here and computed afterwards by gemm_wide_wave
//   over the same range (int64, any limb count, 64-bit atomics).
// ------------------------------------------------------------------------------------------------------
constexpr int kBtMaxBlk = 32;      // blocks per workgroup range (the range's weights sit in LDS)
struct BtArgs {
  GemmArgs s[kMaxSegs];
  int64_t tend[kMaxSegs];          // cumulative output groups of 128 through segment i
  uint32_t bt_bytes[kMaxSegs], sc_bytes[kMaxSegs];
  uint32_t xg_bytes, tg_bytes;
  int cnt, nkr, kf;
};

template <int MT>
struct __align__(16) BtASlot {
  v4i A[kNarrowLimbs * 16 * MT * 8];   // [limb][token][chunk slot], slot = chunk ^ ((token >> 1) & 7)
  int64_t tot[64];
};

template <int N>
__device__ inline void bt_wait_vm() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

// LDS DMA issued as inline asm: the compiler does not track it, so it inserts no waits of its own before the LDS
// reads (its tracking cannot tell ring slots apart and would drain every copy in flight); every wait on these
// copies is the kernel's explicit s_waitcnt vmcnt, and the "memory" clobber keeps a block's LDS reads after the
// wait that covers it
__device__ inline void bt_dma(__amdgpu_buffer_rsrc_t r, const void* lds, uint32_t voff, uint32_t soff) {
  const uint32_t base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds;
  soff = __builtin_amdgcn_readfirstlane(soff);       // uniform by construction; the operand must be an SGPR
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" : : "v"(voff), "s"(r), "s"(soff), "{m0}"(base)
               : "memory");
}

template <int MT, int RA>
__global__ __launch_bounds__(256 * MT) void q1_gemm_bt_kernel(BtArgs P) {
  constexpr int NT = 2, NW = 4 * MT, ROWS = 16 * MT, NJA = 6 * MT + 1, QA = (NJA + NW - 1) / NW;
  static_assert((RA - 2) * QA <= 63, "vmcnt range");
  __shared__ uint4 sWb[kBtMaxBlk][128];               // [block][tile][row]
  __shared__ int32_t sWs[kBtMaxBlk][128];
  __shared__ BtASlot<MT> SA[RA];
  __shared__ int s_lw[kGemmMaxSlabs];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tw = wave & 3, ig = wave >> 2;            // output tile pair, 16-token group
  int64_t og = blockIdx.x;
  const int seg = (og >= P.tend[0] ? 1 : 0) + (P.cnt > 2 && og >= P.tend[1] ? 1 : 0);
  const GemmArgs& a = seg == 0 ? P.s[0] : (seg == 1 ? P.s[1] : P.s[2]);
  const uint32_t bt_bytes = seg == 0 ? P.bt_bytes[0] : (seg == 1 ? P.bt_bytes[1] : P.bt_bytes[2]);
  const uint32_t sc_bytes = seg == 0 ? P.sc_bytes[0] : (seg == 1 ? P.sc_bytes[1] : P.sc_bytes[2]);
  if (seg) og -= P.tend[seg - 1];
  const int64_t b0 = (int64_t)blockIdx.y * a.nb / P.nkr, b1 = ((int64_t)blockIdx.y + 1) * a.nb / P.nkr;
  const int64_t nbr = b1 - b0;                        // <= kBtMaxBlk (host)
  const int m = lane & 15, g = lane >> 4;
  const int64_t o0 = og * 128, o0w = o0 + 32 * tw;
  const __amdgpu_buffer_rsrc_t rA = pm_rsrc(a.xg, P.xg_bytes), rT = pm_rsrc(a.tg, P.tg_bytes),
                               rB = pm_rsrc(a.bitsT, bt_bytes), rS = pm_rsrc(a.scaleT, sc_bytes);
  const int64_t ntl = a.ntiles16 >> 4;
  // the range's blocks in a rotated order (workgroup-dependent start), so workgroups running together read
  // different blocks' digit rows
  const int64_t rot = nbr > 1 ? ((int64_t)blockIdx.x * 7) % nbr : 0;
  auto phys = [&](int64_t k) { const int64_t v = k + rot; return b0 + (v >= nbr ? v - nbr : v); };
  // slab limb counts over the T tokens (wave 0; T <= 64: one lane per token), loaded before any copy is issued
  // (the compiler's wait for these loads then drains nothing else)
  if (wave == 0)
    for (int64_t sl = b0 >> 2; sl <= (b1 - 1) >> 2; ++sl) {
      int L = lane < a.T ? a.lt[(int64_t)lane * a.nslabs + sl] : 0;
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) { const int w2 = __shfl_xor(L, o, 64); L = w2 > L ? w2 : L; }
      if (lane == 0) s_lw[sl] = L;
    }
  // every weight copy of the range first: job j = (logical block j / 3, part j % 3: bits of tiles 0-3, 4-7, scales)
  {
    const int64_t otb = min((o0 >> 4) + (lane >> 4), ntl - 1), otb2 = min((o0 >> 4) + 4 + (lane >> 4), ntl - 1);
    const int64_t ots = min((o0 >> 4) + (lane >> 2), ntl - 1);
    const uint32_t vb0 = (uint32_t)((otb * a.nslabs * 64 + (lane & 15)) * 16);
    const uint32_t vb1 = (uint32_t)((otb2 * a.nslabs * 64 + (lane & 15)) * 16);
    const uint32_t vs = (uint32_t)((ots * a.nslabs * 64 + 4 * (lane & 3)) * 4);
    for (int j = wave; j < 3 * nbr; j += NW) {
      const int kb = j / 3, part = j - 3 * kb;
      const int64_t b = phys(kb);
      const uint32_t sb = (uint32_t)(((b >> 2) * 64) + 16 * (b & 3));
      if (part < 2) bt_dma(rB, &sWb[kb][64 * part], part ? vb1 : vb0, sb * 16u);
      else if (lane < 32) bt_dma(rS, &sWs[kb][0], vs, sb * 4u);
    }
  }
  // digit-row copy jobs of a block: 0 the totals, 1.. 8 rows of 128 B each; a wave's jobs beyond the last repeat
  // it (the same bytes to the same place)
  const uint32_t limb_stride = (uint32_t)a.nbp * (uint32_t)a.Tp * 128u;
  int ja[QA];
  uint32_t va[QA];
#pragma unroll
  for (int q = 0; q < QA; ++q) {
    const int j = min(wave + NW * q, NJA - 1);
    ja[q] = j;
    if (j == 0) {
      va[q] = (uint32_t)lane * 16u;
    } else {
      const int rr = 8 * (j - 1) + (lane >> 3), l = rr / ROWS, t = rr - l * ROWS;
      va[q] = (uint32_t)l * limb_stride + (uint32_t)t * 128u + (uint32_t)((lane & 7) ^ ((t >> 1) & 7)) * 16u;
    }
  }
  auto issue_a = [&](int64_t b, BtASlot<MT>& d) {
#pragma unroll
    for (int q = 0; q < QA; ++q) {
      const int j = ja[q];
      if (j == 0) {
        if (lane < 8 * MT) bt_dma(rT, &d.tot[0], va[q], (uint32_t)b * (uint32_t)a.Tp * 8u);
      } else {
        bt_dma(rA, &d.A[64 * (j - 1)], va[q], (uint32_t)b * (uint32_t)a.Tp * 128u);
      }
    }
  };
#pragma unroll
  for (int k = 0; k < RA - 1; ++k)
    if (k < nbr) issue_a(phys(k), SA[k]);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();                       // s_lw (a bare barrier: the copies stay in flight)
  int64_t acc[NT][4];
  int32_t part[NT][4];
#pragma unroll
  for (int jj = 0; jj < NT; ++jj)
#pragma unroll
    for (int r = 0; r < 4; ++r) { acc[jj][r] = 0; part[jj][r] = 0; }
  int fc = 0;
  // the range's slab limb counts in one register: 4 bits per slab from the first (the range spans <= 9 slabs)
  const int64_t sl0 = b0 >> 2;
  uint64_t lwm = 0;
  bool wide = false;
  for (int64_t sl = sl0; sl <= (b1 - 1) >> 2; ++sl) {
    const int v = s_lw[sl];
    wide = wide || v > kNarrowLimbs;
    lwm |= (uint64_t)(v > kNarrowLimbs ? 15 : v) << (4 * (sl - sl0));
  }
  const int sw = (m >> 1) & 7;
  // one block with L limbs: every LDS operand read issued together, then the Horner chains of the two tiles
  auto block = [&](auto LC, int64_t k, const BtASlot<MT>& c) {
    constexpr int L = decltype(LC)::value;
    uint4 w[NT];
    int32_t sc[NT];
    v4i av[L][2];
    int64_t tv[4];
#pragma unroll
    for (int jj = 0; jj < NT; ++jj) {
      w[jj] = sWb[k][(2 * tw + jj) * 16 + m];
      sc[jj] = sWs[k][(2 * tw + jj) * 16 + m];
    }
#pragma unroll
    for (int l = 0; l < L; ++l)
#pragma unroll
      for (int h = 0; h < 2; ++h) av[l][h] = c.A[(l * ROWS + 16 * ig + m) * 8 + ((4 * h + g) ^ sw)];
#pragma unroll
    for (int r = 0; r < 4; ++r) tv[r] = c.tot[16 * ig + 4 * g + r];
    v4i bx[NT][2];
#pragma unroll
    for (int jj = 0; jj < NT; ++jj) {
      bx[jj][0] = expand_bits(w[jj], g);
      bx[jj][1] = expand_bits(w[jj], 4 + g);
    }
    v4i D[NT];
#pragma unroll
    for (int l = L - 1; l >= 0; --l)
#pragma unroll
      for (int jj = 0; jj < NT; ++jj) {
        v4i x = v4i{0, 0, 0, 0};
        if (l < L - 1)
          x = v4i{(int)((uint32_t)D[jj][0] << 8), (int)((uint32_t)D[jj][1] << 8), (int)((uint32_t)D[jj][2] << 8),
                  (int)((uint32_t)D[jj][3] << 8)};
        x = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[l][0], bx[jj][0], x, 0, 0, 0);
        D[jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[l][1], bx[jj][1], x, 0, 0, 0);
      }
#pragma unroll
    for (int jj = 0; jj < NT; ++jj) {
      const int32_t scp = (int32_t)((uint32_t)sc[jj] << (32 - a.frac));
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int32_t S = (int32_t)(((uint32_t)D[jj][r] << 1) - (uint32_t)tv[r]);
        part[jj][r] = (int32_t)((uint32_t)part[jj][r] + (uint32_t)__mulhi(S, scp));
      }
    }
  };
  for (int64_t k = 0; k < nbr; ++k) {
    if (k + RA - 2 < nbr) bt_wait_vm<(RA - 2) * QA>();
    else bt_wait_vm<0>();
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    if (k + RA - 1 < nbr) issue_a(phys(k + RA - 1), SA[(k + RA - 1) % RA]);
    const int lw = (int)((lwm >> (4 * ((phys(k) >> 2) - sl0))) & 15);
    if (lw > kNarrowLimbs || lw == 0) continue;   // wide slab (done afterwards) or all-zero digits
    const BtASlot<MT>& c = SA[k % RA];
    if (lw == 3) block(std::integral_constant<int, 3>{}, k, c);
    else if (lw == 2) block(std::integral_constant<int, 2>{}, k, c);
    else block(std::integral_constant<int, 1>{}, k, c);
    if (++fc == P.kf) {
      fc = 0;
#pragma unroll
      for (int jj = 0; jj < NT; ++jj)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          acc[jj][r] = (int64_t)((uint64_t)acc[jj][r] + (uint64_t)(int64_t)part[jj][r]);
          part[jj][r] = 0;
        }
    }
  }
  const bool atomic = P.nkr > 1;
#pragma unroll
  for (int jj = 0; jj < NT; ++jj) {
    const int64_t o = o0w + 16 * jj + m;
    if (o >= a.N) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t t = 16 * ig + 4 * g + r;
      if (t >= a.T) continue;
      const int64_t v = (int64_t)((uint64_t)acc[jj][r] + (uint64_t)(int64_t)part[jj][r]);
      int64_t* dst = a.out + t * a.N + o;
      if (atomic) atomicAdd((unsigned long long*)dst, (unsigned long long)v);
      else *dst = a.accumulate ? (int64_t)((uint64_t)*dst + (uint64_t)v) : v;
    }
  }
  if (wide && o0w < a.N) {                            // uniform over the workgroup
    __threadfence();
    gemm_wide_wave<false, 1, NT, true>(a, 16 * ig, o0w, s_lw, b0, b1);
  }
}

// Executed int8 MFMA ops of one GEMM launch pair (profiling only): per (token tile, slab) the limb count the
// kernels use (max over the tile's tokens) x the slab's blocks x the output tiles x 64 MFMAs of 2*16*16*64 ops.
__global__ void gemm_opcount_kernel(const int* __restrict__ lt, int64_t T, int64_t nslabs, int64_t nb, int64_t nto,
                                    unsigned long long* __restrict__ ops) {
  const int64_t tt = blockIdx.x;
  unsigned long long sum = 0;
  for (int64_t sl = threadIdx.x; sl < nslabs; sl += blockDim.x) {
    int lw = 0;
    for (int64_t t = tt * 64; t < min(T, tt * 64 + 64); ++t) lw = lt[t * nslabs + sl] > lw ? lt[t * nslabs + sl] : lw;
    const int64_t blocks = min((int64_t)kSlabBlocks, nb - sl * kSlabBlocks);
    sum += (unsigned long long)(nto * blocks * lw) * 64ull * 32768ull;
  }
  if (sum) atomicAdd(ops, sum);
}
// narrow GEMM LDS buffering (IMIE_GEMM_NBUF = 1 or 2 overrides; tuning)
static int gemm_nbuf() {
  static const int v = [] {
    const char* e = getenv("IMIE_GEMM_NBUF");
    const int n = e ? atoi(e) : 0;
    return n == 1 || n == 2 ? n : 1;
  }();
  return v;
}

// batched-decode GEMM for T <= 64 (IMIE_GEMM_BT=0 disables; tuning and tests)
static bool gemm_bt() {
  static const bool v = [] { const char* e = getenv("IMIE_GEMM_BT"); return !(e && atoi(e) == 0); }();
  return v;
}

// batched-decode GEMM: workgroups below which the K range is split (IMIE_BT_MINWG; tuning)
static int64_t bt_min_wgs() {
  static const int64_t v = [] { const char* e = getenv("IMIE_BT_MINWG"); return (int64_t)(e ? atoi(e) : 128); }();
  return v;
}

// high-dword GEMM epilogue where the scales allow it (IMIE_GEMM_FASTEPI=0 disables; tuning and tests)
static bool gemm_fast_epi() {
  static const bool v = [] { const char* e = getenv("IMIE_GEMM_FASTEPI"); return !(e && atoi(e) == 0); }();
  return v;
}

__global__ void q1_zero_kernel(int64_t* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0;
}

// +-1 sign GEMM for T >= kPmMinT (IMIE_GEMM_PM=0 disables; tuning and tests)
static bool gemm_pm() {
  static const bool v = [] { const char* e = getenv("IMIE_GEMM_PM"); return !(e && atoi(e) == 0); }();
  return v;
}

static int ps_shape() {
  static const int v = [] { const char* e = getenv("IMIE_PS_SHAPE"); return e ? atoi(e) : 1; }();
  return v;
}
static int ps_map() { const char* e = getenv("IMIE_PS_MAP"); return e ? atoi(e) : 1; }

// the multi-weight unfolded-partial kernel where its bounds hold (IMIE_GEMM_PS=0 disables; tuning and tests)
static bool gemm_ps() {
  static const bool v = [] { const char* e = getenv("IMIE_GEMM_PS"); return !(e && atoi(e) == 0); }();
  return v;
}

// The weight's sign copy, made on first use (1 byte per weight). Not made while `st` is being captured into a
// graph (allocation is not capturable); the caller then uses the bit kernels.
static int q1_ensure_signs(Q1Weight& w, hipStream_t st) {
  if (w.signs) return 0;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return 1;
  const size_t bytes = (size_t)w.N * w.nb * 128;
  if (hipMalloc((void**)&w.signs, bytes) != hipSuccess) { w.signs = nullptr; (void)hipGetLastError(); return 1; }
  const int64_t n = w.N * w.nb;
  hipLaunchKernelGGL(q1_signs_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, (const uint4*)w.bits, w.N,
                     w.nb, w.nslabs, w.signs);
  if (hipGetLastError() != hipSuccess) { imie_free(w.signs); w.signs = nullptr; return 1; }
  w.bytes += bytes;
  g_resident_bytes += bytes;
  return 0;
}

// The GEMM table of T tokens for weights of nb blocks (imie_q1_gemm_target and the prep below agree on it).
static int gemm_table(Q1Ws& wk, int64_t nb, int64_t T, GemmPrepOut* gp) {
  const int64_t nslabs = (nb + kSlabBlocks - 1) / kSlabBlocks, nbp = nslabs * kSlabBlocks;
  const int64_t Tp = (T + kPmTok - 1) / kPmTok * kPmTok;
  if (nslabs > kGemmMaxSlabs) return IMIE_EARG;
  if (wk.xq.ensure((size_t)kMaxLimbs * nbp * Tp * 128) || wk.totals.ensure((size_t)nbp * Tp * 8) ||
      wk.lslab.ensure((size_t)T * nslabs * 4) || wk.wide.ensure((size_t)(Tp / 64) * 4))
    return IMIE_EARG;
  *gp = GemmPrepOut{(uint4*)wk.xq.p, (int64_t*)wk.totals.p, (int*)wk.lslab.p, nb, nbp, nslabs, Tp};
  return IMIE_OK;
}

// prepped != 0: the table is already in wk (a fused producer wrote it through imie_q1_gemm_target)
static int q1_gemm_multi(const Q1Weight* const* ws, int cnt, const int64_t* x_dev, int64_t T, int64_t frac,
                         int64_t* const* outs, int accumulate, Q1Ws& wk, hipStream_t st, int prepped = 0) {
  const Q1Weight& w0 = *ws[0];
  GemmPrepOut gp;
  if (gemm_table(wk, w0.nb, T, &gp)) return IMIE_EARG;
  const int64_t nslabs = gp.nslabs, nbp = gp.nbp, Tp = gp.Tp;
  if (!prepped) {
    imie_prof_mark(IMIE_K_Q1_PREP, st, true);
    hipLaunchKernelGGL(q1_prep_gemm_kernel, dim3((unsigned)((nslabs + 3) / 4), (unsigned)T), dim3(256), 0, st, x_dev,
                       w0.nb * 128, gp);
    imie_prof_mark(IMIE_K_Q1_PREP, st, false);
    IMIE_HIP(hipGetLastError());
  }
  imie_prof_mark(IMIE_K_Q1_GEMM, st, true);
  GemmArgs gas[kMaxSegs];
  int nps[kMaxSegs];
  bool all_ps = T >= kPmMinT && gemm_pm() && gemm_ps();
  const uint64_t xg_bytes = (uint64_t)kNarrowLimbs * nbp * Tp * 128;
  for (int i = 0; i < cnt; ++i) {
    const Q1Weight& w = *ws[i];
    GemmArgs& ga = gas[i];
    ga.signs = nullptr;
    ga.wide_any = nullptr;
    ga.ksplit = 1;
    ga.bitsT = w.bits; ga.scaleT = w.scale; ga.xg = (const uint4*)wk.xq.p; ga.tg = (const int64_t*)wk.totals.p;
    ga.lt = (const int*)wk.lslab.p; ga.T = T; ga.Tp = Tp; ga.N = w.N; ga.nb = w.nb; ga.nbp = nbp;
    ga.nslabs = nslabs; ga.ntt = (T + 63) / 64; ga.nto = (w.N + 127) / 128; ga.ntiles16 = w.ntiles * 16;
    ga.frac = (int)(frac > 63 ? 63 : frac); ga.accumulate = accumulate; ga.out = outs[i];
    // high-dword epilogue: int32 scales below 2^(frac-1); |q| = |floor(S * scale / 2^frac)| <= max_q with
    // |S| < 2^30 (narrow blocks); fold before |A| + max_q could reach 2^31
    ga.kfold = 0;
    if (!w.scale64 && ga.frac >= 1 && ga.frac <= 31 && w.maxsc < ((int64_t)1 << (ga.frac - 1)) && gemm_fast_epi()) {
      const int64_t max_q = (((int64_t)w.maxsc << 30) >> ga.frac) + 2;
      const int64_t k = (((int64_t)1 << 31) - 1) / max_q - 1;
      ga.kfold = (int)(k < 1 ? 1 : (k > (1 << 20) ? (1 << 20) : k));
    }
    // unfolded int32 partials (q1_gemm_ps_kernel): over a range of blocks the sum of |floor(S * scale / 2^frac)|
    // with |S| < 2^30 is at most ((2^30 * range sum of |scale|) >> frac) + blocks, which must stay below 2^31;
    // one range, or two halves
    nps[i] = 0;
    if (ga.kfold > 0)
      for (int r = 1; r <= 2 && !nps[i]; ++r) {
        const int64_t rl = (w.nb + r - 1) / r;
        const unsigned __int128 bound = (((unsigned __int128)w.rsum[r - 1] << 30) >> ga.frac) + (uint64_t)rl;
        if (bound < ((unsigned __int128)1 << 31) - 1) { nps[i] = r; ga.rlen = (int)rl; }
      }
    const uint64_t sg_bytes = (uint64_t)w.N * w.nb * 128, sc_bytes = (uint64_t)w.ntiles * nslabs * 64 * 4;
    all_ps = all_ps && nps[i] > 0 && xg_bytes < (1ull << 32) && sg_bytes < (1ull << 32) && sc_bytes < (1ull << 32);
  }
  for (int i = 0; i < cnt && all_ps; ++i) all_ps = q1_ensure_signs(const_cast<Q1Weight&>(*ws[i]), st) == 0;
  // batched decode (one token tile of <= 64): q1_gemm_bt_kernel where its int32 partial folds can be exact
  bool bt = false;
  if (!all_ps && T <= 64 && gemm_bt()) {
    int64_t ncol = 0, worst = 0;
    bt = true;
    for (int i = 0; i < cnt; ++i) {
      bt = bt && gas[i].kfold > 0;
      ncol += (ws[i]->N + 127) / 128;
      const int64_t q = (((int64_t)ws[i]->maxsc << 30) >> gas[i].frac) + 1;
      worst = q > worst ? q : worst;
    }
    const int64_t kf = worst > 0 ? ((((int64_t)1 << 31) - 2) / worst) : 0;
    const uint64_t tg_bytes = (uint64_t)nbp * Tp * 8;
    for (int i = 0; i < cnt && bt; ++i) {
      const uint64_t bb = (uint64_t)ws[i]->ntiles * nslabs * 64 * 16, sb = (uint64_t)ws[i]->ntiles * nslabs * 64 * 4;
      bt = bb < (1ull << 32) && sb < (1ull << 32);
    }
    // very wide outputs (an LM head) run several rounds of these one-per-CU workgroups: the narrow kernel instead
    bt = bt && kf >= 1 && xg_bytes < (1ull << 32) && tg_bytes < (1ull << 32) && ncol <= 512;
    if (bt) {
      BtArgs P;
      int64_t cols = 0;
      for (int i = 0; i < cnt; ++i) {
        P.s[i] = gas[i];
        cols += (ws[i]->N + 127) / 128;
        P.tend[i] = cols;
        P.bt_bytes[i] = (uint32_t)((uint64_t)ws[i]->ntiles * nslabs * 64 * 16);
        P.sc_bytes[i] = (uint32_t)((uint64_t)ws[i]->ntiles * nslabs * 64 * 4);
      }
      for (int i = cnt; i < kMaxSegs; ++i) { P.s[i] = gas[0]; P.tend[i] = cols; P.bt_bytes[i] = P.sc_bytes[i] = 0; }
      P.cnt = cnt;
      P.kf = (int)(kf > (1 << 20) ? (1 << 20) : kf);
      P.xg_bytes = (uint32_t)xg_bytes;
      P.tg_bytes = (uint32_t)tg_bytes;
      // K ranges (64-bit atomics across them) only when the output groups alone leave most of the chip idle
      int nkr = 1;
      while (nkr < 4 && cols * nkr < bt_min_wgs() && w0.nb / (2 * nkr) >= 8) nkr *= 2;
      while ((w0.nb + nkr - 1) / nkr > kBtMaxBlk) ++nkr;   // the range's weights must fit the workgroup's LDS
      P.nkr = nkr;
      if (nkr > 1 && !accumulate && prepped != 3)
        for (int i = 0; i < cnt; ++i) {
          const int64_t n = T * ws[i]->N;
          hipLaunchKernelGGL(q1_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, outs[i], n);
        }
      const dim3 grid((unsigned)cols, (unsigned)nkr);
      if (T <= 16) hipLaunchKernelGGL((q1_gemm_bt_kernel<1, 6>), grid, dim3(256), 0, st, P);
      else if (T <= 32) hipLaunchKernelGGL((q1_gemm_bt_kernel<2, 6>), grid, dim3(512), 0, st, P);
      else hipLaunchKernelGGL((q1_gemm_bt_kernel<4, 3>), grid, dim3(1024), 0, st, P);
      IMIE_HIP(hipGetLastError());
    }
  }
  if (bt) {
  } else if (all_ps) {
    // one launch for every weight: their output tiles side by side
    PsArgs P;
    int np = 1;
    int64_t tiles = 0;
    for (int i = 0; i < cnt; ++i) {
      gas[i].signs = ws[i]->signs;
      P.s[i] = gas[i];
      tiles += gas[i].nto;
      P.tend[i] = tiles;
      P.sg_bytes[i] = (uint32_t)((uint64_t)ws[i]->N * ws[i]->nb * 128);
      P.sc_bytes[i] = (uint32_t)((uint64_t)ws[i]->ntiles * nslabs * 64 * 4);
      np = nps[i] > np ? nps[i] : np;
    }
    for (int i = cnt; i < kMaxSegs; ++i) { P.s[i] = gas[0]; P.tend[i] = tiles; P.sg_bytes[i] = P.sc_bytes[i] = 0; }
    P.xg_bytes = (uint32_t)xg_bytes;
    P.cnt = cnt;
    const int64_t ntt128 = (T + kPmTok - 1) / kPmTok;
    P.map = ps_map();
    const int64_t nblk = ((ntt128 + kPsBt - 1) / kPsBt) * ((tiles + kPsBo - 1) / kPsBo);
    const dim3 pgrid((unsigned)(P.map ? (nblk + 7) / 8 * 8 * (kPsBt * kPsBo)
                                      : (ntt128 >= 8 ? 8 * ((ntt128 + 7) / 8) * tiles : ntt128 * tiles)));
    // 8 waves of 32 x 64 (IMIE_PS_SHAPE=0 with one partial: 16 waves of 32 x 32, four per SIMD, which read
    // twice the LDS operand bytes per MFMA)
    bool acc = false;
    for (int i = 0; i < cnt; ++i) acc = acc || gas[i].accumulate != 0;
    if (np == 1 && ps_shape() == 0) {
      if (acc) hipLaunchKernelGGL((q1_gemm_ps_kernel<2, 2, 1, true>), pgrid, dim3(1024), 0, st, P);
      else hipLaunchKernelGGL((q1_gemm_ps_kernel<2, 2, 1, false>), pgrid, dim3(1024), 0, st, P);
    } else if (np == 1) {
      if (acc) hipLaunchKernelGGL((q1_gemm_ps_kernel<2, 4, 1, true>), pgrid, dim3(512), 0, st, P);
      else hipLaunchKernelGGL((q1_gemm_ps_kernel<2, 4, 1, false>), pgrid, dim3(512), 0, st, P);
    } else {
      if (acc) hipLaunchKernelGGL((q1_gemm_ps_kernel<2, 4, 2, true>), pgrid, dim3(512), 0, st, P);
      else hipLaunchKernelGGL((q1_gemm_ps_kernel<2, 4, 2, false>), pgrid, dim3(512), 0, st, P);
    }
    IMIE_HIP(hipGetLastError());
  } else {
    for (int i = 0; i < cnt; ++i) {
      const Q1Weight& w = *ws[i];
      GemmArgs& ga = gas[i];
      const dim3 grid((unsigned)(ga.ntt >= 8 ? 8 * ((ga.ntt + 7) / 8) * ga.nto : ga.ntt * ga.nto));
      const int nbuf = gemm_nbuf();
      const uint64_t sg_bytes = (uint64_t)w.N * w.nb * 128, sc_bytes = (uint64_t)w.ntiles * nslabs * 64 * 4;
      if (!w.scale64 && ga.kfold > 0 && T >= kPmMinT && gemm_pm() && xg_bytes < (1ull << 32) &&
          sg_bytes < (1ull << 32) && sc_bytes < (1ull << 32) && q1_ensure_signs(const_cast<Q1Weight&>(w), st) == 0) {
        ga.signs = w.signs;
        ga.wide_any = (int*)wk.wide.p;
        const int64_t ntt128 = (T + kPmTok - 1) / kPmTok;
        const dim3 pgrid((unsigned)(ntt128 >= 8 ? 8 * ((ntt128 + 7) / 8) * ga.nto : ntt128 * ga.nto));
        if (ga.accumulate)
          hipLaunchKernelGGL(q1_gemm_pm_kernel<true>, pgrid, dim3(512), 0, st, ga, (uint32_t)xg_bytes,
                             (uint32_t)sg_bytes, (uint32_t)sc_bytes);
        else
          hipLaunchKernelGGL(q1_gemm_pm_kernel<false>, pgrid, dim3(512), 0, st, ga, (uint32_t)xg_bytes,
                             (uint32_t)sg_bytes, (uint32_t)sc_bytes);
        hipLaunchKernelGGL(q1_gemm_wide_kernel<false>, grid, dim3(256), 0, st, ga);
      } else {
        // few token tiles (batched decode): split K over grid.y so the launch fills the chip; each split adds its
        // partial sums with 64-bit atomics (exact: integer sums mod 2^64 in any order)
        const int64_t tiles = (int64_t)grid.x;
        ga.ksplit = 1;
        if (tiles < 256 && w.nb >= 8) {
          const int64_t want = (512 + tiles - 1) / tiles, cap = w.nb / 4;
          ga.ksplit = (int)(want < cap ? want : cap);
          if (ga.ksplit < 1) ga.ksplit = 1;
        }
        const dim3 ngrid(grid.x, (unsigned)ga.ksplit);
        if (ga.ksplit > 1 && !accumulate && prepped != 3) {   // prepped == 3: the producer cleared the outputs
          const int64_t n = T * w.N;
          hipLaunchKernelGGL(q1_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, outs[i], n);
        }
        if (w.scale64) {
          if (nbuf == 1) hipLaunchKernelGGL((q1_gemm_narrow_kernel<true, 1, false>), ngrid, dim3(256), 0, st, ga);
          else hipLaunchKernelGGL((q1_gemm_narrow_kernel<true, 2, false>), ngrid, dim3(256), 0, st, ga);
          hipLaunchKernelGGL(q1_gemm_wide_kernel<true>, grid, dim3(256), 0, st, ga);
        } else {
          if (ga.kfold > 0) {
            if (nbuf == 1) hipLaunchKernelGGL((q1_gemm_narrow_kernel<false, 1, true>), ngrid, dim3(256), 0, st, ga);
            else hipLaunchKernelGGL((q1_gemm_narrow_kernel<false, 2, true>), ngrid, dim3(256), 0, st, ga);
          } else {
            if (nbuf == 1) hipLaunchKernelGGL((q1_gemm_narrow_kernel<false, 1, false>), ngrid, dim3(256), 0, st, ga);
            else hipLaunchKernelGGL((q1_gemm_narrow_kernel<false, 2, false>), ngrid, dim3(256), 0, st, ga);
          }
          hipLaunchKernelGGL(q1_gemm_wide_kernel<false>, grid, dim3(256), 0, st, ga);
        }
      }
      IMIE_HIP(hipGetLastError());
    }
  }
  imie_prof_mark(IMIE_K_Q1_GEMM, st, false);
  if (imie_prof_on() && !imie_prof_suspend(true)) {   // count outside the timed window
    imie_prof_suspend(false);
    if (!g_gemm_ops.ensure(64)) {
      for (int i = 0; i < cnt; ++i)
        hipLaunchKernelGGL(gemm_opcount_kernel, dim3((unsigned)((T + 63) / 64)), dim3(64), 0, st, (const int*)wk.lslab.p,
                           T, nslabs, w0.nb, (ws[i]->N + 127) / 128, (unsigned long long*)g_gemm_ops.p);
      IMIE_HIP(hipGetLastError());
    }
  }
  return IMIE_OK;
}

// ------------------------------------------------------------------------------------------------------
// Launch helpers
// ------------------------------------------------------------------------------------------------------
// One prep (digit table of x, shared by every segment) and one matvec launch over up to kMaxSegs weights with
// the same n_blocks and scale width; outs[i] receives (T, N_i). accumulate != 0 adds into the outputs.
// prepped != 0: the caller's producer already wrote the digit table into wk (imie_q1_prep_target) and cleared
// every non-accumulated output, so no prep kernel is launched.
static int q1_apply_multi(const Q1Weight* const* ws, int cnt, const int64_t* x_dev, int64_t T, int64_t frac,
                          int64_t* const* outs, int accumulate, Q1Ws& wk, hipStream_t st, int prepped = 0) {
  if (T <= 0) return IMIE_OK;
  if (cnt < 1 || cnt > kMaxSegs) return IMIE_EARG;
  const Q1Weight& w0 = *ws[0];
  for (int i = 1; i < cnt; ++i)
    if (ws[i]->nb != w0.nb || ws[i]->scale64 != w0.scale64) return IMIE_EARG;
  if (T >= kGemmMinT) {
    if (prepped == 1) return IMIE_EARG;               // a matvec table (T < kGemmMinT) cannot feed the GEMM
    return q1_gemm_multi(ws, cnt, x_dev, T, frac, outs, accumulate, wk, st, prepped);
  }
  const int64_t nslabs = w0.nslabs, nbp = nslabs * kSlabBlocks;
  if (wk.xq.ensure((size_t)T * kMaxLimbs * nbp * 8 * 16) || wk.totals.ensure((size_t)T * nbp * 8) ||
      wk.lslab.ensure((size_t)T * nslabs * 4))
    return IMIE_EARG;
  // Work split: waves = tile groups of R tiles; grid.y splits the slabs when there are too few tile groups
  // to keep ~8 waves per CU busy (decode-sized matvecs).
  int64_t ntiles_all = 0;
  for (int i = 0; i < cnt; ++i) ntiles_all += ws[i]->ntiles;
  // R = 4 only for single-token launches (four tokens x four tiles would exceed the register budget)
  const int R = (ntiles_all >= 4 * 16384 && T == 1) ? 4 : (ntiles_all >= 2 * 8192 ? 2 : 1);
  Q1Segs sg = {};
  sg.cnt = cnt;
  int64_t groups = 0;
  for (int i = 0; i < cnt; ++i) {
    sg.bits[i] = ws[i]->bits;
    sg.scale[i] = ws[i]->scale;
    sg.N[i] = ws[i]->N;
    sg.ntiles[i] = ws[i]->ntiles;
    sg.gbegin[i] = groups;
    groups += (ws[i]->ntiles + R - 1) / R;
  }
  sg.gbegin[cnt] = groups;
  int64_t ksplit = 1, spk = nslabs;
  int pf = 0;
  if (T == 1 && R == 1 && groups * nslabs <= 64 * 1024) {
    // decode-sized: the largest slab range of 4 / 2 / 1 that still gives >= 2048 waves; each wave requests
    // its whole range at once, so one round of resident waves covers the matrix
    pf = 1;
    for (int c = 4; c >= 2; c >>= 1)
      if (groups * ((nslabs + c - 1) / c) >= 2048) { pf = c; break; }
    spk = pf < nslabs ? pf : nslabs;
    ksplit = (nslabs + spk - 1) / spk;
    if (pf == 1) pf = 0;                              // one slab per wave: the pipelined kernel is the same
  } else {
    while (groups * ksplit < 8 * 1024 && ksplit * 2 <= nslabs && ksplit < 8) ksplit *= 2;
    spk = (nslabs + ksplit - 1) / ksplit;
    ksplit = (nslabs + spk - 1) / spk;
  }
  const int TT = T <= 1 ? 1 : (T <= 2 ? 2 : 4);
  if (TT == 4 && R == 4) return IMIE_EARG;
  // large single-token launches on one weight: persistent waves (IMIE_Q1_PERS = workgroups per CU, 0 = off)
  static const int pers_wpc = [] { const char* e = getenv("IMIE_Q1_PERS"); return e ? atoi(e) : 3; }();
  const bool pers = pers_wpc > 0 && R == 4 && T == 1 && cnt == 1 && ksplit == 1 && pf == 0;            // not instantiated: R is 4 only for T == 1
  const int Tc = TT;
  // the prep kernel clears the outputs when the matvec adds into them (K-split) and no residual is kept
  Q1Zero zero = {};
  if (ksplit > 1 && !accumulate) {
    zero.cnt = cnt;
    for (int i = 0; i < cnt; ++i) { zero.p[i] = outs[i]; zero.n[i] = T * ws[i]->N; }
  }
  const int64_t K = w0.nb * 128;
  // the persistent launch on K <= 4096 builds its digit table itself (copy prologue): no prep launch
  static const bool pers_pro_on = [] { const char* e = getenv("IMIE_Q1_PERS_PRO"); return !(e && atoi(e) == 0); }();
  const bool pers_pro = pers && !prepped && pers_pro_on && nslabs <= 8 && x_dev;
  if (!prepped && !pers_pro) {
    imie_prof_mark(IMIE_K_Q1_PREP, st, true);
    Q1PrepOut po = {(uint32_t*)wk.xq.p, (int64_t*)wk.totals.p, (int*)wk.lslab.p, w0.nb, nbp, nslabs};
    hipLaunchKernelGGL(q1_prep_kernel, dim3((unsigned)nslabs, (unsigned)T), dim3(64), 0, st, x_dev, K, po, zero);
    imie_prof_mark(IMIE_K_Q1_PREP, st, false);
  }
  IMIE_HIP(hipGetLastError());
  const size_t budget = 48 * 1024;
  // staged limbs come in whole groups of four (a limb group reads either LDS or the global table)
  int Lcap = (int)(budget / ((size_t)Tc * spk * 512));
  Lcap = Lcap >= 8 ? 8 : (Lcap >= 4 ? 4 : 0);
  if (pers_pro) Lcap = 8;                            // the prologue stages every limb (spk <= 8: 32 KB)
  // + the zero slot (8 x 16 B); a prologue also keeps the slab limb counts and block totals
  const size_t lds = (size_t)Tc * spk * Lcap * 512 + 128 + (pers_pro ? 32 + 256 : 0);
  const int fr = (int)(frac > 63 ? 63 : frac);
  const dim3 grid((unsigned)((groups + 3) / 4), (unsigned)ksplit);
  dim3 pgrid = grid;
  if (pers) {
    static int cus_of[64] = {};
    int dev = 0;
    IMIE_HIP(hipGetDevice(&dev));
    int& cus = cus_of[dev & 63];
    if (cus == 0) IMIE_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    const int64_t cap = (int64_t)cus * pers_wpc;
    if ((int64_t)pgrid.x > cap) pgrid.x = (unsigned)cap;
  }
  const int mode = ksplit > 1 ? 1 : (accumulate ? 2 : 0);
  imie_prof_mark(IMIE_K_Q1_GEMV, st, true);
  for (int64_t t0 = 0; t0 < T; t0 += Tc) {
    const int tn = (int)(T - t0 < Tc ? T - t0 : Tc);
    Q1Segs sgt = sg;
    for (int i = 0; i < cnt; ++i) sgt.out[i] = outs[i] + t0 * ws[i]->N;
    const uint4* xq = (const uint4*)wk.xq.p + t0 * kMaxLimbs * nbp * 8;
    const int64_t* tot = (const int64_t*)wk.totals.p + t0 * nbp;
    const int* ls = (const int*)wk.lslab.p + t0 * nslabs;
#define IMIE_Q1_LAUNCH(S64_, R_, TT_)                                                                        \
  hipLaunchKernelGGL((q1_gemv_mfma_kernel<S64_, R_, TT_>), grid, dim3(256), lds, st, sgt, xq, tot, ls, nslabs,  \
                     nbp, tn, fr, spk, Lcap, mode, Q1Pro{})
#define IMIE_Q1_LAUNCH_R(S64_, TT_)                                                                          \
  if (R == 4) IMIE_Q1_LAUNCH(S64_, 4, TT_); else if (R == 2) IMIE_Q1_LAUNCH(S64_, 2, TT_); else IMIE_Q1_LAUNCH(S64_, 1, TT_)
#define IMIE_Q1_LAUNCH_T(S64_)                                                                               \
  if (TT == 1) { IMIE_Q1_LAUNCH_R(S64_, 1); } else if (TT == 2) { IMIE_Q1_LAUNCH_R(S64_, 2); }                 \
  else if (R == 2) { IMIE_Q1_LAUNCH(S64_, 2, 4); } else { IMIE_Q1_LAUNCH(S64_, 1, 4); }
#define IMIE_Q1_LAUNCH_PF(S64_, PF_)                                                                         \
  hipLaunchKernelGGL((q1_gemv_mfma_kernel<S64_, 1, 1, PF_>), grid, dim3(256), lds, st, sgt, xq, tot, ls, nslabs, \
                     nbp, tn, fr, spk, Lcap, mode, Q1Pro{})
    if (pers_pro) {
      Q1Pro pro = {};
      pro.x = x_dev;
      pro.cols = K;
      if (w0.scale64)
        hipLaunchKernelGGL((q1_gemv_mfma_kernel<true, 4, 1, 0, kProCopy, 256, true>), pgrid, dim3(256), lds, st, sgt,
                           nullptr, nullptr, nullptr, nslabs, nbp, tn, fr, spk, Lcap, mode, pro);
      else
        hipLaunchKernelGGL((q1_gemv_mfma_kernel<false, 4, 1, 0, kProCopy, 256, true>), pgrid, dim3(256), lds, st, sgt,
                           nullptr, nullptr, nullptr, nslabs, nbp, tn, fr, spk, Lcap, mode, pro);
    } else if (pers) {
      if (w0.scale64)
        hipLaunchKernelGGL((q1_gemv_mfma_kernel<true, 4, 1, 0, kProNone, 256, true>), pgrid, dim3(256), lds, st, sgt,
                           xq, tot, ls, nslabs, nbp, tn, fr, spk, Lcap, mode, Q1Pro{});
      else
        hipLaunchKernelGGL((q1_gemv_mfma_kernel<false, 4, 1, 0, kProNone, 256, true>), pgrid, dim3(256), lds, st, sgt,
                           xq, tot, ls, nslabs, nbp, tn, fr, spk, Lcap, mode, Q1Pro{});
    } else if (pf == 4) { if (w0.scale64) IMIE_Q1_LAUNCH_PF(true, 4); else IMIE_Q1_LAUNCH_PF(false, 4); }
    else if (pf == 2) { if (w0.scale64) IMIE_Q1_LAUNCH_PF(true, 2); else IMIE_Q1_LAUNCH_PF(false, 2); }
    else if (w0.scale64) { IMIE_Q1_LAUNCH_T(true); } else { IMIE_Q1_LAUNCH_T(false); }
#undef IMIE_Q1_LAUNCH_PF
#undef IMIE_Q1_LAUNCH_T
#undef IMIE_Q1_LAUNCH_R
#undef IMIE_Q1_LAUNCH
  }
  imie_prof_mark(IMIE_K_Q1_GEMV, st, false);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

// Single-token matvec whose workgroups build their own digit table from the producer's inputs (Q1Pro). The
// K-split outputs must already be clear (accumulate == 0: a kernel before this one cleared them) or are added to
// (accumulate != 0). Slab ranges of spk in {1, 2, 4, 8}: the largest that still leaves the target number of
// workgroups (q1_pro_target_wgs).
// Workgroups to aim for: a normalising prologue is repeated by every workgroup of a slab range, so RMSNorm launches
// take fewer, longer workgroups (twice the tile-group count, at least 192; measured on the 8B q/k/v and gate/up
// shapes), the cheap prologues 768 (IMIE_PRO_WGS overrides, tuning).
static int64_t q1_pro_target_wgs(int kind, int64_t wg_x) {
  static const int v = [] { const char* e = getenv("IMIE_PRO_WGS"); return e ? atoi(e) : 0; }();
  if (v > 0) return v;
  if (kind == kProNorm) return wg_x * 2 > 192 ? wg_x * 2 : 192;
  return 768;
}

static bool q1_pro_shape_ok(const Q1Weight* const* ws, int cnt, int kind, int64_t cols) {
  if (cnt < 1 || cnt > kMaxSegs || kind < kProCopy || kind > kProNorm) return false;
  for (int i = 0; i < cnt; ++i)
    if (ws[i]->scale64 || ws[i]->nb != ws[0]->nb) return false;
  if (ws[0]->nb * 128 != cols) return false;
  return kind != kProNorm || cols <= kProNormCols;
}

static int q1_apply_pro(const Q1Weight* const* ws, int cnt, const Q1Pro& pro, int kind, int64_t frac,
                        int64_t* const* outs, int accumulate, hipStream_t st) {
  if (!q1_pro_shape_ok(ws, cnt, kind, pro.cols)) return IMIE_EARG;
  const int64_t nslabs = ws[0]->nslabs, nbp = nslabs * kSlabBlocks;
  Q1Segs sg = {};
  sg.cnt = cnt;
  int64_t groups = 0;
  for (int i = 0; i < cnt; ++i) {
    sg.bits[i] = ws[i]->bits;
    sg.scale[i] = ws[i]->scale;
    sg.N[i] = ws[i]->N;
    sg.ntiles[i] = ws[i]->ntiles;
    sg.out[i] = outs[i];
    sg.gbegin[i] = groups;
    groups += ws[i]->ntiles;
  }
  sg.gbegin[cnt] = groups;
  constexpr int NT = 512;                            // 8 waves share one prologue (256 VGPRs per thread: no spills)
  const int64_t wg_x = (groups + NT / 64 - 1) / (NT / 64);
  int64_t spk = 1;
  for (int64_t c = 8; c >= 2; c >>= 1)
    if (wg_x * ((nslabs + c - 1) / c) >= q1_pro_target_wgs(kind, wg_x)) { spk = c; break; }
  if (spk > nslabs) spk = nslabs <= 1 ? 1 : (nslabs <= 2 ? 2 : (nslabs <= 4 ? 4 : 8));
  const int64_t ksplit = (nslabs + spk - 1) / spk;
  const int mode = ksplit > 1 ? 1 : (accumulate ? 2 : 0);
  const size_t lds = (size_t)spk * 8 * 512 + 128 + 32 + 256;   // table (values alias it), zero slot, L, totals
  const int fr = (int)(frac > 63 ? 63 : frac);
  const dim3 grid((unsigned)wg_x, (unsigned)ksplit);
  imie_prof_mark(IMIE_K_Q1_GEMV, st, true);
#define IMIE_Q1_PRO(PF_, PRO_)                                                                                 \
  hipLaunchKernelGGL((q1_gemv_mfma_kernel<false, 1, 1, PF_, PRO_, NT>), grid, dim3(NT), lds, st, sg, nullptr,   \
                     nullptr, nullptr, nslabs, nbp, 1, fr, spk, 8, mode, pro)
#define IMIE_Q1_PRO_K(PF_)                                                                                     \
  if (kind == kProCopy) IMIE_Q1_PRO(PF_, kProCopy);                                                           \
  else if (kind == kProSiluMul) IMIE_Q1_PRO(PF_, kProSiluMul);                                                \
  else IMIE_Q1_PRO(PF_, kProNorm)
  if (spk == 8) { IMIE_Q1_PRO_K(8); }
  else if (spk == 4) { IMIE_Q1_PRO_K(4); }
  else if (spk == 2) { IMIE_Q1_PRO_K(2); }
  else { IMIE_Q1_PRO_K(1); }
#undef IMIE_Q1_PRO_K
#undef IMIE_Q1_PRO
  imie_prof_mark(IMIE_K_Q1_GEMV, st, false);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

static int q1_apply_dev(const Q1Weight& w, const int64_t* x_dev, int64_t T, int64_t frac, int64_t* out_dev,
                        hipStream_t st, int accumulate = 0) {
  const Q1Weight* ws[1] = {&w};
  int64_t* outs[1] = {out_dev};
  return q1_apply_multi(ws, 1, x_dev, T, frac, outs, accumulate, g_ws.w, st);
}

static int64_t q1_register(const uint8_t* bits, const void* scale, int64_t N, int64_t nb, int src32) {
  if (!bits || !scale || N <= 0 || nb <= 0 || imie_device_ready() != 0) return -1;
  // narrow the scales to int32 when every value fits (lossless); keep int64 otherwise
  int scale64 = 0;
  uint64_t maxsc = 0;
  std::vector<int64_t> s64((size_t)(N * nb));
  for (int64_t i = 0; i < N * nb; ++i) {
    const int64_t v = src32 ? (int64_t)((const int32_t*)scale)[i] : ((const int64_t*)scale)[i];
    s64[(size_t)i] = v;
    if (v < INT32_MIN || v > INT32_MAX) scale64 = 1;
    const uint64_t av = v < 0 ? 0 - (uint64_t)v : (uint64_t)v;
    maxsc = av > maxsc ? av : maxsc;
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
  if (hipMalloc(&w.scale, hs.size()) != hipSuccess) { imie_free(w.bits); return -1; }
  if (hipMemcpy(w.bits, hb.data(), hb.size(), hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(w.scale, hs.data(), hs.size(), hipMemcpyHostToDevice) != hipSuccess) {
    imie_free(w.bits); imie_free(w.scale); return -1;
  }
  w.scale64 = scale64;
  w.maxsc = maxsc > (uint64_t)INT64_MAX ? INT64_MAX : (int64_t)maxsc;
  for (int64_t o = 0; o < N; ++o)                   // range sums of |scale| per row (saturating)
    for (int r = 1; r <= 8; ++r) {
      const int64_t rl = (nb + r - 1) / r;
      for (int64_t b0 = 0; b0 < nb; b0 += rl) {
        uint64_t sum = 0;
        for (int64_t b = b0; b < nb && b < b0 + rl; ++b) {
          const int64_t v = s64[(size_t)(o * nb + b)];
          const uint64_t av = v < 0 ? 0 - (uint64_t)v : (uint64_t)v;
          sum = sum + av < sum ? UINT64_MAX : sum + av;
        }
        w.rsum[r - 1] = sum > w.rsum[r - 1] ? sum : w.rsum[r - 1];
      }
    }
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

int imie_q1_launch(int64_t handle, const int64_t* x, int64_t T, int64_t frac, int64_t* out, int accumulate,
                   hipStream_t st) {
  const Q1Weight* w = q1_get(handle);
  if (!w) return IMIE_EARG;
  return q1_apply_dev(*w, x, T, frac, out, st, accumulate);
}

int imie_q1_launch_multi(const int64_t* handles, int cnt, const int64_t* x, int64_t T, int64_t frac,
                         int64_t* const* outs, int accumulate, Q1Ws* wk, hipStream_t st, int prepped) {
  if (cnt < 1 || cnt > kMaxSegs) return IMIE_EARG;
  const Q1Weight* ws[kMaxSegs];
  for (int i = 0; i < cnt; ++i)
    if (!(ws[i] = q1_get(handles[i]))) return IMIE_EARG;
  bool same = true;
  for (int i = 1; i < cnt; ++i) same = same && ws[i]->nb == ws[0]->nb && ws[i]->scale64 == ws[0]->scale64;
  Q1Ws& w = wk ? *wk : g_ws.w;
  if (same) return q1_apply_multi(ws, cnt, x, T, frac, outs, accumulate, w, st, prepped);
  for (int i = 0; i < cnt; ++i) {
    const int rc = q1_apply_multi(&ws[i], 1, x, T, frac, &outs[i], accumulate, w, st, prepped);
    if (rc) return rc;
  }
  return IMIE_OK;
}

int imie_q1_pro_ok(const int64_t* handles, int cnt, int kind, int64_t cols) {
  if (cnt < 1 || cnt > kMaxSegs) return 0;
  const Q1Weight* ws[kMaxSegs];
  for (int i = 0; i < cnt; ++i)
    if (!(ws[i] = q1_get(handles[i]))) return 0;
  return q1_pro_shape_ok(ws, cnt, kind, cols) ? 1 : 0;
}

int imie_q1_launch_pro(const int64_t* handles, int cnt, const Q1Pro& pro, int kind, int64_t frac,
                       int64_t* const* outs, int accumulate, hipStream_t st) {
  if (cnt < 1 || cnt > kMaxSegs) return IMIE_EARG;
  const Q1Weight* ws[kMaxSegs];
  for (int i = 0; i < cnt; ++i)
    if (!(ws[i] = q1_get(handles[i]))) return IMIE_EARG;
  return q1_apply_pro(ws, cnt, pro, kind, frac, outs, accumulate, st);
}

int imie_q1_gemm_splits(int64_t handle, int64_t T) {
  const Q1Weight* w = q1_get(handle);
  if (!w || T < kGemmMinT || T >= kPmMinT) return 0;
  if (T <= 64 && gemm_bt()) return 1;                // the batched-decode kernel adds into cleared outputs
  const int64_t ntt = (T + 63) / 64, nto = (w->N + 127) / 128;
  const int64_t tiles = ntt >= 8 ? 8 * ((ntt + 7) / 8) * nto : ntt * nto;
  return tiles < 256 && w->nb >= 8 ? 1 : 0;
}

int imie_q1_gemm_target(Q1Ws* wk, int64_t nb, int64_t T, GemmPrepOut* gp) {
  if (!wk || !gp || nb <= 0 || T < kGemmMinT) return IMIE_EARG;
  return gemm_table(*wk, nb, T, gp);
}

int imie_q1_prep_target(Q1Ws* wk, int64_t nb, int64_t T, Q1PrepOut* po) {
  if (!wk || !po || nb <= 0 || T <= 0) return IMIE_EARG;
  const int64_t nslabs = (nb + kSlabBlocks - 1) / kSlabBlocks, nbp = nslabs * kSlabBlocks;
  if (wk->xq.ensure((size_t)T * kMaxLimbs * nbp * 8 * 16) || wk->totals.ensure((size_t)T * nbp * 8) ||
      wk->lslab.ensure((size_t)T * nslabs * 4))
    return IMIE_EARG;
  *po = Q1PrepOut{(uint32_t*)wk->xq.p, (int64_t*)wk->totals.p, (int*)wk->lslab.p, nb, nbp, nslabs};
  return IMIE_OK;
}

int imie_q1_dims(int64_t handle, int64_t* N, int64_t* nb) {
  const Q1Weight* w = q1_get(handle);
  if (!w) return IMIE_EARG;
  *N = w->N;
  *nb = w->nb;
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
  imie_free(w.bits); imie_free(w.scale);
  if (w.signs) imie_free(w.signs);
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

// bonsai_q1_gpu.cu:2350-2366 `bonsai_q1_register_weight_i32_gpu_layout` (gpu_native.py:89-96, 286-306). The
// reference keeps a second, coalesced runtime layout for its CUDA kernels; here every registration is already the
// tile-major layout the gfx950 kernels stream (one wave reads 1 KB contiguous per tile and slab), so this is the
// int32 registration under the name its callers bind. Same refusals: null pointers or empty shapes give -1.
int64_t bonsai_q1_register_weight_i32_gpu_layout(const uint8_t* bits, const int32_t* scale, int64_t out_features,
                                                 int64_t n_blocks) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!bits || !scale || out_features <= 0 || n_blocks <= 0) return -1;
  return q1_register(bits, scale, out_features, n_blocks, 1);
}

// bonsai_q1_gpu.cu:2368-2385 `bonsai_q1_register_weight_i32_bmma` (gpu_native.py:98-105, 286-306): the reference's
// tensor-core layout needs out_features % 8 == 0 and refuses other shapes with -1; that refusal is kept so a
// caller sees the same handles, and the weight is stored in the same tile-major layout as every registration.
int64_t bonsai_q1_register_weight_i32_bmma(const uint8_t* bits, const int32_t* scale, int64_t out_features,
                                           int64_t n_blocks) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!bits || !scale || out_features <= 0 || n_blocks <= 0 || out_features % 8) return -1;
  return q1_register(bits, scale, out_features, n_blocks, 1);
}

// bonsai_q1_gpu.cu:2245-2300 `bonsai_q1_linear_dp4a_gpu` (gpu_native.py:55-64, called :235-261): the Q1 linear of
// x written as L balanced base-256 digits (|L| in 1..8; L < 0 selects the reference's warp variant, which gives
// the same bytes). Digits are taken from the low end exactly as bonsai_q1_gpu.cu:419-432 does, so for an x that
// needs more than L digits the result is the Q1 linear of the L-digit truncation (mod 2^64), as there; with
// L = 8 every int64 is exact. |L| == 4 refuses (rc 4, nothing computed) any |x| > 2,139,062,143, the reference's
// L=4 guard (:475-481). rc 1 on bad arguments. Here the digits are the kernels' own limb planes: the truncated
// activations are formed on the host only when some value does not fit L digits.
int bonsai_q1_linear_dp4a_gpu(const int64_t* x, const uint8_t* bits, const int64_t* scale, int64_t tokens,
                              int64_t out_features, int64_t n_blocks, int64_t frac, int L, int64_t* out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  const int LL = L < 0 ? -L : L;
  if (!x || !bits || !scale || !out || tokens <= 0 || out_features <= 0 || n_blocks <= 0 || LL < 1 || LL > 8 ||
      frac < 0)
    return IMIE_EARG;
  const size_t n = (size_t)(tokens * n_blocks * 128);
  const uint64_t cap = imie_balanced_cap(LL);
  bool fits = true;
  for (size_t i = 0; i < n && fits; ++i) {
    const uint64_t a = x[i] < 0 ? (uint64_t)0 - (uint64_t)x[i] : (uint64_t)x[i];
    fits = LL == 8 || a <= cap;
  }
  if (LL == 4 && !fits) return 4;
  if (fits) return bonsai_q1_linear_gpu(x, bits, scale, tokens, out_features, n_blocks, frac, out);
  std::vector<int64_t> xt(n);
  for (size_t i = 0; i < n; ++i) {
    uint64_t r = (uint64_t)x[i], acc = 0, w = 1;
    for (int l = 0; l < LL; ++l) {
      const int lb = (int)(r & 0xFFu);
      const int d = lb >= 128 ? lb - 256 : lb;
      acc += (uint64_t)(int64_t)d * w;
      w <<= 8;
      r = (r - (uint64_t)(int64_t)d) >> 8;
    }
    xt[i] = (int64_t)acc;
  }
  return bonsai_q1_linear_gpu(xt.data(), bits, scale, tokens, out_features, n_blocks, frac, out);
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
    if (w.live) { imie_free(w.bits); imie_free(w.scale); if (w.signs) imie_free(w.signs); }
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
  return q1_apply_dev(*w, x_dev, tokens, frac, out_dev, (hipStream_t)stream);
}

}  // extern "C"

// ---- fixed scratch for callers that cannot allocate ------------------------------------------------------
// The matvec path (T < kGemmMinT) keeps its per-call digit table (xq), block totals and slab limb counts in a
// workspace; imie_q1_apply_dev_noalloc takes that workspace from this file-scope array instead of the allocator.
// Sized for kNaMaxT tokens of up to kNaMaxSlabs 512-column slabs (K <= 32768). Each device holds its own copy for
// the life of the process; host code reaches it only through the address hipGetSymbolAddress gives on that device.
constexpr int64_t kNaMaxT = kGemmMinT - 1;
constexpr int64_t kNaMaxSlabs = 64;
constexpr size_t kNaXqBytes = (size_t)kNaMaxT * kMaxLimbs * (kNaMaxSlabs * kSlabBlocks) * 8 * 16;
constexpr size_t kNaTotBytes = (size_t)kNaMaxT * (kNaMaxSlabs * kSlabBlocks) * 8;
constexpr size_t kNaLsBytes = (size_t)kNaMaxT * kNaMaxSlabs * 4;
constexpr size_t kNaAlign(size_t b) { return (b + 255) / 256 * 256; }
constexpr size_t kNaBytes = kNaAlign(kNaXqBytes) + kNaAlign(kNaTotBytes) + kNaAlign(kNaLsBytes);
static __device__ __align__(256) uint8_t scratch[kNaBytes];

// this device's address of `scratch`, looked up once per device (nullptr if the lookup fails)
static uint8_t* na_scratch_ptr() {
  static std::vector<uint8_t*> per_dev;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return nullptr;
  if ((size_t)dev >= per_dev.size()) per_dev.resize((size_t)dev + 1, nullptr);
  if (!per_dev[(size_t)dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) { imie_note_error(e, "hipGetSymbolAddress(scratch)"); return nullptr; }
    per_dev[(size_t)dev] = (uint8_t*)p;
  }
  return per_dev[(size_t)dev];
}

extern "C" {

// imie_q1_apply_dev without any allocation (no reference counterpart): for callers that cannot call hipMalloc
// (graph capture, tight serving loops). tokens in 1..7 and n_blocks <= 256 (K <= 32768), else rc 1 with the reason
// in imie_last_error. The digit-table workspace is the fixed device array above, shared by every call on this
// device: calls that overlap on one device (two streams, two threads) race on it. Nothing in it must start at zero
// (each call writes every entry it reads), and the K-split outputs are cleared by the call's own prep kernel.
int imie_q1_apply_dev_noalloc(int64_t handle, const int64_t* x_dev, int64_t tokens, int64_t frac, int64_t* out_dev,
                              void* stream) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  const Q1Weight* w = q1_get(handle);
  if (!w || !x_dev || !out_dev || tokens < 0 || frac < 0) return IMIE_EARG;
  if (tokens == 0) return IMIE_OK;
  if (tokens > kNaMaxT || w->nslabs > kNaMaxSlabs) {
    imie_note_message("imie_q1_apply_dev_noalloc: at most 7 tokens and 32768 input columns fit its fixed scratch");
    return IMIE_EARG;
  }
  uint8_t* base = na_scratch_ptr();
  if (!base) return IMIE_EARG;
  Q1Ws wk;                                            // views into the fixed array: ensure() never allocates here
  wk.xq.p = base;
  wk.xq.cap = kNaXqBytes;
  wk.totals.p = base + kNaAlign(kNaXqBytes);
  wk.totals.cap = kNaTotBytes;
  wk.lslab.p = base + kNaAlign(kNaXqBytes) + kNaAlign(kNaTotBytes);
  wk.lslab.cap = kNaLsBytes;
  const Q1Weight* ws[1] = {w};
  int64_t* outs[1] = {out_dev};
  const bool prof = imie_prof_suspend(true);          // the profiler's per-kernel events are created on demand
  const int rc = q1_apply_multi(ws, 1, x_dev, tokens, frac, outs, 0, wk, (hipStream_t)stream);
  imie_prof_suspend(prof);
  return rc;
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
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(q1_linear_simple_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x_dev,
                     bits_dev, scale_dev, tokens, out_features, n_blocks, (int)(frac > 63 ? 63 : frac), out_dev);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

}  // extern "C"
