// Integer samplers over fixed-point logits rows, on the device (gfx950). Semantics follow
// bonsai/src/trinote/infer_int/sampler.py:
//   repetition penalty / n-gram ban   apply_rep_penalty :182-211 (ban value :176)
//   temperature                       _apply_temp_fp :261-275 (fail-loud int64 guard)
//   probabilities                     _probs_fp :318-323 over fixedpoint.py:99-140
//   top-k / nucleus                   _truncate :351-381 (stable descending order: ties keep the higher token id)
//   min-p                             _truncate_min_p :384-400
//   seeded draw                       _prng_word / draw_uniform_int :283-315 (SHA-256 counter word, Lemire)
//   token                             sample_token :403-437
// The reference's own device sampler (bonsai/tools/bonsai_q1_gpu.cu:905-1042, :3342-3418) runs one serial thread
// per row and draws the target on the host. Here every vocabulary pass is spread over 64 workgroups per row, the
// top-k / nucleus order comes from a segmented radix sort of unique (probability, token id) keys (any sort of
// unique keys yields the reference's tie order), and the SHA-256 draw runs on the device, so a sampled decode
// step needs no logits row on the host and can be captured in a graph.
#include "imie_common.h"
#include "imie_kernels.h"
#include <hipcub/device/device_segmented_radix_sort.hpp>

namespace {

typedef unsigned __int128 u128;
constexpr int kSmpParts = 64;                        // workgroups per row for the vocabulary passes
constexpr int kSmpScan = 1024;                       // threads of the one-workgroup-per-row scans

struct SmpRow {                                       // per-row sampler state (device)
  int64_t best, best_tok, best_s;                     // adjusted max (first index) and its temperature-scaled value
  uint64_t peak, z, sum, maxp;
  int64_t amax, thresh, total;
  int done;                                           // token already decided (greedy, guard, degenerate)
  int pad;
};

__device__ inline int64_t smp_rshift(int64_t a, int64_t s) {   // numpy int64 `a >> s` incl. out-of-range counts
  if (s < 0 || s >= 64) return a < 0 ? -1 : 0;
  return a >> s;
}

// 2^-(u / 2^frac): cubic polynomial on the fraction, shift by the integer part (fixedpoint.py:74-96)
__device__ inline int64_t smp_exp2_neg(int64_t u, int frac) {
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
  return smp_rshift(poly, k < 63 ? k : 63);
}

__device__ inline int64_t smp_floor_div(int64_t n, int64_t d) {   // d > 0
  const int64_t q = n / d, r = n % d;
  return r < 0 ? q - 1 : q;
}

__device__ inline int64_t smp_scale(int64_t v, const ImieSamplerConfig& c) {   // (v * inv_temp) >> frac, int64 wrap
  return (int64_t)((uint64_t)v * (uint64_t)c.inv_temp) >> c.frac;
}

// (value, index) max with the lower index on ties (numpy first-max)
__device__ inline void smp_amx(int64_t& v, int64_t& i, int64_t v2, int64_t i2) {
  if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
}

// workgroup reductions (256 threads): first-max and u64 sum / max
__device__ inline void smp_block_amx(int64_t& v, int64_t& i) {
  __shared__ int64_t sv[4], si[4];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) smp_amx(v, i, __shfl_xor(v, o, 64), __shfl_xor(i, o, 64));
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) { sv[w] = v; si[w] = i; }
  __syncthreads();
  if (threadIdx.x == 0)
    for (int k = 1; k < (int)(blockDim.x >> 6); ++k) smp_amx(v, i, sv[k], si[k]);
}

template <bool MAX>
__device__ inline uint64_t smp_block_u64(uint64_t v) {
  __shared__ uint64_t s[16];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint64_t u = (uint64_t)__shfl_xor((long long)v, o, 64);
    v = MAX ? (u > v ? u : v) : v + u;
  }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) s[w] = v;
  __syncthreads();
  if (threadIdx.x == 0)
    for (int k = 1; k < (int)(blockDim.x >> 6); ++k) v = MAX ? (s[k] > v ? s[k] : v) : v + s[k];
  return v;                                           // valid in thread 0
}

// exclusive prefix of per-thread u64 values over a kSmpScan-thread workgroup
__device__ inline uint64_t smp_block_excl(uint64_t v, uint64_t* total) {
  __shared__ uint64_t s[kSmpScan / 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  uint64_t inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t u = (uint64_t)__shfl_up((long long)inc, o, 64);
    if (lane >= o) inc += u;
  }
  __syncthreads();
  if (lane == 63) s[w] = inc;
  __syncthreads();
  uint64_t before = 0, all = 0;
  for (int k = 0; k < kSmpScan / 64; ++k) {
    if (k < w) before += s[k];
    all += s[k];
  }
  *total = all;
  return before + inc - v;
}

// ---- SHA-256 (FIPS 180-4) of the 47-byte draw message, one 64-byte block -----------------------------------
__constant__ uint32_t kSha256K[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};

__device__ inline uint32_t smp_rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

// SHA-256 over one padded block (w[16] big-endian message words); returns the first 8 digest bytes as a
// big-endian u64
__device__ inline uint64_t smp_sha256_first8(const uint32_t m[16]) {
  uint32_t w[64];
#pragma unroll
  for (int i = 0; i < 16; ++i) w[i] = m[i];
  for (int i = 16; i < 64; ++i) {
    const uint32_t s0 = smp_rotr(w[i - 15], 7) ^ smp_rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
    const uint32_t s1 = smp_rotr(w[i - 2], 17) ^ smp_rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
    w[i] = w[i - 16] + s0 + w[i - 7] + s1;
  }
  uint32_t a = 0x6a09e667, b = 0xbb67ae85, c = 0x3c6ef372, d = 0xa54ff53a;
  uint32_t e = 0x510e527f, f = 0x9b05688c, g = 0x1f83d9ab, h = 0x5be0cd19;
  for (int i = 0; i < 64; ++i) {
    const uint32_t S1 = smp_rotr(e, 6) ^ smp_rotr(e, 11) ^ smp_rotr(e, 25);
    const uint32_t ch = (e & f) ^ (~e & g);
    const uint32_t t1 = h + S1 + ch + kSha256K[i] + w[i];
    const uint32_t S0 = smp_rotr(a, 2) ^ smp_rotr(a, 13) ^ smp_rotr(a, 22);
    const uint32_t mj = (a & b) ^ (a & c) ^ (b & c);
    const uint32_t t2 = S0 + mj;
    h = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
  }
  return ((uint64_t)(0x6a09e667u + a) << 32) | (uint64_t)(0xbb67ae85u + b);
}

// One SHA-256 compression of a 64-byte block (w[0..15] big-endian message words) into the running state
__device__ inline void smp_sha256_compress(uint32_t st[8], uint32_t w[16]) {
  uint32_t a = st[0], b = st[1], c = st[2], d = st[3], e = st[4], f = st[5], g = st[6], h = st[7];
#pragma unroll
  for (int i = 0; i < 64; ++i) {
    uint32_t wi;
    if (i < 16) {
      wi = w[i];
    } else {                                          // rolling 16-word schedule
      const uint32_t w15 = w[(i - 15) & 15], w2 = w[(i - 2) & 15];
      const uint32_t s0 = smp_rotr(w15, 7) ^ smp_rotr(w15, 18) ^ (w15 >> 3);
      const uint32_t s1 = smp_rotr(w2, 17) ^ smp_rotr(w2, 19) ^ (w2 >> 10);
      wi = w[i & 15] + s0 + w[(i - 7) & 15] + s1;
      w[i & 15] = wi;
    }
    const uint32_t S1 = smp_rotr(e, 6) ^ smp_rotr(e, 11) ^ smp_rotr(e, 25);
    const uint32_t ch = (e & f) ^ (~e & g);
    const uint32_t t1 = h + S1 + ch + kSha256K[i] + wi;
    const uint32_t S0 = smp_rotr(a, 2) ^ smp_rotr(a, 13) ^ smp_rotr(a, 22);
    const uint32_t mj = (a & b) ^ (a & c) ^ (b & c);
    h = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + S0 + mj;
  }
  st[0] += a; st[1] += b; st[2] += c; st[3] += d; st[4] += e; st[5] += f; st[6] += g; st[7] += h;
}

// logits_digest (sampler.py:421-425): SHA-256 of a row's little-endian int64 bytes, one lane per row. The
// message is vocab * 8 bytes, so whole 8-byte values fill the blocks and the tail holds 0..7 values.
__global__ __launch_bounds__(64) void smp_digest_kernel(const int64_t* __restrict__ x, int64_t rows, int64_t vocab,
                                                        int64_t ld, uint32_t* __restrict__ out) {
  const int64_t r = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (r >= rows) return;
  const uint64_t* p = reinterpret_cast<const uint64_t*>(x + r * ld);
  uint32_t st[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                    0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
  uint32_t w[16];
  const int64_t full = vocab / 8;                     // 8 values = one 64-byte block
  for (int64_t blk = 0; blk < full; ++blk) {
    uint64_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = __builtin_nontemporal_load(p + blk * 8 + j);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      w[2 * j] = __builtin_bswap32((uint32_t)v[j]);
      w[2 * j + 1] = __builtin_bswap32((uint32_t)(v[j] >> 32));
    }
    smp_sha256_compress(st, w);
  }
  const int tail = (int)(vocab - full * 8);           // 0..7 values left
#pragma unroll
  for (int j = 0; j < 8; ++j) {                       // static indices keep w in registers
    const uint64_t v = j < tail ? p[full * 8 + j] : 0;
    w[2 * j] = j < tail ? __builtin_bswap32((uint32_t)v) : (j == tail ? 0x80000000u : 0u);   // 0x80 pad byte
    w[2 * j + 1] = j < tail ? __builtin_bswap32((uint32_t)(v >> 32)) : 0u;
  }
  const uint64_t bits = (uint64_t)vocab * 64;
  if (tail >= 7) {                                    // no room for the 8-byte length: one more block
    smp_sha256_compress(st, w);
#pragma unroll
    for (int j = 0; j < 16; ++j) w[j] = 0;
  }
  w[14] = (uint32_t)(bits >> 32);
  w[15] = (uint32_t)bits;
  smp_sha256_compress(st, w);
#pragma unroll
  for (int j = 0; j < 8; ++j) out[r * 8 + j] = __builtin_bswap32(st[j]);   // digest bytes in order
}

// "trinote-sampler-draw/v1" || seed || position || counter (8 bytes each, big-endian), SHA-256, first 8 bytes
__device__ inline uint64_t smp_prng_word(uint64_t seed, uint64_t pos, uint64_t ctr) {
  uint8_t msg[64];
  const char tag[] = "trinote-sampler-draw/v1";
#pragma unroll
  for (int i = 0; i < 23; ++i) msg[i] = (uint8_t)tag[i];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    msg[23 + i] = (uint8_t)(seed >> (56 - 8 * i));
    msg[31 + i] = (uint8_t)(pos >> (56 - 8 * i));
    msg[39 + i] = (uint8_t)(ctr >> (56 - 8 * i));
  }
  msg[47] = 0x80;
#pragma unroll
  for (int i = 48; i < 62; ++i) msg[i] = 0;
  msg[62] = (uint8_t)((47 * 8) >> 8);
  msg[63] = (uint8_t)((47 * 8) & 0xFF);
  uint32_t m[16];
#pragma unroll
  for (int i = 0; i < 16; ++i)
    m[i] = ((uint32_t)msg[4 * i] << 24) | ((uint32_t)msg[4 * i + 1] << 16) | ((uint32_t)msg[4 * i + 2] << 8) |
           (uint32_t)msg[4 * i + 3];
  return smp_sha256_first8(m);
}

// unbiased integer in [0, n) by Lemire's multiply-shift over the counter words (draw_uniform_int)
__device__ inline int64_t smp_draw(uint64_t n, uint64_t seed, uint64_t pos) {
  if (n <= 1) return 0;
  uint64_t j = 0;
  u128 m = (u128)smp_prng_word(seed, pos, j++) * n;
  uint64_t low = (uint64_t)m;
  if (low < n) {
    const uint64_t t = (0 - n) % n;                   // 2^64 mod n
    while (low < t) {
      m = (u128)smp_prng_word(seed, pos, j++) * n;
      low = (uint64_t)m;
    }
  }
  return (int64_t)(uint64_t)(m >> 64);
}

// ---- kernels ------------------------------------------------------------------------------------------------
// history flags: rep[t] for every seen token, ban[t] for every n-gram continuation (val 1 to set, 0 to clear)
__global__ __launch_bounds__(256) void smp_flags_kernel(ImieSamplerConfig c, const int64_t* __restrict__ hist,
                                                        int64_t hld, const int64_t* __restrict__ hlen, int64_t V,
                                                        uint8_t* __restrict__ rep, uint8_t* __restrict__ ban,
                                                        uint8_t val, int* __restrict__ status) {
  const int64_t r = blockIdx.y, i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  int64_t len = hlen[r];
  len = len < 0 ? 0 : (len > hld ? hld : len);
  if (i >= len) return;
  const int64_t* h = hist + r * hld;
  const int64_t t = h[i];
  if (t < 0 || t >= V) {
    if (val) atomicOr(status, IMIE_EARG);
    return;
  }
  if (c.rep_penalty) rep[r * V + t] = val;
  const int64_t n = c.no_repeat_ngram;
  if (n > 1 && len >= n && i <= len - n) {
    bool match = true;
    for (int64_t j = 0; j < n - 1 && match; ++j) match = h[i + j] == h[len - (n - 1) + j];
    const int64_t nx = h[i + n - 1];
    if (match && nx >= 0 && nx < V) ban[r * V + nx] = val;
  }
}

// adjusted row (penalty, ban) into adj; per-part first-max and peak |value|
__global__ __launch_bounds__(256) void smp_adjust_kernel(ImieSamplerConfig c, const int64_t* __restrict__ logits,
                                                         int64_t ld, int64_t V, const uint8_t* __restrict__ rep,
                                                         const uint8_t* __restrict__ ban, int has_hist,
                                                         int64_t* __restrict__ adj, int64_t* __restrict__ part) {
  const int64_t r = blockIdx.y, per = (V + kSmpParts - 1) / kSmpParts;
  const int64_t c0 = (int64_t)blockIdx.x * per, c1 = min(V, c0 + per);
  const int64_t fp = (int64_t)1 << c.frac, den = fp + c.rep_penalty;
  int64_t bv = INT64_MIN, bi = INT64_MAX;
  uint64_t peak = 0;
  for (int64_t k = c0 + threadIdx.x; k < c1; k += 256) {
    int64_t v = logits[r * ld + k];
    if (has_hist) {
      if (c.rep_penalty && rep[r * V + k]) {
        const int64_t prod = v >= 0 ? (int64_t)((uint64_t)v * (uint64_t)fp) : (int64_t)((uint64_t)v * (uint64_t)den);
        v = smp_floor_div(prod, v >= 0 ? den : fp);
      }
      if (ban[r * V + k]) v = -((int64_t)1 << 40);
    }
    adj[r * V + k] = v;
    smp_amx(bv, bi, v, k);
    const uint64_t a = v < 0 ? 0 - (uint64_t)v : (uint64_t)v;
    peak = a > peak ? a : peak;
  }
  smp_block_amx(bv, bi);
  peak = smp_block_u64<true>(peak);
  if (threadIdx.x == 0) {
    int64_t* p = part + (r * kSmpParts + blockIdx.x) * 4;
    p[0] = bv; p[1] = bi; p[2] = (int64_t)peak;
  }
}

// row stats after the adjust pass: argmax, the temperature guard, the scaled max
__global__ void smp_stats1_kernel(ImieSamplerConfig c, const int64_t* __restrict__ part, SmpRow* __restrict__ st,
                                  int64_t* __restrict__ token, int* __restrict__ status) {
  const int64_t r = blockIdx.x;
  if (threadIdx.x) return;
  int64_t bv = INT64_MIN, bi = INT64_MAX;
  uint64_t peak = 0;
  for (int k = 0; k < kSmpParts; ++k) {
    const int64_t* p = part + (r * kSmpParts + k) * 4;
    if (p[1] != INT64_MAX) smp_amx(bv, bi, p[0], p[1]);
    peak = (uint64_t)p[2] > peak ? (uint64_t)p[2] : peak;
  }
  SmpRow s = {};
  s.best = bv; s.best_tok = bi == INT64_MAX ? 0 : bi; s.peak = peak;
  if (c.mode == 0) {
    s.done = 1;
    token[r] = s.best_tok;
  } else if ((u128)peak * (u128)(uint64_t)c.inv_temp >= ((u128)1 << 63)) {   // _apply_temp_fp guard
    s.done = 1;
    token[r] = s.best_tok;
    atomicOr(status, IMIE_EOVF);
  } else {
    s.best_s = c.inv_temp != ((int64_t)1 << c.frac) ? smp_scale(bv, c) : bv;   // the scaling is monotone
  }
  st[r] = s;
}

// e = 2^-(min(m - s, d_clip) * log2e >> frac) in place of adj; per-part sums
__global__ __launch_bounds__(256) void smp_exp_kernel(ImieSamplerConfig c, int64_t V, const SmpRow* __restrict__ st,
                                                      int64_t log2e, int64_t dclip, int64_t* __restrict__ pr,
                                                      int64_t* __restrict__ part) {
  const int64_t r = blockIdx.y, per = (V + kSmpParts - 1) / kSmpParts;
  if (st[r].done) return;
  const int64_t c0 = (int64_t)blockIdx.x * per, c1 = min(V, c0 + per);
  const bool temp = c.inv_temp != ((int64_t)1 << c.frac);
  const int64_t m = st[r].best_s;
  uint64_t z = 0;
  for (int64_t k = c0 + threadIdx.x; k < c1; k += 256) {
    int64_t s = pr[r * V + k];
    if (temp) s = smp_scale(s, c);
    int64_t d = (int64_t)((uint64_t)m - (uint64_t)s);
    if (d > dclip) d = dclip;
    const int64_t e = smp_exp2_neg((int64_t)((uint64_t)d * (uint64_t)log2e) >> c.frac, (int)c.frac);
    pr[r * V + k] = e;
    z += (uint64_t)e;
  }
  z = smp_block_u64<false>(z);
  if (threadIdx.x == 0) part[(r * kSmpParts + blockIdx.x) * 4] = (int64_t)z;
}

__global__ void smp_sum_kernel(const int64_t* __restrict__ part, SmpRow* __restrict__ st, int which) {
  const int64_t r = blockIdx.x;
  if (threadIdx.x || st[r].done) return;
  uint64_t z = 0;
  for (int k = 0; k < kSmpParts; ++k) z += (uint64_t)part[(r * kSmpParts + k) * 4];
  if (which == 0) st[r].z = z;
  else {                                              // after the min-p pass
    st[r].total = (int64_t)z;
  }
}

// p = (e << frac) // Z; per-part sum and first-max of p
__global__ __launch_bounds__(256) void smp_prob_kernel(ImieSamplerConfig c, int64_t V, const SmpRow* __restrict__ st,
                                                       int64_t* __restrict__ pr, int64_t* __restrict__ part) {
  const int64_t r = blockIdx.y, per = (V + kSmpParts - 1) / kSmpParts;
  if (st[r].done) return;
  const int64_t c0 = (int64_t)blockIdx.x * per, c1 = min(V, c0 + per);
  const uint64_t z = st[r].z;
  uint64_t sum = 0;
  int64_t bv = INT64_MIN, bi = INT64_MAX;
  for (int64_t k = c0 + threadIdx.x; k < c1; k += 256) {
    const int64_t p = z ? (int64_t)(((uint64_t)pr[r * V + k] << c.frac) / z) : 0;
    pr[r * V + k] = p;
    sum += (uint64_t)p;
    smp_amx(bv, bi, p, k);
  }
  smp_block_amx(bv, bi);
  sum = smp_block_u64<false>(sum);
  if (threadIdx.x == 0) {
    int64_t* p = part + (r * kSmpParts + blockIdx.x) * 4;
    p[0] = bv; p[1] = bi; p[2] = (int64_t)sum;
  }
}

__global__ void smp_stats3_kernel(ImieSamplerConfig c, const int64_t* __restrict__ part, SmpRow* __restrict__ st) {
  const int64_t r = blockIdx.x;
  if (threadIdx.x || st[r].done) return;
  int64_t bv = INT64_MIN, bi = INT64_MAX;
  uint64_t sum = 0;
  for (int k = 0; k < kSmpParts; ++k) {
    const int64_t* p = part + (r * kSmpParts + k) * 4;
    if (p[1] != INT64_MAX) smp_amx(bv, bi, p[0], p[1]);
    sum += (uint64_t)p[2];
  }
  SmpRow& s = st[r];
  s.sum = sum; s.maxp = (uint64_t)bv; s.amax = bi == INT64_MAX ? 0 : bi;
  s.total = (int64_t)sum;
  s.thresh = -1;                                      // no min-p pass
  if (c.mode == 4 && c.min_p > 0 && bv > 0) s.thresh = (int64_t)(((uint64_t)c.min_p * (uint64_t)bv) >> c.frac);
}

// min-p: zero p < threshold (threshold relative to the top probability); per-part sums
__global__ __launch_bounds__(256) void smp_minp_kernel(int64_t V, const SmpRow* __restrict__ st,
                                                       int64_t* __restrict__ pr, int64_t* __restrict__ part) {
  const int64_t r = blockIdx.y, per = (V + kSmpParts - 1) / kSmpParts;
  if (st[r].done || st[r].thresh < 0) return;
  const int64_t c0 = (int64_t)blockIdx.x * per, c1 = min(V, c0 + per);
  const int64_t th = st[r].thresh;
  uint64_t sum = 0;
  for (int64_t k = c0 + threadIdx.x; k < c1; k += 256) {
    int64_t p = pr[r * V + k];
    if (p < th) { p = 0; pr[r * V + k] = 0; }
    sum += (uint64_t)p;
  }
  sum = smp_block_u64<false>(sum);
  if (threadIdx.x == 0) part[(r * kSmpParts + blockIdx.x) * 4] = (int64_t)sum;
}

__global__ void smp_minp_final_kernel(const int64_t* __restrict__ part, SmpRow* __restrict__ st,
                                      int64_t* __restrict__ pr, int64_t V) {
  const int64_t r = blockIdx.x;
  if (threadIdx.x || st[r].done || st[r].thresh < 0) return;
  uint64_t sum = 0;
  for (int k = 0; k < kSmpParts; ++k) sum += (uint64_t)part[(r * kSmpParts + k) * 4];
  if (sum == 0) { pr[r * V + st[r].amax] = 1; sum = 1; }   // never an all-zero distribution
  st[r].total = (int64_t)sum;
}

// keys for the descending order: (p << 32) | token id, unique, so any sort reproduces the reference's ties. Only
// nonzero probabilities are keyed (compacted per row): a zero-probability token adds nothing to the kept total
// or to the draw whether it is kept or not, and the all-zero fallback (the highest id) is handled directly.
__global__ __launch_bounds__(256) void smp_count_kernel(int64_t V, const SmpRow* __restrict__ st,
                                                        const int64_t* __restrict__ pr, int64_t* __restrict__ part) {
  const int64_t r = blockIdx.y, per = (V + kSmpParts - 1) / kSmpParts;
  const int64_t c0 = (int64_t)blockIdx.x * per, c1 = min(V, c0 + per);
  uint64_t n = 0;
  if (!st[r].done)
    for (int64_t k = c0 + threadIdx.x; k < c1; k += 256) n += pr[r * V + k] != 0;
  n = smp_block_u64<false>(n);
  if (threadIdx.x == 0) part[(r * kSmpParts + blockIdx.x) * 4 + 3] = (int64_t)n;
}

// per-row exclusive offsets of the parts' nonzero counts (part[.. + 3] <- offset) and the sort segment ends
__global__ void smp_offsets_kernel(int64_t V, int64_t* __restrict__ part, int* __restrict__ seg_beg,
                                   int* __restrict__ seg_end) {
  const int64_t r = blockIdx.x;
  if (threadIdx.x) return;
  seg_beg[r] = (int)(r * V);
  int64_t run = 0;
  for (int k = 0; k < kSmpParts; ++k) {
    int64_t* p = part + (r * kSmpParts + k) * 4 + 3;
    const int64_t n = *p;
    *p = run;
    run += n;
  }
  seg_end[r] = (int)(r * V + run);
}

__global__ __launch_bounds__(256) void smp_scatter_kernel(int64_t V, const SmpRow* __restrict__ st,
                                                          const int64_t* __restrict__ pr,
                                                          const int64_t* __restrict__ part, uint64_t* __restrict__ keys) {
  __shared__ int s_base;
  __shared__ int s_w[4];
  const int64_t r = blockIdx.y, per = (V + kSmpParts - 1) / kSmpParts;
  if (st[r].done) return;
  const int64_t c0 = (int64_t)blockIdx.x * per, c1 = min(V, c0 + per);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (threadIdx.x == 0) s_base = (int)part[(r * kSmpParts + blockIdx.x) * 4 + 3];
  __syncthreads();
  for (int64_t k0 = c0; k0 < c1; k0 += 256) {       // order-preserving compaction, 256 ids per step
    const int64_t k = k0 + threadIdx.x;
    const int64_t p = k < c1 ? pr[r * V + k] : 0;
    const uint64_t m = __ballot(p != 0);
    const int before = __popcll(m & ((1ull << lane) - 1));
    if (lane == 0) s_w[w] = __popcll(m);
    __syncthreads();
    int wb = 0, tot = 0;
    for (int i = 0; i < 4; ++i) { if (i < w) wb += s_w[i]; tot += s_w[i]; }
    if (p != 0) keys[r * V + s_base + wb + before] = ((uint64_t)p << 32) | (uint64_t)k;
    __syncthreads();
    if (threadIdx.x == 0) s_base += tot;
    __syncthreads();
  }
}

// top-k / nucleus over the sorted keys (one workgroup per row): keep the first `keep` ranks, where the nucleus
// ends at the first rank whose running sum reaches top_p (that rank included); zero the rest; total of the kept
__global__ __launch_bounds__(kSmpScan) void smp_trunc_kernel(ImieSamplerConfig c, int64_t V,
                                                             const uint64_t* __restrict__ sorted,
                                                             const int* __restrict__ seg_end,
                                                             SmpRow* __restrict__ st, int64_t* __restrict__ pr) {
  __shared__ int64_t s_nuc;
  const int64_t r = blockIdx.x;
  if (st[r].done) return;
  const uint64_t* sk = sorted + r * V;
  const int64_t nnz = (int64_t)seg_end[r] - r * V;    // ranks past nnz hold zero probabilities
  int64_t keep = c.top_k > 0 ? (c.top_k < V ? c.top_k : V) : V;
  if (keep > nnz) keep = nnz;
  const int t = threadIdx.x;
  if (t == 0) s_nuc = INT64_MAX;
  __syncthreads();
  if (c.top_p < ((int64_t)1 << c.frac)) {
    const int64_t S = (keep + kSmpScan - 1) / kSmpScan, a = (int64_t)t * S, b = min(keep, a + S);
    uint64_t ts = 0;
    for (int64_t k = a; k < b; ++k) ts += sk[k] >> 32;
    uint64_t all;
    const uint64_t ex = smp_block_excl(ts, &all);
    const uint64_t tp = (uint64_t)c.top_p;
    if (ex < tp && ex + ts >= tp) {                   // the crossing rank lies in this thread's ranks
      uint64_t run = ex;
      for (int64_t k = a; k < b; ++k) {
        run += sk[k] >> 32;
        if (run >= tp) { s_nuc = k; break; }
      }
    }
    __syncthreads();
    if (s_nuc != INT64_MAX && s_nuc + 1 < keep) keep = s_nuc + 1;
  }
  // zero the dropped nonzero ranks and sum the kept probabilities
  uint64_t kept = 0;
  for (int64_t k = t; k < nnz; k += kSmpScan) {
    const int64_t id = (int64_t)(sk[k] & 0xFFFFFFFFu);
    if (k < keep) kept += sk[k] >> 32;
    else pr[r * V + id] = 0;
  }
  __syncthreads();
  uint64_t total;
  (void)smp_block_excl(kept, &total);
  if (t == 0) {
    if (total == 0) { pr[r * V + V - 1] = 1; total = 1; }   // all zero: the first rank is the highest id
    st[r].total = (int64_t)total;
  }
}

// seeded draw and selection (one workgroup per row): target = Lemire(total, seed, position); token = the first
// id whose running probability sum exceeds the target
__global__ __launch_bounds__(kSmpScan) void smp_select_kernel(ImieSamplerConfig c, int64_t V,
                                                              const int64_t* __restrict__ pos, SmpRow* __restrict__ st,
                                                              const int64_t* __restrict__ pr, int64_t* __restrict__ token) {
  __shared__ int64_t s_target, s_tok;
  const int64_t r = blockIdx.x;
  if (st[r].done) return;
  const int t = threadIdx.x;
  if (t == 0) {
    s_tok = -1;
    const int64_t total = st[r].total;
    s_target = total <= 0 ? -1 : smp_draw((uint64_t)total, (uint64_t)c.seed, (uint64_t)pos[r]);
  }
  __syncthreads();
  const int64_t target = s_target;
  if (target < 0) {                                   // degenerate distribution: the adjusted argmax
    if (t == 0) token[r] = st[r].best_tok;
    return;
  }
  const int64_t* p = pr + r * V;
  const int64_t S = (V + kSmpScan - 1) / kSmpScan, a = (int64_t)t * S, b = min(V, a + S);
  uint64_t ts = 0;
  for (int64_t k = a; k < b; ++k) ts += (uint64_t)p[k];
  uint64_t all;
  const uint64_t ex = smp_block_excl(ts, &all);
  if (ex <= (uint64_t)target && (uint64_t)target < ex + ts) {
    uint64_t run = ex;
    for (int64_t k = a; k < b; ++k) {
      run += (uint64_t)p[k];
      if (run > (uint64_t)target) { s_tok = k; break; }
    }
  }
  __syncthreads();
  if (t == 0) token[r] = s_tok >= 0 ? s_tok : st[r].best_tok;
}

struct SmpWs {
  DevBuf rep, ban, pr, part, st, keys, sorted, offs, tmp;
  int64_t cap_rv = 0;
} g_smp;

int64_t smp_log2e(int frac) {
  const int sh = 16 - frac;
  return sh >= 0 ? (94548 >> sh) : ((int64_t)94548 << -sh);
}

int64_t smp_dclip(int frac) {
  const int64_t l = smp_log2e(frac);
  const int64_t a = ((int64_t)(frac + 2) << (2 * frac)) / l, b = ((int64_t)1 << 62) / l;
  return a < b ? a : b;
}

// the reference ABI's envelope (bonsai_q1_gpu.cu:3349-3354) plus validate_sampler_config (sampler.py:71-91)
bool smp_config_ok(const ImieSamplerConfig& c) {
  if (c.frac < 1 || c.frac > 29 || c.mode < 0 || c.mode > 4) return false;
  const int64_t fp = (int64_t)1 << c.frac;
  if (c.inv_temp <= 0 || c.top_k < 0 || c.min_p < 0 || c.min_p > fp ||
      c.rep_penalty < 0 || c.no_repeat_ngram < 0)
    return false;
  if (c.mode == 2 && c.top_k <= 0) return false;
  if (c.mode == 4 && c.min_p <= 0) return false;
  return true;
}

}  // namespace

int imie_sample_launch(const int64_t* logits, int64_t rows, int64_t V, int64_t ld, const ImieSamplerConfig& c_in,
                       const int64_t* hist, int64_t hld, const int64_t* hlen, const int64_t* pos, int64_t* token,
                       int* status, hipStream_t st) {
  // The nucleus threshold only acts in top_k / top_p modes (sampler.py:403-437 passes it to _truncate there only),
  // so other modes take 2^frac whatever the config carries. Within those modes _truncate (sampler.py:334-363)
  // keeps the first token for any threshold <= 0 (exactly what threshold 1 keeps, the top probability being >= 1
  // whenever the total is positive) and truncates nothing for a threshold >= 2^frac: clamp to [1, 2^frac].
  ImieSamplerConfig c = c_in;
  if (c.frac >= 1 && c.frac <= 29) {
    const int64_t fp = (int64_t)1 << c.frac;
    c.top_p = (c.mode == 2 || c.mode == 3) ? (c.top_p < 1 ? 1 : (c.top_p > fp ? fp : c.top_p)) : fp;
  }
  if (!logits || rows <= 0 || V <= 0 || V >= ((int64_t)1 << 32) || ld < V || !pos || !token || !status ||
      !smp_config_ok(c))
    return IMIE_EARG;
  const bool has_hist = hist && hlen && hld > 0 && (c.rep_penalty || c.no_repeat_ngram);
  const size_t rv = (size_t)(rows * V);
  if ((int64_t)rv > g_smp.cap_rv) {                   // flag arrays start (and are left) all zero
    if (g_smp.rep.ensure(rv) || g_smp.ban.ensure(rv)) return IMIE_EARG;
    IMIE_HIP(hipMemset(g_smp.rep.p, 0, rv));
    IMIE_HIP(hipMemset(g_smp.ban.p, 0, rv));
    g_smp.cap_rv = (int64_t)rv;
  }
  const bool sorted = (c.mode == 2 || c.mode == 3) && (c.top_k > 0 || c.top_p < ((int64_t)1 << c.frac));
  if (g_smp.pr.ensure(rv * 8) || g_smp.part.ensure((size_t)rows * kSmpParts * 32) ||
      g_smp.st.ensure((size_t)rows * sizeof(SmpRow)))
    return IMIE_EARG;
  uint8_t* rep = (uint8_t*)g_smp.rep.p;
  uint8_t* ban = (uint8_t*)g_smp.ban.p;
  int64_t* pr = (int64_t*)g_smp.pr.p;
  int64_t* part = (int64_t*)g_smp.part.p;
  SmpRow* srow = (SmpRow*)g_smp.st.p;
  const dim3 gv(kSmpParts, (unsigned)rows);
  if (has_hist)
    hipLaunchKernelGGL(smp_flags_kernel, dim3((unsigned)((hld + 255) / 256), (unsigned)rows), dim3(256), 0, st, c, hist,
                       hld, hlen, V, rep, ban, (uint8_t)1, status);
  hipLaunchKernelGGL(smp_adjust_kernel, gv, dim3(256), 0, st, c, logits, ld, V, rep, ban, has_hist ? 1 : 0, pr, part);
  hipLaunchKernelGGL(smp_stats1_kernel, dim3((unsigned)rows), dim3(64), 0, st, c, part, srow, token, status);
  if (c.mode != 0) {
    hipLaunchKernelGGL(smp_exp_kernel, gv, dim3(256), 0, st, c, V, srow, smp_log2e((int)c.frac),
                       smp_dclip((int)c.frac), pr, part);
    hipLaunchKernelGGL(smp_sum_kernel, dim3((unsigned)rows), dim3(64), 0, st, part, srow, 0);
    hipLaunchKernelGGL(smp_prob_kernel, gv, dim3(256), 0, st, c, V, srow, pr, part);
    hipLaunchKernelGGL(smp_stats3_kernel, dim3((unsigned)rows), dim3(64), 0, st, c, part, srow);
    if (c.mode == 4) {
      hipLaunchKernelGGL(smp_minp_kernel, gv, dim3(256), 0, st, V, srow, pr, part);
      hipLaunchKernelGGL(smp_minp_final_kernel, dim3((unsigned)rows), dim3(64), 0, st, part, srow, pr, V);
    }
    if (sorted) {
      if (g_smp.keys.ensure(rv * 8) || g_smp.sorted.ensure(rv * 8) || g_smp.offs.ensure((size_t)(2 * rows + 1) * 4))
        return IMIE_EARG;
      if (rv >= ((size_t)1 << 31)) return IMIE_EARG;
      // segment r is [r * V, r * V + its nonzero count): both ends written on the device, in stream order
      const int* begs = (const int*)g_smp.offs.p;
      int* ends = (int*)g_smp.offs.p + rows;
      hipLaunchKernelGGL(smp_count_kernel, gv, dim3(256), 0, st, V, srow, pr, part);
      hipLaunchKernelGGL(smp_offsets_kernel, dim3((unsigned)rows), dim3(64), 0, st, V, part, (int*)g_smp.offs.p, ends);
      hipLaunchKernelGGL(smp_scatter_kernel, gv, dim3(256), 0, st, V, srow, pr, part, (uint64_t*)g_smp.keys.p);
      const int end_bit = 33 + (int)c.frac;           // p <= 2^frac
      size_t tmp_bytes = 0;
      IMIE_HIP(hipcub::DeviceSegmentedRadixSort::SortKeysDescending(nullptr, tmp_bytes, (const uint64_t*)g_smp.keys.p,
                                                                     (uint64_t*)g_smp.sorted.p, (int)rv, (int)rows,
                                                                     begs, (const int*)ends, 0, end_bit, st));
      if (g_smp.tmp.ensure(tmp_bytes)) return IMIE_EARG;
      IMIE_HIP(hipcub::DeviceSegmentedRadixSort::SortKeysDescending(g_smp.tmp.p, tmp_bytes,
                                                                     (const uint64_t*)g_smp.keys.p,
                                                                     (uint64_t*)g_smp.sorted.p, (int)rv, (int)rows,
                                                                     begs, (const int*)ends, 0, end_bit, st));
      hipLaunchKernelGGL(smp_trunc_kernel, dim3((unsigned)rows), dim3(kSmpScan), 0, st, c, V,
                         (const uint64_t*)g_smp.sorted.p, (const int*)ends, srow, pr);
    }
    hipLaunchKernelGGL(smp_select_kernel, dim3((unsigned)rows), dim3(kSmpScan), 0, st, c, V, pos, srow, pr, token);
  }
  if (has_hist)
    hipLaunchKernelGGL(smp_flags_kernel, dim3((unsigned)((hld + 255) / 256), (unsigned)rows), dim3(256), 0, st, c, hist,
                       hld, hlen, V, rep, ban, (uint8_t)0, status);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

extern "C" {

// Device rows: tokens for `rows` logits rows (row stride ld) under one sampler config; per-row history
// (hist_dev[r * hist_ld + i], i < hist_len_dev[r]) and absolute positions pos_dev[r] (the draw key). Asynchronous
// on `stream`; *status_dev gets IMIE_EOVF when the temperature guard trips (the reference raises OverflowError)
// and IMIE_EARG for a history token outside the vocabulary.
int imie_sample_dev(const int64_t* logits_dev, int64_t rows, int64_t vocab, int64_t ld, const ImieSamplerConfig* cfg,
                    const int64_t* hist_dev, int64_t hist_ld, const int64_t* hist_len_dev, const int64_t* pos_dev,
                    int64_t* token_dev, int* status_dev, void* stream) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!cfg || imie_device_ready() != 0) return IMIE_EARG;
  return imie_sample_launch(logits_dev, rows, vocab, ld, *cfg, hist_dev, hist_ld, hist_len_dev, pos_dev, token_dev,
                            status_dev, (hipStream_t)stream);
}

// Host row: sample_token(logits_row, cfg, position, frac, history_ids) (sampler.py:403-437). rc 0, 1 (bad
// arguments / history token outside the vocabulary), 2 (temperature overflow: the reference's OverflowError).
int imie_sample_token(const int64_t* logits, int64_t vocab, const ImieSamplerConfig* cfg, const int64_t* hist,
                      int64_t hist_n, int64_t position, int64_t* token) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!logits || !cfg || !token || vocab <= 0 || hist_n < 0 || (hist_n && !hist) || imie_device_ready() != 0)
    return IMIE_EARG;
  static DevBuf dl, dh, dsmall;
  hipStream_t st = imie_stream();
  const int64_t hn = hist_n > 0 ? hist_n : 1;
  if (dl.ensure((size_t)vocab * 8) || dh.ensure((size_t)hn * 8) || dsmall.ensure(64)) return IMIE_EARG;
  int64_t* sm = (int64_t*)dsmall.p;                   // [0] hist_len, [1] position, [2] token, [3] status
  const int64_t hv[2] = {hist_n, position};
  IMIE_HIP(hipMemcpyAsync(dl.p, logits, (size_t)vocab * 8, hipMemcpyHostToDevice, st));
  if (hist_n) IMIE_HIP(hipMemcpyAsync(dh.p, hist, (size_t)hist_n * 8, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemcpyAsync(sm, hv, 16, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemsetAsync(sm + 3, 0, 8, st));
  int rc = imie_sample_launch((const int64_t*)dl.p, 1, vocab, vocab, *cfg, hist_n ? (const int64_t*)dh.p : nullptr,
                              hn, sm, sm + 1, sm + 2, (int*)(sm + 3), st);
  if (rc) return rc;
  int64_t out[2];
  IMIE_HIP(hipMemcpyAsync(out, sm + 2, 16, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipStreamSynchronize(st));
  const int stat = (int)out[1];
  if (stat & IMIE_EARG) return IMIE_EARG;
  if (stat & IMIE_EOVF) return IMIE_EOVF;
  *token = out[0];
  return IMIE_OK;
}

// logits_digest on the device (sampler.py:421-425): digests (rows, 32) bytes of SHA-256 over each row's
// little-endian int64 bytes. Asynchronous on `stream`.
int imie_logits_digest_dev(const int64_t* logits_dev, int64_t rows, int64_t vocab, int64_t ld, uint8_t* digest_dev,
                           void* stream) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!logits_dev || !digest_dev || rows <= 0 || vocab <= 0 || ld < vocab || imie_device_ready() != 0)
    return IMIE_EARG;
  if ((reinterpret_cast<uintptr_t>(digest_dev) & 3) != 0) return IMIE_EARG;
  hipLaunchKernelGGL(smp_digest_kernel, dim3((unsigned)((rows + 63) / 64)), dim3(64), 0,
                     (hipStream_t)stream, logits_dev, rows, vocab, ld, (uint32_t*)digest_dev);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

// Test hook: the draw word and Lemire value for (total, seed, position) on the device (sampler.py:283-315).
int imie_sample_draw_probe(int64_t total, int64_t seed, int64_t position, uint64_t* word0, int64_t* target);

}  // extern "C"

namespace {
__global__ void smp_draw_probe_kernel(int64_t total, int64_t seed, int64_t pos, uint64_t* out) {
  out[0] = smp_prng_word((uint64_t)seed, (uint64_t)pos, 0);
  out[1] = (uint64_t)smp_draw((uint64_t)total, (uint64_t)seed, (uint64_t)pos);
}
}  // namespace

extern "C" int imie_sample_draw_probe(int64_t total, int64_t seed, int64_t position, uint64_t* word0, int64_t* target) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!word0 || !target || total < 0 || imie_device_ready() != 0) return IMIE_EARG;
  static DevBuf d;
  if (d.ensure(16)) return IMIE_EARG;
  hipStream_t st = imie_stream();
  hipLaunchKernelGGL(smp_draw_probe_kernel, dim3(1), dim3(1), 0, st, total, seed, position, (uint64_t*)d.p);
  uint64_t h[2];
  IMIE_HIP(hipMemcpyAsync(h, d.p, 16, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipStreamSynchronize(st));
  *word0 = h[0];
  *target = (int64_t)h[1];
  return IMIE_OK;
}
