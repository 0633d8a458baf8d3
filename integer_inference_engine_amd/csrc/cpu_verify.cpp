// Host (CPU) re-execution of a Bonsai forward for receipt verification, independent of the GPU producer.
//
// The reference's verifier re-derives a committed turn on the canonical integer reference engine on the CPU
// (bonsai/src/trinote/infer_int/verify.py:156-272 over reference_bonsai.py). This file is that role for this
// library: the same integer semantics as the reference's numpy path, computed on the host with plain C++ threads,
// sharing no code with the device kernels, so a verifier does not have to trust the GPU that produced the turn.
//   * Q1_0 linear (reference_bonsai.py:149-219): per (token, 128-block) a table of the 16 subset sums of each
//     4-weight nibble (32 nibbles x 16 entries), then per output row 32 lookups give pos = sum of the x under set
//     bits; S = 2 pos - total; += (S * scale) >> frac, everything wrapping mod 2^64 like numpy int64.
//   * RMSNorm (fixedpoint.py:31-71): exact 128-bit sum of squares, isqrt, floor((x << f) / rms), gain with the
//     fail-loud envelope; head RMSNorm per (head, position) (reference_bonsai.py:286-297).
//   * NeoX RoPE (rope_v2.py:92-117) with its envelope guard (rope.py:26-39), over all heads and positions.
//   * causal attention (reference_bonsai.py:586-598, 656-720): scores ((q k) >> f * inv_sqrt) >> f, masked keys
//     at -(1 << (f + 30)) included in the softmax, 2^-x cubic softmax (fixedpoint.py:74-140), (P V) >> f, both
//     matmul bounds (fixedpoint.py:207-227) per head.
//   * SiLU(gate) * up and the residual adds wrapping (reference_bonsai.py:245-264, 603-615); the output head.
//   * the integer sampler (sampler.py:160-437): repetition penalty and n-gram ban, temperature, softmax, top-k /
//     top-p / min-p truncation, and the SHA-256 counter draw with Lemire's reduction.
// Return codes: 0 ok; 1 bad arguments; 2 an int64 envelope the reference raises on (attention / RoPE / sampler
// temperature); 4 RMSNorm (sum of squares beyond 128 bits, or the gain envelope).
#include <stdint.h>
#include <string.h>
#include <algorithm>
#include <atomic>
#include <mutex>
#include <thread>
#include <vector>

namespace {

typedef unsigned __int128 u128;
typedef __int128 i128;
constexpr uint64_t kI64Max = 0x7FFFFFFFFFFFFFFFull;

inline int64_t fshift(int64_t v, int64_t s) { return v >> (s > 63 ? 63 : s); }   // numpy int64 >> s, s >= 0
inline uint64_t uabs(int64_t v) { return v < 0 ? (uint64_t)0 - (uint64_t)v : (uint64_t)v; }
inline int64_t wmul(int64_t a, int64_t b) { return (int64_t)((uint64_t)a * (uint64_t)b); }
inline int64_t wadd(int64_t a, int64_t b) { return (int64_t)((uint64_t)a + (uint64_t)b); }
inline int64_t wsub(int64_t a, int64_t b) { return (int64_t)((uint64_t)a - (uint64_t)b); }
inline int64_t floordiv(int64_t a, int64_t b) {   // numpy // for b > 0
  int64_t q = a / b;
  if ((a % b) != 0 && a < 0) --q;
  return q;
}

int g_threads = 0;
int nthreads() {
  if (g_threads > 0) return g_threads;
  const unsigned h = std::thread::hardware_concurrency();
  return h ? (int)std::min(h, 64u) : 4;
}

// run f(i) for i in [0, n) over the worker threads, contiguous chunks
template <typename F>
void parallel_for(int64_t n, F f) {
  const int nt = (int)std::min<int64_t>(nthreads(), std::max<int64_t>(n, 1));
  if (nt <= 1 || n < 64) {
    for (int64_t i = 0; i < n; ++i) f(i);
    return;
  }
  std::vector<std::thread> th;
  std::atomic<int64_t> next{0};
  const int64_t grain = std::max<int64_t>(1, n / (nt * 8));
  for (int w = 0; w < nt; ++w)
    th.emplace_back([&]() {
      for (;;) {
        const int64_t b = next.fetch_add(grain);
        if (b >= n) break;
        const int64_t e = std::min(n, b + grain);
        for (int64_t i = b; i < e; ++i) f(i);
      }
    });
  for (auto& t : th) t.join();
}

// ---- Q1_0 linear ------------------------------------------------------------------------------------------
// out (T, N) = x (T, K) over bits (N, nb, 16) / scale (N, nb), K = nb * 128
void q1_linear(const int64_t* x, const uint8_t* bits, const int64_t* scale, int64_t T, int64_t N, int64_t nb,
               int64_t frac, int64_t* out) {
  std::vector<int64_t> lut((size_t)(nb * 32 * 16)), tot((size_t)nb);
  for (int64_t t = 0; t < T; ++t) {
    const int64_t* xr = x + t * nb * 128;
    for (int64_t b = 0; b < nb; ++b) {
      int64_t total = 0;
      for (int j = 0; j < 32; ++j) {
        const int64_t* v = xr + b * 128 + 4 * j;
        int64_t* e = &lut[(size_t)((b * 32 + j) * 16)];
        e[0] = 0;
        for (int m = 1; m < 16; ++m) {                // subset sums by the lowest set bit
          const int low = __builtin_ctz((unsigned)m);
          e[m] = wadd(e[m & (m - 1)], v[low]);
        }
        total = wadd(total, e[15]);
      }
      tot[(size_t)b] = total;
    }
    int64_t* orow = out + t * N;
    parallel_for(N, [&](int64_t o) {
      const uint8_t* br = bits + o * nb * 16;
      const int64_t* sr = scale + o * nb;
      int64_t acc = 0;
      for (int64_t b = 0; b < nb; ++b) {
        const int64_t* e = &lut[(size_t)(b * 32 * 16)];
        int64_t pos = 0;
        for (int k = 0; k < 16; ++k) {
          const uint8_t by = br[b * 16 + k];
          pos = wadd(pos, wadd(e[(2 * k) * 16 + (by & 15)], e[(2 * k + 1) * 16 + (by >> 4)]));
        }
        const int64_t S = wsub(wmul(2, pos), tot[(size_t)b]);
        acc = wadd(acc, fshift(wmul(S, sr[b]), frac));
      }
      orow[o] = acc;
    });
  }
}

// ---- RMSNorm --------------------------------------------------------------------------------------------
uint64_t isqrt128(u128 v) {
  if (v == 0) return 0;
  uint64_t r = 0;
  for (int b = 63; b >= 0; --b) {                     // bitwise: exact, the verifier's speed is not here
    const uint64_t c = r | ((uint64_t)1 << b);
    if ((u128)c * c <= v) r = c;
  }
  return r;
}

// rows x cols; gain nullable. rc 4 where the oracle cannot (128-bit sum) or raises (gain envelope)
int rmsnorm(const int64_t* x, int64_t rows, int64_t cols, int64_t frac, int64_t eps, const int64_t* gain,
            int64_t* out) {
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t* xr = x + r * cols;
    u128 ssq = 0;
    for (int64_t c = 0; c < cols; ++c) {
      const u128 sq = (u128)uabs(xr[c]) * uabs(xr[c]);
      if (ssq + sq < ssq) return 4;
      ssq += sq;
    }
    const u128 mean = ssq / (u128)cols;
    if (mean + (u128)(uint64_t)eps < mean) return 4;
    const uint64_t rms = isqrt128(mean + (u128)(uint64_t)eps);
    if (rms == 0) return 4;
    for (int64_t c = 0; c < cols; ++c) {
      const i128 num = (i128)xr[c] * ((i128)1 << frac);
      i128 q = num / (i128)rms;
      if (num % (i128)rms != 0 && num < 0) q -= 1;
      if (q > (i128)INT64_MAX || q < (i128)INT64_MIN) return 4;
      out[r * cols + c] = (int64_t)q;
    }
  }
  if (gain) {
    uint64_t mn = 0, mg = 0;
    for (int64_t i = 0; i < rows * cols; ++i) mn = std::max(mn, uabs(out[i]));
    for (int64_t c = 0; c < cols; ++c) mg = std::max(mg, uabs(gain[c]));
    if ((u128)mn * mg > (u128)kI64Max) return 4;
    for (int64_t i = 0; i < rows * cols; ++i) out[i] = fshift(out[i] * gain[i % cols], frac);
  }
  return 0;
}

// ---- softmax --------------------------------------------------------------------------------------------
int64_t scaled_log2e(int64_t frac) {
  const int64_t s = 16 - frac;
  return s >= 0 ? (94548 >> s) : ((int64_t)94548 << -s);
}

int64_t exp2_neg(int64_t u, int64_t frac) {
  const int64_t FP = (int64_t)1 << frac;
  const int64_t k = u >> frac, f = u & (FP - 1);
  const int64_t s = 16 - frac;
  int64_t c0, c1, c2, c3;
  if (s >= 0) { c0 = 65536 >> s; c1 = 45426 >> s; c2 = 15743 >> s; c3 = 3638 >> s; }
  else { c0 = (int64_t)65536 << -s; c1 = (int64_t)45426 << -s; c2 = (int64_t)15743 << -s; c3 = (int64_t)3638 << -s; }
  const int64_t f2 = wmul(f, f) >> frac, f3 = wmul(f2, f) >> frac;
  int64_t poly = c0 - (wmul(c1, f) >> frac) + (wmul(c2, f2) >> frac) - (wmul(c3, f3) >> frac);
  if (poly < 0) poly = 0;
  if (k < 0) return 0;
  return poly >> (k < 63 ? k : 63);
}

int64_t d_clip(int64_t frac) {
  const int64_t l = scaled_log2e(frac);
  const int64_t a = ((frac + 2) << (2 * frac)) / l, b = ((int64_t)1 << 62) / l;
  return a < b ? a : b;
}

// row softmax in place (fixedpoint.py:99-140, numpy int64 arithmetic)
void softmax_row(int64_t* z, int64_t n, int64_t frac) {
  const int64_t log2e = scaled_log2e(frac), dc = d_clip(frac);
  int64_t m = INT64_MIN;
  for (int64_t j = 0; j < n; ++j) m = std::max(m, z[j]);
  int64_t Z = 0;
  for (int64_t j = 0; j < n; ++j) {
    int64_t d = wsub(m, z[j]);
    d = d < dc ? d : dc;
    z[j] = exp2_neg(wmul(d, log2e) >> frac, frac);
    Z = wadd(Z, z[j]);
  }
  for (int64_t j = 0; j < n; ++j) z[j] = Z == 0 ? 0 : floordiv(z[j] << frac, Z);
}

// ---- model ----------------------------------------------------------------------------------------------
struct CpuModel {
  int64_t nl, H, Hkv, hd, d, dff, vocab, frac, eps, inv_sqrt, rope_rows;
  std::vector<const uint8_t*> wb;       // [layer * 7 + proj]
  std::vector<const int64_t*> ws;
  std::vector<const int64_t*> g;        // [layer * 4 + {n1, n2, qn, kn}]
  const uint8_t *ebits, *obits;
  const int64_t *escale, *oscale, *finalg, *cos, *sin;
  bool live = true;
};
std::vector<CpuModel*> g_models;
std::mutex g_mu;

uint64_t absmax(const int64_t* a, int64_t n) {
  uint64_t m = 0;
  for (int64_t i = 0; i < n; ++i) m = std::max(m, uabs(a[i]));
  return m;
}

// NeoX rotation of t (n, T, hd) at positions 0..T-1, with the envelope over the whole tensor and table rows
int rope(int64_t* t, int64_t n, int64_t T, int64_t hd, const CpuModel& M) {
  const int64_t half = hd / 2;
  const uint64_t mx = absmax(t, n * T * hd);
  const uint64_t mc = std::max(absmax(M.cos, T * half), absmax(M.sin, T * half));
  if (n * T * hd && T * half && (u128)2 * mx * mc > (u128)kI64Max) return 2;
  for (int64_t h = 0; h < n; ++h)
    for (int64_t p = 0; p < T; ++p) {
      int64_t* v = t + (h * T + p) * hd;
      const int64_t* c = M.cos + p * half;
      const int64_t* s = M.sin + p * half;
      for (int64_t i = 0; i < half; ++i) {
        const int64_t x0 = v[i], x1 = v[i + half];
        v[i] = wsub(wmul(x0, c[i]), wmul(x1, s[i])) >> M.frac;
        v[i + half] = wadd(wmul(x0, s[i]), wmul(x1, c[i])) >> M.frac;
      }
    }
  return 0;
}

// causal attention over T positions: q (H, T, hd), k/v (Hkv, T, hd) -> out (T, H * hd)
int attention(const int64_t* q, const int64_t* k, const int64_t* v, const CpuModel& M, int64_t T, int64_t* out) {
  const int64_t H = M.H, Hkv = M.Hkv, hd = M.hd, rep = H / Hkv, f = M.frac;
  const int64_t neg = -((int64_t)1 << (f + 30));
  std::atomic<int> rc{0};
  std::vector<uint64_t> mk((size_t)Hkv), mv((size_t)Hkv);
  for (int64_t j = 0; j < Hkv; ++j) { mk[(size_t)j] = absmax(k + j * T * hd, T * hd); mv[(size_t)j] = absmax(v + j * T * hd, T * hd); }
  for (int64_t h = 0; h < H; ++h)
    if ((u128)absmax(q + h * T * hd, T * hd) * mk[(size_t)(h / rep)] * (u128)hd > (u128)kI64Max) return 2;
  std::vector<int64_t> P((size_t)(H * T * T));
  parallel_for(H * T, [&](int64_t hm) {
    const int64_t h = hm / T, m = hm % T, kv = h / rep;
    const int64_t* qr = q + (h * T + m) * hd;
    int64_t* pr = P.data() + hm * T;
    for (int64_t j = 0; j < T; ++j) {
      if (j > m) { pr[j] = neg; continue; }
      const int64_t* kr = k + (kv * T + j) * hd;
      int64_t dot = 0;
      for (int64_t c = 0; c < hd; ++c) dot = wadd(dot, wmul(qr[c], kr[c]));
      pr[j] = wmul(dot >> f, M.inv_sqrt) >> f;
    }
    softmax_row(pr, T, f);
  });
  for (int64_t h = 0; h < H; ++h)
    if ((u128)absmax(P.data() + h * T * T, T * T) * mv[(size_t)(h / rep)] * (u128)T > (u128)kI64Max) return 2;
  parallel_for(H * T, [&](int64_t hm) {
    const int64_t h = hm / T, m = hm % T, kv = h / rep;
    const int64_t* pr = P.data() + hm * T;
    std::vector<int64_t> acc((size_t)hd, 0);
    for (int64_t j = 0; j < T; ++j) {
      const int64_t* vr = v + (kv * T + j) * hd;
      for (int64_t c = 0; c < hd; ++c) acc[(size_t)c] = wadd(acc[(size_t)c], wmul(pr[j], vr[c]));
    }
    for (int64_t c = 0; c < hd; ++c) out[m * H * hd + h * hd + c] = acc[(size_t)c] >> f;
  });
  return rc.load();
}

int64_t silu(int64_t x, int64_t frac) {            // (x * sigmoid(x)) >> frac, sigmoid = 2-logit softmax
  const int64_t log2e = scaled_log2e(frac), dc = d_clip(frac);
  const int64_t m = x > 0 ? x : 0;
  int64_t d0 = m < dc ? m : dc;
  int64_t d1 = wsub(m, x);
  d1 = d1 < dc ? d1 : dc;
  const int64_t e0 = exp2_neg(wmul(d0, log2e) >> frac, frac), e1 = exp2_neg(wmul(d1, log2e) >> frac, frac);
  const int64_t z = wadd(e0, e1);
  const int64_t sig = z == 0 ? 0 : floordiv(e1 << frac, z);
  return wmul(x, sig) >> frac;
}

// hidden rows x (T, d) through every layer, positions 0..T-1, in place
int forward_layers(const CpuModel& M, int64_t* x, int64_t T) {
  const int64_t d = M.d, H = M.H, Hkv = M.Hkv, hd = M.hd, dff = M.dff, f = M.frac, qd = H * hd, kd = Hkv * hd;
  std::vector<int64_t> n((size_t)(T * d)), q((size_t)(T * qd)), k((size_t)(T * kd)), v((size_t)(T * kd));
  std::vector<int64_t> qh((size_t)(T * qd)), kh((size_t)(T * kd)), vh((size_t)(T * kd)), att((size_t)(T * qd));
  std::vector<int64_t> y((size_t)(T * std::max(d, dff))), gt((size_t)(T * dff)), up((size_t)(T * dff));
  for (int64_t l = 0; l < M.nl; ++l) {
    auto W = [&](int p) { return M.wb[(size_t)(l * 7 + p)]; };
    auto S = [&](int p) { return M.ws[(size_t)(l * 7 + p)]; };
    int rc = rmsnorm(x, T, d, f, M.eps, M.g[(size_t)(l * 4 + 0)], n.data());
    if (rc) return rc;
    q1_linear(n.data(), W(0), S(0), T, qd, d / 128, f, q.data());
    q1_linear(n.data(), W(1), S(1), T, kd, d / 128, f, k.data());
    q1_linear(n.data(), W(2), S(2), T, kd, d / 128, f, v.data());
    // (T, heads, hd) -> (heads, T, hd); per-(head, position) RMSNorm of q and k
    for (int64_t t = 0; t < T; ++t) {
      for (int64_t h = 0; h < H; ++h) memcpy(&qh[(size_t)((h * T + t) * hd)], &q[(size_t)(t * qd + h * hd)], hd * 8);
      for (int64_t h = 0; h < Hkv; ++h) {
        memcpy(&kh[(size_t)((h * T + t) * hd)], &k[(size_t)(t * kd + h * hd)], hd * 8);
        memcpy(&vh[(size_t)((h * T + t) * hd)], &v[(size_t)(t * kd + h * hd)], hd * 8);
      }
    }
    if ((rc = rmsnorm(qh.data(), H * T, hd, f, M.eps, M.g[(size_t)(l * 4 + 2)], qh.data()))) return rc;
    if ((rc = rmsnorm(kh.data(), Hkv * T, hd, f, M.eps, M.g[(size_t)(l * 4 + 3)], kh.data()))) return rc;
    if ((rc = rope(qh.data(), H, T, hd, M))) return rc;
    if ((rc = rope(kh.data(), Hkv, T, hd, M))) return rc;
    if ((rc = attention(qh.data(), kh.data(), vh.data(), M, T, att.data()))) return rc;
    q1_linear(att.data(), W(3), S(3), T, d, qd / 128, f, y.data());
    for (int64_t i = 0; i < T * d; ++i) x[i] = wadd(x[i], y[(size_t)i]);
    if ((rc = rmsnorm(x, T, d, f, M.eps, M.g[(size_t)(l * 4 + 1)], n.data()))) return rc;
    q1_linear(n.data(), W(4), S(4), T, dff, d / 128, f, gt.data());
    q1_linear(n.data(), W(5), S(5), T, dff, d / 128, f, up.data());
    for (int64_t i = 0; i < T * dff; ++i) gt[(size_t)i] = wmul(silu(gt[(size_t)i], f), up[(size_t)i]) >> f;
    q1_linear(gt.data(), W(6), S(6), T, d, dff / 128, f, y.data());
    for (int64_t i = 0; i < T * d; ++i) x[i] = wadd(x[i], y[(size_t)i]);
  }
  return 0;
}

// ---- sampler (sampler.py:160-437) -----------------------------------------------------------------------
struct SamplerCfg {                                 // ImieSamplerConfig (include/imie_bonsai.h)
  int64_t mode, frac, inv_temp, top_k, top_p, min_p, rep_penalty, no_repeat_ngram, seed;
};

// SHA-256 (FIPS 180-4) of a message of at most 55 bytes (one block)
void sha256_short(const uint8_t* msg, size_t len, uint8_t out[32]) {
  static const uint32_t K[64] = {
      0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5, 0xd807aa98,
      0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174, 0xe49b69c1, 0xefbe4786,
      0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da, 0x983e5152, 0xa831c66d, 0xb00327c8,
      0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967, 0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13,
      0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85, 0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819,
      0xd6990624, 0xf40e3585, 0x106aa070, 0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a,
      0x5b9cca4f, 0x682e6ff3, 0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7,
      0xc67178f2};
  uint8_t blk[64] = {0};
  memcpy(blk, msg, len);
  blk[len] = 0x80;
  const uint64_t bitlen = (uint64_t)len * 8;
  for (int i = 0; i < 8; ++i) blk[63 - i] = (uint8_t)(bitlen >> (8 * i));
  uint32_t w[64];
  for (int i = 0; i < 16; ++i)
    w[i] = ((uint32_t)blk[4 * i] << 24) | ((uint32_t)blk[4 * i + 1] << 16) | ((uint32_t)blk[4 * i + 2] << 8) | blk[4 * i + 3];
  auto rotr = [](uint32_t x, int n) { return (x >> n) | (x << (32 - n)); };
  for (int i = 16; i < 64; ++i) {
    const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
    const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
    w[i] = w[i - 16] + s0 + w[i - 7] + s1;
  }
  uint32_t hs[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a, 0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
  uint32_t a = hs[0], b = hs[1], c = hs[2], dd = hs[3], e = hs[4], f = hs[5], g = hs[6], h = hs[7];
  for (int i = 0; i < 64; ++i) {
    const uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25), ch = (e & f) ^ (~e & g);
    const uint32_t t1 = h + S1 + ch + K[i] + w[i];
    const uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22), mj = (a & b) ^ (a & c) ^ (b & c);
    const uint32_t t2 = S0 + mj;
    h = g; g = f; f = e; e = dd + t1; dd = c; c = b; b = a; a = t1 + t2;
  }
  hs[0] += a; hs[1] += b; hs[2] += c; hs[3] += dd; hs[4] += e; hs[5] += f; hs[6] += g; hs[7] += h;
  for (int i = 0; i < 8; ++i)
    for (int j = 0; j < 4; ++j) out[4 * i + j] = (uint8_t)(hs[i] >> (24 - 8 * j));
}

// first 8 bytes (big-endian) of SHA-256("trinote-sampler-draw/v1" || seed || position || counter), sampler.py:280-298
uint64_t prng_word(int64_t seed, int64_t position, uint64_t counter) {
  static const char tag[] = "trinote-sampler-draw/v1";
  uint8_t msg[23 + 24];
  memcpy(msg, tag, 23);
  const uint64_t f3[3] = {(uint64_t)seed, (uint64_t)position, counter};
  for (int k = 0; k < 3; ++k)
    for (int i = 0; i < 8; ++i) msg[23 + 8 * k + i] = (uint8_t)(f3[k] >> (56 - 8 * i));
  uint8_t dg[32];
  sha256_short(msg, sizeof(msg), dg);
  uint64_t r = 0;
  for (int i = 0; i < 8; ++i) r = (r << 8) | dg[i];
  return r;
}

// uniform in [0, total) by Lemire's multiply-shift with rejection below 2^64 mod total (sampler.py:301-319)
uint64_t draw_uniform(uint64_t total, int64_t seed, int64_t position) {
  if (total <= 1) return 0;
  uint64_t j = 0;
  u128 m = (u128)prng_word(seed, position, j++) * total;
  uint64_t low = (uint64_t)m;
  if (low < total) {
    const uint64_t t = (uint64_t)((((u128)1) << 64) % total);
    while (low < t) {
      m = (u128)prng_word(seed, position, j++) * total;
      low = (uint64_t)m;
    }
  }
  return (uint64_t)(m >> 64);
}

int64_t argmax_first(const int64_t* r, int64_t n) {
  int64_t b = 0;
  for (int64_t i = 1; i < n; ++i)
    if (r[i] > r[b]) b = i;
  return b;
}

// sample_token (sampler.py:403-437); rc 2 on the temperature envelope, 1 on a history id outside the vocabulary
int sample_token(const int64_t* logits, int64_t V, const SamplerCfg& c, const int64_t* hist, int64_t hl,
                 int64_t position, int64_t* token) {
  const int64_t f = c.frac, FP = (int64_t)1 << f;
  std::vector<int64_t> row(logits, logits + V);
  if ((c.rep_penalty || c.no_repeat_ngram) && hist && hl > 0) {      // apply_rep_penalty (sampler.py:189-211)
    for (int64_t i = 0; i < hl; ++i)
      if (hist[i] < 0 || hist[i] >= V) return 1;
    if (c.rep_penalty) {
      const int64_t den = FP + c.rep_penalty;
      std::vector<int64_t> seen(hist, hist + hl);
      std::sort(seen.begin(), seen.end());
      seen.erase(std::unique(seen.begin(), seen.end()), seen.end());
      for (int64_t t : seen) {
        const int64_t l = row[(size_t)t];
        row[(size_t)t] = l >= 0 ? floordiv(wmul(l, FP), den) : floordiv(wmul(l, den), FP);
      }
    }
    const int64_t n = c.no_repeat_ngram;
    if (n > 1 && hl >= n) {
      for (int64_t i = 0; i + n <= hl; ++i) {
        bool same = true;
        for (int64_t q = 0; q < n - 1 && same; ++q) same = hist[i + q] == hist[hl - (n - 1) + q];
        if (same) row[(size_t)hist[i + n - 1]] = -((int64_t)1 << 40);
      }
    }
  }
  if (c.mode == 0) { *token = argmax_first(row.data(), V); return 0; }
  std::vector<int64_t> p(row);
  if (c.inv_temp != FP) {                                            // _apply_temp_fp (sampler.py:244-262)
    int64_t lo = 0, hi = 0;
    for (int64_t i = 0; i < V; ++i) { lo = std::min(lo, p[(size_t)i]); hi = std::max(hi, p[(size_t)i]); }
    const u128 peak = (u128)std::max(uabs(lo), uabs(hi)) * (u128)(uint64_t)c.inv_temp;
    if (peak >= ((u128)1 << 63)) return 2;
    for (auto& v : p) v = wmul(v, c.inv_temp) >> f;
  }
  softmax_row(p.data(), V, f);
  if (c.mode == 2 || c.mode == 3) {                                 // _truncate (sampler.py:334-363)
    std::vector<int64_t> order((size_t)V);
    for (int64_t i = 0; i < V; ++i) order[(size_t)i] = i;
    std::stable_sort(order.begin(), order.end(), [&](int64_t a, int64_t b) { return p[(size_t)a] < p[(size_t)b]; });
    std::reverse(order.begin(), order.end());                       // descending, high-id ties first
    int64_t keep = c.top_k > 0 ? std::min(std::max<int64_t>(1, c.top_k), V) : V;
    if (c.top_p < FP) {
      int64_t csum = 0, nn = keep;
      for (int64_t i = 0; i < keep; ++i) {
        csum += p[(size_t)order[(size_t)i]];
        if (csum >= c.top_p) { nn = i; break; }
      }
      keep = std::max<int64_t>(1, std::min(nn + 1, keep));
    }
    std::vector<int64_t> res((size_t)V, 0);
    bool any = false;
    for (int64_t i = 0; i < keep; ++i) { res[(size_t)order[(size_t)i]] = p[(size_t)order[(size_t)i]]; any = any || p[(size_t)order[(size_t)i]] != 0; }
    if (!any) res[(size_t)order[0]] = 1;
    p.swap(res);
  } else if (c.mode == 4 && c.min_p > 0) {                          // _truncate_min_p (sampler.py:366-380)
    const int64_t amax = argmax_first(p.data(), V), pmax = p[(size_t)amax];
    if (pmax > 0) {
      const int64_t th = (int64_t)(((i128)c.min_p * pmax) >> f);
      bool any = false;
      for (auto& v : p) { if (v < th) v = 0; any = any || v != 0; }
      if (!any) p[(size_t)amax] = 1;
    }
  }
  int64_t total = 0;
  for (auto v : p) total += v;
  if (total <= 0) { *token = argmax_first(row.data(), V); return 0; }
  const uint64_t target = draw_uniform((uint64_t)total, c.seed, position);
  int64_t csum = 0;                                                  // searchsorted(cumsum, target, "right")
  for (int64_t i = 0; i < V; ++i) {
    csum += p[(size_t)i];
    if ((uint64_t)csum > target) { *token = i; return 0; }
  }
  *token = V - 1;
  return 0;
}

}  // namespace

extern "C" {

// Build a host model over the caller's arrays (borrowed: they must outlive the handle). w_bits / w_scale: 7 per
// layer in the order wq, wk, wv, wo, w1, wu, w2; gains: 4 per layer (n1, n2, q-norm, k-norm). -1 on bad shapes.
int64_t imie_cpu_model_create(int64_t n_layers, int64_t H, int64_t Hkv, int64_t hd, int64_t d, int64_t dff,
                              int64_t vocab, int64_t frac, int64_t eps, int64_t inv_sqrt,
                              const uint8_t* const* w_bits, const int64_t* const* w_scale,
                              const int64_t* const* gains, const uint8_t* embed_bits, const int64_t* embed_scale,
                              const uint8_t* out_bits, const int64_t* out_scale, const int64_t* final_gain,
                              const int64_t* cos, const int64_t* sin, int64_t rope_rows) {
  if (n_layers <= 0 || H <= 0 || Hkv <= 0 || H % Hkv || hd <= 0 || (hd & 1) || d <= 0 || d % 128 || dff <= 0 ||
      dff % 128 || (H * hd) % 128 || vocab <= 0 || frac < 1 || frac > 29 || eps < 0 || !w_bits || !w_scale ||
      !gains || !embed_bits || !embed_scale || !out_bits || !out_scale || !final_gain || !cos || !sin ||
      rope_rows <= 0)
    return -1;
  CpuModel* m = new CpuModel();
  m->nl = n_layers; m->H = H; m->Hkv = Hkv; m->hd = hd; m->d = d; m->dff = dff; m->vocab = vocab; m->frac = frac;
  m->eps = eps; m->inv_sqrt = inv_sqrt; m->rope_rows = rope_rows;
  m->wb.assign(w_bits, w_bits + 7 * n_layers);
  m->ws.assign(w_scale, w_scale + 7 * n_layers);
  m->g.assign(gains, gains + 4 * n_layers);
  m->ebits = embed_bits; m->escale = embed_scale; m->obits = out_bits; m->oscale = out_scale;
  m->finalg = final_gain; m->cos = cos; m->sin = sin;
  std::lock_guard<std::mutex> lk(g_mu);
  g_models.push_back(m);
  return (int64_t)g_models.size() - 1;
}

void imie_cpu_model_free(int64_t h) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (h >= 0 && h < (int64_t)g_models.size() && g_models[(size_t)h]) {
    delete g_models[(size_t)h];
    g_models[(size_t)h] = nullptr;
  }
}

// Worker threads for the host forward (0: the machine's hardware threads, at most 64).
void imie_cpu_set_threads(int n) { g_threads = n; }

// Teacher-forced logits of ids (positions 0..T-1, T <= rope rows): (T, vocab), or the last row only.
int imie_cpu_forward(int64_t h, const int64_t* ids, int64_t T, int last_only, int64_t* logits) {
  CpuModel* M = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    if (h >= 0 && h < (int64_t)g_models.size()) M = g_models[(size_t)h];
  }
  if (!M || !ids || !logits || T <= 0 || T > M->rope_rows) return 1;
  const int64_t d = M->d, nb = d / 128;
  for (int64_t t = 0; t < T; ++t)
    if (ids[t] < 0 || ids[t] >= M->vocab) return 1;
  std::vector<int64_t> x((size_t)(T * d));
  for (int64_t t = 0; t < T; ++t)                   // embedding rows sign * scale (reference_bonsai.py:138-146)
    for (int64_t b = 0; b < nb; ++b) {
      const uint8_t* br = M->ebits + (ids[t] * nb + b) * 16;
      const int64_t s = M->escale[ids[t] * nb + b];
      for (int i = 0; i < 128; ++i) x[(size_t)(t * d + b * 128 + i)] = ((br[i >> 3] >> (i & 7)) & 1) ? s : -s;
    }
  int rc = forward_layers(*M, x.data(), T);
  if (rc) return rc;
  const int64_t r0 = last_only ? T - 1 : 0, R = T - r0;
  std::vector<int64_t> n((size_t)(R * d));
  if ((rc = rmsnorm(x.data() + r0 * d, R, d, M->frac, M->eps, M->finalg, n.data()))) return rc;
  q1_linear(n.data(), M->obits, M->oscale, R, M->vocab, nb, M->frac, logits);
  return 0;
}

// sample_token (sampler.py:403-437) of one host row on the host: history (nullable) = the committed prefix, its
// length the draw key when the caller passes position = len(history). rc 0; 1 bad arguments; 2 temperature.
int imie_cpu_sample_token(const int64_t* logits, int64_t vocab, const void* cfg, const int64_t* history,
                          int64_t hist_len, int64_t position, int64_t* token) {
  if (!logits || vocab <= 0 || !cfg || !token || hist_len < 0 || (hist_len > 0 && !history)) return 1;
  const SamplerCfg c = *(const SamplerCfg*)cfg;
  if (c.frac < 1 || c.frac > 29 || c.mode < 0 || c.mode > 4 || (c.mode != 0 && c.inv_temp <= 0)) return 1;
  return sample_token(logits, vocab, c, history, hist_len, position, token);
}

}  // extern "C"
