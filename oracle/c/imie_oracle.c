// imie CPU oracle, C/OpenMP restatement (TEST INFRASTRUCTURE ONLY: used by tests/ and bench.py's cpu_baseline
// as the checker, never by the product).
//
// Restates, with numpy int64 semantics (wrap mod 2^64, floor shifts):
//   * Q1_0 linear      reference_bonsai.py:149-219 / bonsai_q1_kernel.c:85-106 (byte subset-sum LUT form)
//   * RMSNorm          fixedpoint.py:31-71 (exact 128-bit ssq; rc 4 when 128 bits do not suffice -> the Python
//                      wrapper falls back to the big-int numpy oracle)
//   * attention        reference_bonsai.py:656-720 numpy path, INCLUDING the masked sentinel entries in the
//                      softmax, and the fail-loud bounds of fixedpoint.py:207-227 (rc 2)
//   * SiLU * up       reference_bonsai.py:245-264, :614 over fixedpoint.py:143-174
//   * nmc linear       north-mini-code/src/nmc/cohere2.py:102-106 + qk_codec.py (exact int128 dot, one floor;
//                      rc 2 when a result does not fit int64, where numpy's astype would raise)
// Parity of this file with the numpy oracle is asserted in tests/test_oracle_c.py.
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef __int128 i128;
typedef unsigned __int128 u128;

static inline int64_t floor_shift(int64_t v, int64_t s) { return v >> (s > 63 ? 63 : s); }

// ---------------------------------------------------------------------------------------------------------
// Q1_0: out[t,o] = sum_b floor((2*pos - total) * scale, frac), pos from a 16x256 subset-sum table per (t,b).
// ---------------------------------------------------------------------------------------------------------
int imo_q1_linear(const int64_t *x, const uint8_t *bits, const int64_t *scale, int64_t T, int64_t N, int64_t nb,
                  int64_t frac, int64_t *out) {
  if (!x || !bits || !scale || !out || T < 0 || N < 0 || nb <= 0 || frac < 0) return 1;
  const int64_t K = nb * 128;
  const int64_t TC = 8;  // tokens per LUT chunk
  memset(out, 0, (size_t)(T * N) * 8);
  uint64_t *lut = (uint64_t *)malloc((size_t)TC * 16 * 256 * 8);
  uint64_t *tot = (uint64_t *)malloc((size_t)TC * 8);
  if (!lut || !tot) { free(lut); free(tot); return 1; }
  for (int64_t t0 = 0; t0 < T; t0 += TC) {
    const int64_t tn = T - t0 < TC ? T - t0 : TC;
    for (int64_t b = 0; b < nb; ++b) {
      for (int64_t t = 0; t < tn; ++t) {
        const int64_t *xb = x + (t0 + t) * K + b * 128;
        uint64_t total = 0;
        for (int j = 0; j < 16; ++j) {
          uint64_t *L = lut + ((size_t)t * 16 + j) * 256;
          L[0] = 0;
          for (int i = 0; i < 8; ++i) {
            const uint64_t xv = (uint64_t)xb[8 * j + i];
            total += xv;
            for (int v = 0; v < (1 << i); ++v) L[(1 << i) + v] = L[v] + xv;
          }
        }
        tot[t] = total;
      }
#pragma omp parallel for schedule(static)
      for (int64_t o = 0; o < N; ++o) {
        const uint8_t *bb = bits + (o * nb + b) * 16;
        const uint64_t sc = (uint64_t)scale[o * nb + b];
        for (int64_t t = 0; t < tn; ++t) {
          const uint64_t *L = lut + (size_t)t * 16 * 256;
          uint64_t pos = 0;
          for (int j = 0; j < 16; ++j) pos += L[j * 256 + bb[j]];
          const uint64_t S = 2u * pos - tot[t];
          const int64_t term = floor_shift((int64_t)(S * sc), frac);
          out[(t0 + t) * N + o] = (int64_t)((uint64_t)out[(t0 + t) * N + o] + (uint64_t)term);
        }
      }
    }
  }
  free(lut);
  free(tot);
  return 0;
}

// ---------------------------------------------------------------------------------------------------------
// RMSNorm (rc 4 = needs the big-int path; rc 2 = gain envelope exceeded, where the oracle raises)
// ---------------------------------------------------------------------------------------------------------
static uint64_t isqrt_u128(u128 v) {
  if (v == 0) return 0;
  uint64_t r = 0;
  for (int b = 63; b >= 0; --b) {
    const uint64_t c = r | ((uint64_t)1 << b);
    if ((u128)c * c <= v) r = c;
  }
  return r;
}

static inline int64_t floor_div_i128(i128 a, i128 b) {  // b > 0
  i128 q = a / b;
  if ((a % b) != 0 && a < 0) q -= 1;
  return (int64_t)q;
}

int imo_rmsnorm(const int64_t *x, int64_t rows, int64_t cols, int64_t frac, int64_t eps, const int64_t *gain,
                int64_t *out) {
  if (!x || !out || rows < 0 || cols <= 0 || frac < 0 || frac > 62 || eps < 0) return 1;
  int rc = 0;
  u128 maxn = 0, maxg = 0;
  if (gain)
    for (int64_t c = 0; c < cols; ++c) {
      const u128 a = gain[c] < 0 ? (u128)(-(i128)gain[c]) : (u128)gain[c];
      if (a > maxg) maxg = a;
    }
#pragma omp parallel for schedule(static) reduction(max : rc)
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t *row = x + r * cols;
    u128 ssq = 0;
    int bad = 0;
    for (int64_t c = 0; c < cols; ++c) {
      const u128 a = row[c] < 0 ? (u128)(-(i128)row[c]) : (u128)row[c];
      const u128 sq = a * a;
      if (ssq > ~(u128)0 - sq) { bad = 1; break; }
      ssq += sq;
    }
    if (bad) { rc = rc > 4 ? rc : 4; continue; }
    const uint64_t rms = isqrt_u128(ssq / (u128)cols + (u128)eps);
    if (rms == 0) { rc = rc > 4 ? rc : 4; continue; }
    for (int64_t c = 0; c < cols; ++c) out[r * cols + c] = floor_div_i128((i128)row[c] << frac, (i128)rms);
  }
  if (rc) return rc;
  if (gain) {
    for (int64_t i = 0; i < rows * cols; ++i) {
      const u128 a = out[i] < 0 ? (u128)(-(i128)out[i]) : (u128)out[i];
      if (a > maxn) maxn = a;
    }
    if (maxn != 0 && maxg != 0 && maxn * maxg > (u128)INT64_MAX) return 2;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < rows * cols; ++i) out[i] = floor_shift(out[i] * gain[i % cols], frac);
  }
  return 0;
}

// ---------------------------------------------------------------------------------------------------------
// Fixed-point softmax pieces (fixedpoint.py:74-140), numpy shift semantics for negative counts.
// ---------------------------------------------------------------------------------------------------------
static int64_t scaled_log2e(int64_t frac) {
  const int64_t s = 16 - frac;
  return s >= 0 ? (94548 >> s) : (94548LL << (-s));
}

static int64_t exp2_neg(int64_t u, int64_t frac) {
  const int64_t FP = (int64_t)1 << frac;
  const int64_t k = u >> frac, f = u & (FP - 1);
  const int64_t s = 16 - frac;
  int64_t c0, c1, c2, c3;
  if (s >= 0) { c0 = 65536 >> s; c1 = 45426 >> s; c2 = 15743 >> s; c3 = 3638 >> s; }
  else { c0 = 65536LL << -s; c1 = 45426LL << -s; c2 = 15743LL << -s; c3 = 3638LL << -s; }
  const int64_t f2 = (int64_t)((uint64_t)f * (uint64_t)f) >> frac;
  const int64_t f3 = (int64_t)((uint64_t)f2 * (uint64_t)f) >> frac;
  int64_t poly = c0 - ((c1 * f) >> frac) + ((c2 * f2) >> frac) - ((c3 * f3) >> frac);
  if (poly < 0) poly = 0;
  const int64_t kk = k < 63 ? k : 63;
  if (kk < 0) return 0;  // numpy: a negative shift count gives 0 for a non-negative value
  return poly >> kk;
}

// SiLU(gate) * up of the FFN (reference_bonsai.py:245-264 fixed_point_silu over fixedpoint.py:143-174 sigmoid,
// then :614 mulshift): sig = (e1 << f) // (e0 + e1), e0 = 2^-min(max(x,0), dclip), e1 = 2^-min(max(x,0) - x, dclip)
// (hard-capped dclip), silu = (x * sig) >> f, h = (silu * up) >> f, every product wrapping mod 2^64 as in numpy.
int imo_silu_mul(const int64_t *gate, const int64_t *up, int64_t n, int64_t frac, int64_t *out) {
  if (!gate || !up || !out || n < 0 || frac < 1 || frac > 29) return 1;
  const int64_t log2e = scaled_log2e(frac);
  const int64_t dca = ((frac + 2) << (2 * frac)) / log2e, dcb = ((int64_t)1 << 62) / log2e;
  const int64_t dclip = dca < dcb ? dca : dcb;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const int64_t x = gate[i];
    const int64_t m = x > 0 ? x : 0;
    int64_t d0 = m < dclip ? m : dclip;
    int64_t d1 = (int64_t)((uint64_t)m - (uint64_t)x);
    d1 = d1 < dclip ? d1 : dclip;
    const int64_t e0 = exp2_neg((int64_t)((uint64_t)d0 * (uint64_t)log2e) >> frac, frac);
    const int64_t e1 = exp2_neg((int64_t)((uint64_t)d1 * (uint64_t)log2e) >> frac, frac);
    const int64_t z = (int64_t)((uint64_t)e0 + (uint64_t)e1);
    int64_t sig = 0;
    if (z != 0) {
      const int64_t num = (int64_t)((uint64_t)e1 << frac);
      sig = num / z;
      if ((num % z) != 0 && ((num < 0) != (z < 0))) sig -= 1;
    }
    const int64_t silu = (int64_t)((uint64_t)x * (uint64_t)sig) >> frac;
    out[i] = (int64_t)((uint64_t)silu * (uint64_t)up[i]) >> frac;
  }
  return 0;
}

static uint64_t absu(int64_t v) { return v < 0 ? (uint64_t)0 - (uint64_t)v : (uint64_t)v; }

// q (H,M,hd); k,v (Hkv,L,hd) with L = start + M, kv head h2's row j at (h2 * ldk + j) * hd (ldk >= L: a cache
// with room for more rows); out (H,M,hd). numpy path of reference_bonsai.py:708-719. rc 2 where the numpy oracle
// raises OverflowError. Sums wrap mod 2^64, so their order (here row-major over V) does not change them.
int imo_attention_ld(const int64_t *q, const int64_t *k, const int64_t *v, int64_t H, int64_t Hkv, int64_t hd,
                     int64_t M, int64_t L, int64_t ldk, int64_t start, int64_t frac, int64_t inv_sqrt,
                     int64_t *out) {
  if (!q || !k || !v || !out || H <= 0 || Hkv <= 0 || H % Hkv || hd <= 0 || M <= 0 || L != start + M ||
      ldk < L || frac < 1 || frac > 29)
    return 1;
  const int64_t rep = H / Hkv;
  const int64_t log2e = scaled_log2e(frac);
  int64_t dca = ((frac + 2) << (2 * frac)) / log2e, dcb = ((int64_t)1 << 62) / log2e;
  const int64_t dclip = dca < dcb ? dca : dcb;
  const int64_t neg = -((int64_t)1 << (frac + 30));
  int rc = 0;
  uint64_t *mk = (uint64_t *)calloc((size_t)(2 * Hkv), 8), *mv = mk + Hkv;
  if (!mk) return 1;
#pragma omp parallel for schedule(static)
  for (int64_t kv = 0; kv < Hkv; ++kv)
    for (int64_t i = 0; i < L * hd; ++i) {
      const uint64_t a = absu(k[kv * ldk * hd + i]), b = absu(v[kv * ldk * hd + i]);
      if (a > mk[kv]) mk[kv] = a;
      if (b > mv[kv]) mv[kv] = b;
    }
  // QK bound per head: max|q_h| * max|K_kv| * hd
  for (int64_t h = 0; h < H && !rc; ++h) {
    uint64_t mq = 0;
    for (int64_t i = 0; i < M * hd; ++i) { const uint64_t a = absu(q[h * M * hd + i]); if (a > mq) mq = a; }
    if ((u128)mq * mk[h / rep] * (u128)hd > (u128)INT64_MAX) rc = 2;
  }
  int64_t *probs = rc ? NULL : (int64_t *)malloc((size_t)(H * M * L) * 8);
  if (!rc && !probs) rc = 1;
  if (!rc) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t h = 0; h < H; ++h)
      for (int64_t m = 0; m < M; ++m) {
        const int64_t kv = h / rep;
        const int64_t *qr = q + (h * M + m) * hd;
        int64_t *p = probs + (h * M + m) * L;
        int64_t mx = INT64_MIN;
        for (int64_t j = 0; j < L; ++j) {
          int64_t s;
          if (j > start + m) s = neg;
          else {
            uint64_t dot = 0;
            const int64_t *kr = k + (kv * ldk + j) * hd;
            for (int64_t d = 0; d < hd; ++d) dot += (uint64_t)qr[d] * (uint64_t)kr[d];
            s = (int64_t)dot >> frac;
            s = (int64_t)((uint64_t)s * (uint64_t)inv_sqrt) >> frac;
          }
          p[j] = s;
          if (s > mx) mx = s;
        }
        uint64_t Z = 0;
        for (int64_t j = 0; j < L; ++j) {
          int64_t d = (int64_t)((uint64_t)mx - (uint64_t)p[j]);
          if (d > dclip) d = dclip;
          const int64_t u = (int64_t)((uint64_t)d * (uint64_t)log2e) >> frac;
          p[j] = exp2_neg(u, frac);
          Z += (uint64_t)p[j];
        }
        for (int64_t j = 0; j < L; ++j) {
          if (Z == 0) p[j] = 0;
          else {
            const int64_t num = (int64_t)((uint64_t)p[j] << frac);
            int64_t qq = num / (int64_t)Z;
            if ((num % (int64_t)Z) != 0 && num < 0) qq -= 1;
            p[j] = qq;
          }
        }
      }
    // PV bound per head: max|P_h| * max|V_kv| * L
    for (int64_t h = 0; h < H && !rc; ++h) {
      uint64_t mp = 0;
      for (int64_t i = 0; i < M * L; ++i) { const uint64_t a = absu(probs[h * M * L + i]); if (a > mp) mp = a; }
      if ((u128)mp * mv[h / rep] * (u128)L > (u128)INT64_MAX) rc = 2;
    }
  }
  if (!rc) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t h = 0; h < H; ++h)
      for (int64_t m = 0; m < M; ++m) {
        const int64_t kv = h / rep;
        const int64_t *p = probs + (h * M + m) * L;
        uint64_t acc[256];
        for (int64_t d = 0; d < hd; ++d) acc[d] = 0;
        for (int64_t j = 0; j < L; ++j) {
          const uint64_t pj = (uint64_t)p[j];
          const int64_t *vr = v + (kv * ldk + j) * hd;
          for (int64_t d = 0; d < hd; ++d) acc[d] += pj * (uint64_t)vr[d];
        }
        for (int64_t d = 0; d < hd; ++d) out[(h * M + m) * hd + d] = (int64_t)acc[d] >> frac;
      }
  }
  free(probs);
  free(mk);
  return rc;
}

int imo_attention(const int64_t *q, const int64_t *k, const int64_t *v, int64_t H, int64_t Hkv, int64_t hd,
                  int64_t M, int64_t L, int64_t start, int64_t frac, int64_t inv_sqrt, int64_t *out) {
  if (hd > 256) return 1;
  return imo_attention_ld(q, k, v, H, Hkv, hd, M, L, L, start, frac, inv_sqrt, out);
}

// The synthetic stream of oracle/prng.py `uniform_int` (counter-based SplitMix64): element i of tensor (seed, tid)
// is (mix(key + (i + 1) * gamma) mod span) + lo, key = mix(seed * 0x100000001B3 + tid * 0x9E3779B1 + c). Writes
// elements i = i0 + r * C + c (r < R, c < C) to out[r * ld + c] (ld >= C).
static inline uint64_t sm_mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

int imo_uniform_fill(uint64_t seed, uint64_t tid, int64_t i0, int64_t R, int64_t C, int64_t ld, int64_t lo,
                     uint64_t span, int64_t *out) {
  if (!out || i0 < 0 || R < 0 || C < 0 || ld < C || span == 0) return 1;
  const uint64_t key = sm_mix(seed * 0x100000001B3ull + tid * 0x9E3779B1ull + 0x632BE59BD9B4E019ull);
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < R; ++r)
    for (int64_t c = 0; c < C; ++c) {
      const uint64_t i = (uint64_t)(i0 + r * C + c);
      out[r * ld + c] = (int64_t)(sm_mix(key + (i + 1) * 0x9E3779B97F4A7C15ull) % span) + lo;
    }
  return 0;
}

// ---------------------------------------------------------------------------------------------------------
// nmc Q4_K / Q6_K exact linear (qk_codec.py:28-206, cohere2.py:102-106)
// ---------------------------------------------------------------------------------------------------------
// round-half-even(fp16 * 2^fw) computed in integers from the fp16 bits (no libm, no FP rounding mode).
int64_t imo_fp16_fixed(uint16_t h, int fw) {
  const int sign = (h >> 15) & 1, e = (h >> 10) & 31;
  const int64_t mant = h & 0x3FF;
  int64_t m;
  int sh;
  if (e == 0) { m = mant; sh = fw - 24; }
  else { m = mant | 0x400; sh = e - 25 + fw; }
  int64_t r;
  if (sh >= 0) r = m << sh;
  else {
    const int s = -sh;
    if (s >= 63) r = 0;
    else {
      const int64_t q = m >> s, rem = m & (((int64_t)1 << s) - 1), half = (int64_t)1 << (s - 1);
      r = q + ((rem > half || (rem == half && (q & 1))) ? 1 : 0);
    }
  }
  return sign ? -r : r;
}

static inline void scale_min_k4(int j, const uint8_t *q, int *d, int *m) {
  if (j < 4) { *d = q[j] & 63; *m = q[j + 4] & 63; }
  else { *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4); *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4); }
}

void imo_dequant_block(const uint8_t *blk, int qtype, int fw, int64_t *wb) {
  if (qtype == 0) {
    const int64_t dq = imo_fp16_fixed((uint16_t)(blk[0] | (blk[1] << 8)), fw);
    const int64_t dmq = imo_fp16_fixed((uint16_t)(blk[2] | (blk[3] << 8)), fw);
    const uint8_t *sc = blk + 4, *qs = blk + 16;
    for (int g = 0; g < 4; ++g) {
      int s, m;
      scale_min_k4(2 * g, sc, &s, &m);
      for (int l = 0; l < 32; ++l) wb[64 * g + l] = dq * s * (qs[32 * g + l] & 0xF) - dmq * m;
      scale_min_k4(2 * g + 1, sc, &s, &m);
      for (int l = 0; l < 32; ++l) wb[64 * g + 32 + l] = dq * s * (qs[32 * g + l] >> 4) - dmq * m;
    }
  } else {
    const uint8_t *ql = blk, *qh = blk + 128;
    const int8_t *sc = (const int8_t *)(blk + 192);
    const int64_t dq = imo_fp16_fixed((uint16_t)(blk[208] | (blk[209] << 8)), fw);
    for (int half = 0; half < 2; ++half) {
      const int qlo = 64 * half, qho = 32 * half, sco = 8 * half, yo = 128 * half;
      for (int l = 0; l < 32; ++l) {
        const int is = l / 16;
        const int64_t q1 = ((ql[qlo + l] & 0xF) | (((qh[qho + l] >> 0) & 3) << 4)) - 32;
        const int64_t q2 = ((ql[qlo + l + 32] & 0xF) | (((qh[qho + l] >> 2) & 3) << 4)) - 32;
        const int64_t q3 = ((ql[qlo + l] >> 4) | (((qh[qho + l] >> 4) & 3) << 4)) - 32;
        const int64_t q4 = ((ql[qlo + l + 32] >> 4) | (((qh[qho + l] >> 6) & 3) << 4)) - 32;
        wb[yo + l] = dq * sc[sco + is + 0] * q1;
        wb[yo + l + 32] = dq * sc[sco + is + 2] * q2;
        wb[yo + l + 64] = dq * sc[sco + is + 4] * q3;
        wb[yo + l + 96] = dq * sc[sco + is + 6] * q4;
      }
    }
  }
}

// out[t, o] = floor((sum_i W[o,i] * x[t,i]) / 2^fw) exactly; rc 2 if any result leaves int64.
int imo_qk_linear(const uint8_t *W, const int64_t *x, int64_t T, int64_t out_f, int64_t nb, int fw, int qtype,
                  int64_t *out) {
  if (!W || !x || !out || T < 0 || out_f < 0 || nb <= 0 || fw < 0 || fw > 62 || (qtype != 0 && qtype != 1)) return 1;
  const int64_t in_f = nb * 256, bs = qtype == 0 ? 144 : 210;
  int rc = 0;
#pragma omp parallel reduction(max : rc)
  {
    int64_t *wb = (int64_t *)malloc((size_t)in_f * 8);
#pragma omp for schedule(static)
    for (int64_t o = 0; o < out_f; ++o) {
      for (int64_t b = 0; b < nb; ++b) imo_dequant_block(W + (o * nb + b) * bs, qtype, fw, wb + b * 256);
      for (int64_t t = 0; t < T; ++t) {
        const int64_t *xt = x + t * in_f;
        i128 acc = 0;
        for (int64_t i = 0; i < in_f; ++i) acc += (i128)wb[i] * xt[i];
        const i128 y = acc >> fw;
        if (y > INT64_MAX || y < INT64_MIN) rc = 2;
        out[t * out_f + o] = (int64_t)y;
      }
    }
    free(wb);
  }
  return rc;
}
