// north-mini-code resident preprocessing and attention bank (gfx950): the steps either side of the MoE block.
//   int64 matrices                  nmc_qk_cuda.cu:1068 `qk_register_i64` (qk_cuda.py:285-303)
//   RMSNorm + router + top-k        nmc_qk_cuda.cu:1116 `qk_rmsnorm_router` (qk_cuda.py:331-372); semantics
//                                   cohere2.py:162-188 (router = exact linear >> fw, lowest-index top-k, sigmoid
//                                   gates without the 2^62 / log2e cap, nmc/_bonsai/fixedpoint.py:148)
//   attention bank                  nmc_qk_cuda.cu:877-1040, :1363-1780 (qk_cuda.py:476-715): per-request K/V
//                                   per layer, M = 1 decode: Q/K/V -> interleaved RoPE (cohere2.py:125-133,
//                                   nmc/_bonsai/rope.py:79-100) -> K/V append -> GQA fixed-point attention over
//                                   the window (cohere2.py:136-161) -> O; MoE layer begin / continue with the
//                                   parallel residual x + Attn(n(x)) + MoE(n(x)) (cohere2.py:191-199)
// Guards follow the reference producer: a RoPE / attention / router / RMSNorm envelope miss returns 3 and
// poisons the bank layer (its K/V length does not advance).
#include "imie_common.h"
#include "imie_kernels.h"
#include <string.h>
#include <climits>

int imie_qk_info(int64_t h, int64_t* out_f, int64_t* nb, int* qtype, const uint8_t** p);
int64_t imie_qk_register_i64(const int64_t* W, int64_t rows, int64_t cols);
int imie_qk_linear_dev(int64_t h, const int64_t* x, int64_t T, int fw, int64_t* out, int* status, hipStream_t st);
int imie_qk_moe_dev(const long long* gate_h, const long long* up_h, const long long* down_h, int k,
                    const int64_t* h_dev, const int64_t* gates_dev, int64_t d_model, int64_t e_ffn, int fa, int fw,
                    int64_t* out_dev, hipStream_t st);

namespace {

typedef __int128 i128;
typedef unsigned __int128 u128;
constexpr int kGuard = 8;                             // bank status bit: an exact envelope guard fired

__device__ inline uint64_t nb_uabs(int64_t v) { return v < 0 ? 0 - (uint64_t)v : (uint64_t)v; }

__device__ inline int64_t nb_exp2_neg(int64_t u, int fa) {     // fixedpoint.py:74-96
  const int64_t fp = (int64_t)1 << fa;
  const int64_t k = u >> fa, f = u & (fp - 1);
  const int sh = 16 - fa;
  int64_t c0, c1, c2, c3;
  if (sh >= 0) { c0 = 65536 >> sh; c1 = 45426 >> sh; c2 = 15743 >> sh; c3 = 3638 >> sh; }
  else { c0 = (int64_t)65536 << -sh; c1 = (int64_t)45426 << -sh; c2 = (int64_t)15743 << -sh; c3 = (int64_t)3638 << -sh; }
  const int64_t f2 = (int64_t)((uint64_t)f * (uint64_t)f) >> fa;
  const int64_t f3 = (int64_t)((uint64_t)f2 * (uint64_t)f) >> fa;
  int64_t poly = c0 - ((int64_t)((uint64_t)c1 * (uint64_t)f) >> fa) + ((int64_t)((uint64_t)c2 * (uint64_t)f2) >> fa) -
                 ((int64_t)((uint64_t)c3 * (uint64_t)f3) >> fa);
  if (poly < 0) poly = 0;
  if (k < 0) return 0;
  return poly >> (k < 63 ? k : 63);
}

__device__ inline int64_t nb_log2e(int fa) {
  const int sh = 16 - fa;
  return sh >= 0 ? (94548 >> sh) : ((int64_t)94548 << -sh);
}

// gate sigmoid (the nmc variant: d_clip without the 2^62 / log2e cap)
__device__ inline int64_t nb_sigmoid(int64_t x, int fa) {
  const int64_t l = nb_log2e(fa), dclip = ((int64_t)(fa + 2) << (2 * fa)) / l;
  const int64_t m = x > 0 ? x : 0;
  int64_t d0 = m, d1 = (int64_t)((uint64_t)m - (uint64_t)x);
  if (d0 > dclip) d0 = dclip;
  if (d1 > dclip) d1 = dclip;
  const int64_t e0 = nb_exp2_neg((int64_t)((uint64_t)d0 * (uint64_t)l) >> fa, fa);
  const int64_t e1 = nb_exp2_neg((int64_t)((uint64_t)d1 * (uint64_t)l) >> fa, fa);
  const int64_t z = e0 + e1;
  return z == 0 ? 0 : (int64_t)(((u128)(uint64_t)e1 << fa) / (u128)(uint64_t)z);
}

// block max of u64 (256 threads); result in every thread
__device__ inline uint64_t nb_block_max(uint64_t v) {
  __shared__ uint64_t s[4];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint64_t u = (uint64_t)__shfl_xor((long long)v, o, 64);
    v = u > v ? u : v;
  }
  __syncthreads();
  if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = v;
  __syncthreads();
  uint64_t m = 0;
  for (int k = 0; k < (int)(blockDim.x >> 6); ++k) m = s[k] > m ? s[k] : m;
  return m;
}

// router: logits[r, e] = (sum_i h[r, i] * W[e, i]) >> fw, exact; the unshifted sum must fit int64
// (nmc_qk_cuda.cu:560-638). One workgroup per (row, expert): when max|h| * max|w| * width fits int64 the int64
// sum is exact; otherwise one thread runs the exact int128 sum with per-term overflow checks.
__global__ __launch_bounds__(256) void nb_router_kernel(const int64_t* __restrict__ h, int64_t width,
                                                        const int64_t* __restrict__ W, int experts, int fw,
                                                        int64_t* __restrict__ logits, int* __restrict__ status) {
  __shared__ int64_t s_sum[4];
  const int64_t row = blockIdx.y;
  const int e = blockIdx.x;
  const int64_t* hr = h + row * width;
  const int64_t* wr = W + (int64_t)e * width;
  uint64_t mh = 0, mw = 0;
  for (int64_t i = threadIdx.x; i < width; i += 256) {
    const uint64_t a = nb_uabs(hr[i]), b = nb_uabs(wr[i]);
    mh = a > mh ? a : mh;
    mw = b > mw ? b : mw;
  }
  mh = nb_block_max(mh);
  mw = nb_block_max(mw);
  const bool fast = mh == 0 || mw == 0 || (u128)mh * mw * (u128)(uint64_t)width <= (u128)INT64_MAX;
  if (fast) {
    int64_t acc = 0;
    for (int64_t i = threadIdx.x; i < width; i += 256) acc += hr[i] * wr[i];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) acc += (int64_t)__shfl_xor((long long)acc, o, 64);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) s_sum[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) logits[row * experts + e] = (s_sum[0] + s_sum[1] + s_sum[2] + s_sum[3]) >> fw;
    return;
  }
  if (threadIdx.x) return;
  const i128 mx = (i128)(((u128)1 << 127) - 1), mn = -mx - 1;
  i128 acc = 0;
  for (int64_t i = 0; i < width; ++i) {
    const i128 t = (i128)hr[i] * wr[i];
    if ((t > 0 && acc > mx - t) || (t < 0 && acc < mn - t)) {
      atomicOr(status, kGuard);
      logits[row * experts + e] = 0;
      return;
    }
    acc += t;
  }
  if (acc > (i128)INT64_MAX || acc < (i128)INT64_MIN) {
    atomicOr(status, kGuard);
    logits[row * experts + e] = 0;
    return;
  }
  logits[row * experts + e] = (int64_t)acc >> fw;
}

// lowest-index top-k by logit and their sigmoid gates (cohere2.py:162-165, :181-182); one thread per row
__global__ void nb_topk_kernel(const int64_t* __restrict__ logits, int64_t rows, int experts, int used, int fa,
                               int* __restrict__ ids, int64_t* __restrict__ gates) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const int64_t* lr = logits + r * experts;
  for (int k = 0; k < used; ++k) {
    int best_id = -1;
    int64_t best = INT64_MIN;
    for (int e = 0; e < experts; ++e) {
      bool taken = false;
      for (int j = 0; j < k; ++j) taken = taken || ids[r * used + j] == e;
      if (!taken && (best_id < 0 || lr[e] > best)) { best = lr[e]; best_id = e; }
    }
    ids[r * used + k] = best_id;
    gates[r * used + k] = nb_sigmoid(best, fa);
  }
}

// interleaved RoPE of q (H heads) and k (Hkv heads) at position pos, with the reference's envelope guard
// (2 max|x| max|cos, sin| <= INT64_MAX, rope.py:26-39) and exact per-element checks; one workgroup
__global__ __launch_bounds__(256) void nb_rope_kernel(int64_t* __restrict__ q, int64_t nq, int64_t* __restrict__ k,
                                                      int64_t nk, int hd, const int64_t* __restrict__ cs,
                                                      const int64_t* __restrict__ sn, int64_t pos, int fa,
                                                      int* __restrict__ status) {
  const int half = hd / 2;
  const int64_t* c = cs + pos * half;
  const int64_t* s = sn + pos * half;
  uint64_t mq = 0, mk = 0, mc = 0;
  for (int64_t i = threadIdx.x; i < nq; i += 256) { const uint64_t a = nb_uabs(q[i]); mq = a > mq ? a : mq; }
  for (int64_t i = threadIdx.x; i < nk; i += 256) { const uint64_t a = nb_uabs(k[i]); mk = a > mk ? a : mk; }
  for (int i = threadIdx.x; i < half; i += 256) {
    const uint64_t a = nb_uabs(c[i]), b = nb_uabs(s[i]);
    mc = a > mc ? a : mc;
    mc = b > mc ? b : mc;
  }
  mq = nb_block_max(mq);
  mk = nb_block_max(mk);
  mc = nb_block_max(mc);
  if ((u128)2 * mq * mc > (u128)INT64_MAX || (u128)2 * mk * mc > (u128)INT64_MAX) {
    if (threadIdx.x == 0) atomicOr(status, kGuard);
    return;
  }
  for (int64_t i = threadIdx.x; i < (nq + nk) / 2; i += 256) {
    int64_t* x = i < nq / 2 ? q + 2 * i : k + 2 * (i - nq / 2);
    const int pr = (int)((i < nq / 2 ? i : i - nq / 2) % half);
    const int64_t a = x[0], b = x[1];
    const i128 p0 = (i128)a * c[pr] - (i128)b * s[pr], p1 = (i128)a * s[pr] + (i128)b * c[pr];
    if (p0 > (i128)INT64_MAX || p0 < (i128)INT64_MIN || p1 > (i128)INT64_MAX || p1 < (i128)INT64_MIN) {
      atomicOr(status, kGuard);
      continue;
    }
    x[0] = (int64_t)p0 >> fa;
    x[1] = (int64_t)p1 >> fa;
  }
}

// K / V append at `pos` (cache [Hkv][max_len][hd]) and the running max|K|, max|V| (kv_max[0..1])
__global__ __launch_bounds__(256) void nb_append_kernel(const int64_t* __restrict__ k, const int64_t* __restrict__ v,
                                                        int nkv, int hd, int64_t pos, int64_t max_len,
                                                        int64_t* __restrict__ ck, int64_t* __restrict__ cv,
                                                        uint64_t* __restrict__ kv_max) {
  uint64_t mk = 0, mv = 0;
  for (int64_t i = threadIdx.x; i < (int64_t)nkv * hd; i += 256) {
    const int64_t h = i / hd, l = i - h * hd;
    const int64_t dst = (h * max_len + pos) * hd + l;
    ck[dst] = k[i];
    cv[dst] = v[i];
    const uint64_t a = nb_uabs(k[i]), b = nb_uabs(v[i]);
    mk = a > mk ? a : mk;
    mv = b > mv ? b : mv;
  }
  mk = nb_block_max(mk);
  mv = nb_block_max(mv);
  if (threadIdx.x == 0) {
    if (mk > kv_max[0]) kv_max[0] = mk;
    if (mv > kv_max[1]) kv_max[1] = mv;
  }
}

// max|x| of n values into out (one workgroup)
__global__ __launch_bounds__(256) void nb_maxabs_kernel(const int64_t* __restrict__ x, int64_t n,
                                                        uint64_t* __restrict__ out) {
  uint64_t m = 0;
  for (int64_t i = threadIdx.x; i < n; i += 256) { const uint64_t a = nb_uabs(x[i]); m = a > m ? a : m; }
  m = nb_block_max(m);
  if (threadIdx.x == 0) *out = m;
}

// GQA fixed-point attention of the new position `pos` over keys [first, pos] (sliding window when window > 0):
// score = (((q . k) >> fa) * inv_sqrt) >> fa, softmax of the 2^-d cubic, out = (p . V) >> fa; every int64
// narrowing is checked (nmc_qk_cuda.cu:343-432). One workgroup per query head; scores in prob (global).
__global__ __launch_bounds__(256) void nb_attention_kernel(const int64_t* __restrict__ q, const int64_t* __restrict__ ck,
                                                           const int64_t* __restrict__ cv, int heads, int nkv, int hd,
                                                           int64_t pos, int64_t max_len, int window, int fa,
                                                           int64_t inv_sqrt, const uint64_t* __restrict__ qmax,
                                                           const uint64_t* __restrict__ kv_max,
                                                           int64_t* __restrict__ prob, int64_t* __restrict__ out,
                                                           int* __restrict__ status) {
  __shared__ int64_t s_v[4];
  __shared__ uint64_t s_z[4];
  const int head = blockIdx.x, kv = head / (heads / nkv), t = threadIdx.x;
  // envelope (max|q| max|K| hd and 2^fa max|V| within int64), checked once
  if (head == 0 && t == 0 &&
      ((u128)qmax[0] * kv_max[0] * (u128)(uint64_t)hd > (u128)INT64_MAX ||
       ((u128)1 << fa) * kv_max[1] > (u128)INT64_MAX))
    atomicOr(status, kGuard);
  const int64_t first = (window > 0 && pos - window >= 0) ? pos - window + 1 : 0;
  const int64_t* qh = q + (int64_t)head * hd;
  int64_t* ph = prob + (int64_t)head * max_len;
  int64_t best = INT64_MIN;
  for (int64_t key = first + t; key <= pos; key += 256) {
    const int64_t* kh = ck + ((int64_t)kv * max_len + key) * hd;
    i128 acc = 0;
    for (int l = 0; l < hd; ++l) acc += (i128)qh[l] * kh[l];
    const i128 sh = acc >> fa, sc = (sh * inv_sqrt) >> fa;
    int64_t score = 0;
    if (sh > (i128)INT64_MAX || sh < (i128)INT64_MIN || sc > (i128)INT64_MAX || sc < (i128)INT64_MIN)
      atomicOr(status, kGuard);
    else
      score = (int64_t)sc;
    ph[key] = score;
    best = score > best ? score : best;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const int64_t u = (int64_t)__shfl_xor((long long)best, o, 64);
    best = u > best ? u : best;
  }
  if ((t & 63) == 0) s_v[t >> 6] = best;
  __syncthreads();
  best = s_v[0];
  for (int k = 1; k < 4; ++k) best = s_v[k] > best ? s_v[k] : best;
  const int64_t l2 = nb_log2e(fa);
  int64_t dclip = ((int64_t)(fa + 2) << (2 * fa)) / l2;
  const int64_t hard = ((int64_t)1 << 62) / l2;
  dclip = hard < dclip ? hard : dclip;
  uint64_t z = 0;
  for (int64_t key = first + t; key <= pos; key += 256) {
    const i128 wide = (i128)best - ph[key];
    const int64_t d = wide > dclip ? dclip : (wide < 0 ? 0 : (int64_t)wide);
    const int64_t e = nb_exp2_neg((int64_t)((uint64_t)d * (uint64_t)l2) >> fa, fa);
    ph[key] = e;
    z += (uint64_t)e;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) z += (uint64_t)__shfl_xor((long long)z, o, 64);
  __syncthreads();
  if ((t & 63) == 0) s_z[t >> 6] = z;
  __syncthreads();
  const uint64_t Z = s_z[0] + s_z[1] + s_z[2] + s_z[3];
  if (Z != 0)
    for (int64_t key = first + t; key <= pos; key += 256)
      ph[key] = (int64_t)(((u128)(uint64_t)ph[key] << fa) / (u128)Z);
  __syncthreads();
  for (int l = t; l < hd; l += 256) {
    i128 acc = 0;
    if (Z != 0)
      for (int64_t key = first; key <= pos; ++key) acc += (i128)ph[key] * cv[((int64_t)kv * max_len + key) * hd + l];
    i128 sh = acc >> fa;
    if (sh > (i128)INT64_MAX || sh < (i128)INT64_MIN) { atomicOr(status, kGuard); sh = 0; }
    out[(int64_t)head * hd + l] = (int64_t)sh;
  }
}

// next = residual + attention + moe, int64 wrap (the reference's committed numpy int64 addition)
__global__ void nb_add3_kernel(const int64_t* __restrict__ a, const int64_t* __restrict__ b,
                               const int64_t* __restrict__ c, int64_t n, int64_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = (int64_t)((uint64_t)a[i] + (uint64_t)b[i] + (uint64_t)c[i]);
}

struct Binding { long long g = -1, u = -1, d = -1; bool bound = false; };

struct Layer {
  DevBuf k, v, kvmax;                                 // [Hkv][max_len][hd] int64 each; running max|K|, max|V|
  int64_t length = 0;
  bool poisoned = false;
  int experts = 0, used = 0;
  int64_t d_model = 0, e_ffn = 0;
  std::vector<Binding> bind;
  std::vector<int> pending_cold;
};

struct Bank {
  bool live = false;
  int n_layers = 0, heads = 0, nkv = 0, hd = 0, fa = 0;
  int64_t max_len = 0, d_model = 0;
  DevBuf cos, sin;
  std::vector<Layer> layers;
  DevBuf res[2], norm, logits, ids, gates, attn, qkv, ao, prob, status, qmax, moe;
  int res_slot = 0;
  bool has_res = false;
  int retained = -1;
  bool pending = false;
  int pending_layer = -1;
  std::vector<int> route_ids;                         // the pending layer's selected experts
};

std::vector<Bank>& banks() {
  static std::vector<Bank> v;
  return v;
}

Bank* bank_get(long long h) {
  if (h < 0 || h >= (long long)banks().size() || !banks()[(size_t)h].live) return nullptr;
  return &banks()[(size_t)h];
}

bool quant_handle(long long h, int64_t* out_f, int64_t* nb) {
  int qt = -1;
  return imie_qk_info(h, out_f, nb, &qt, nullptr) == IMIE_OK && (qt == 0 || qt == 1);
}

int ensure_layer_kv(Bank& b, Layer& L) {
  const size_t bytes = (size_t)(b.nkv * b.max_len * b.hd) * 8;
  if (!L.k.p) {
    if (L.k.ensure(bytes) || L.v.ensure(bytes) || L.kvmax.ensure(16)) return IMIE_EARG;
    IMIE_HIP(hipMemset(L.kvmax.p, 0, 16));
  }
  return IMIE_OK;
}

size_t bank_bytes(const Bank& b) {
  size_t t = b.cos.cap + b.sin.cap;
  for (const DevBuf* d : {&b.res[0], &b.res[1], &b.norm, &b.logits, &b.ids, &b.gates, &b.attn, &b.qkv, &b.ao, &b.prob,
                          &b.status, &b.qmax, &b.moe})
    t += d->cap;
  for (const Layer& L : b.layers) t += L.k.cap + L.v.cap + L.kvmax.cap;
  return t;
}

void bank_release(Bank& b) {
  (void)hipStreamSynchronize(imie_stream());
  for (Layer& L : b.layers) { L.k.release(); L.v.release(); L.kvmax.release(); }
  for (DevBuf* d : {&b.cos, &b.sin, &b.res[0], &b.res[1], &b.norm, &b.logits, &b.ids, &b.gates, &b.attn, &b.qkv,
                    &b.ao, &b.prob, &b.status, &b.qmax, &b.moe})
    d->release();
  b = Bank();
}

// validate the attention handles / window and reserve the layer's storage (qk_cuda.py:548-572 envelope)
int attention_preflight(Bank& b, int layer, long long qh, long long kh, long long vh, long long oh, int window) {
  if (layer < 0 || layer >= b.n_layers || window == 0 || window < -1) return IMIE_EARG;
  Layer& L = b.layers[(size_t)layer];
  if (L.poisoned || L.length >= b.max_len) return IMIE_EARG;
  const int64_t qw = (int64_t)b.heads * b.hd, kw = (int64_t)b.nkv * b.hd;
  int64_t of[4], nb[4];
  const long long hs[4] = {qh, kh, vh, oh};
  for (int i = 0; i < 4; ++i) if (!quant_handle(hs[i], &of[i], &nb[i])) return IMIE_EARG;
  if (nb[0] * 256 != b.d_model || nb[1] * 256 != b.d_model || nb[2] * 256 != b.d_model || of[0] != qw ||
      of[1] != kw || of[2] != kw || nb[3] * 256 != qw || of[3] != b.d_model)
    return IMIE_EARG;
  if (ensure_layer_kv(b, L) || b.qkv.ensure((size_t)(qw + 2 * kw) * 8) || b.attn.ensure((size_t)qw * 8) ||
      b.ao.ensure((size_t)b.d_model * 8) || b.prob.ensure((size_t)(b.heads * b.max_len) * 8) ||
      b.status.ensure(64) || b.qmax.ensure(64))
    return IMIE_EARG;
  return IMIE_OK;
}

// normalized x (device) -> Q/K/V -> RoPE -> append -> attention -> O into b.ao; enqueued on st (no sync)
int attention_enqueue(Bank& b, int layer, long long qh, long long kh, long long vh, long long oh, const int64_t* x,
                      int fw, int window, int rope, int64_t inv_sqrt, hipStream_t st) {
  Layer& L = b.layers[(size_t)layer];
  const int64_t qw = (int64_t)b.heads * b.hd, kw = (int64_t)b.nkv * b.hd;
  int64_t* q = (int64_t*)b.qkv.p;
  int64_t *k = q + qw, *v = k + kw;
  int* status = (int*)b.status.p;
  int rc = imie_qk_linear_dev(qh, x, 1, fw, q, status, st);
  if (!rc) rc = imie_qk_linear_dev(kh, x, 1, fw, k, status, st);
  if (!rc) rc = imie_qk_linear_dev(vh, x, 1, fw, v, status, st);
  if (rc) return rc;
  if (rope)
    hipLaunchKernelGGL(nb_rope_kernel, dim3(1), dim3(256), 0, st, q, qw, k, kw, b.hd, (const int64_t*)b.cos.p,
                       (const int64_t*)b.sin.p, L.length, b.fa, status);
  hipLaunchKernelGGL(nb_append_kernel, dim3(1), dim3(256), 0, st, (const int64_t*)k, (const int64_t*)v, b.nkv, b.hd,
                     L.length, b.max_len, (int64_t*)L.k.p, (int64_t*)L.v.p, (uint64_t*)L.kvmax.p);
  hipLaunchKernelGGL(nb_maxabs_kernel, dim3(1), dim3(256), 0, st, (const int64_t*)q, qw, (uint64_t*)b.qmax.p);
  hipLaunchKernelGGL(nb_attention_kernel, dim3((unsigned)b.heads), dim3(256), 0, st, (const int64_t*)q,
                     (const int64_t*)L.k.p, (const int64_t*)L.v.p, b.heads, b.nkv, b.hd, L.length, b.max_len, window,
                     b.fa, inv_sqrt, (const uint64_t*)b.qmax.p, (const uint64_t*)L.kvmax.p, (int64_t*)b.prob.p,
                     (int64_t*)b.attn.p, status);
  IMIE_HIP(hipGetLastError());
  return imie_qk_linear_dev(oh, (const int64_t*)b.attn.p, 1, fw, (int64_t*)b.ao.p, status, st);
}

// status after the enqueued work: 0 ok, 3 a guard fired (layer poisoned), 1 runtime failure
int finish(Bank& b, Layer& L, hipStream_t st) {
  int stat = 0;
  if (hipMemcpyAsync(&stat, b.status.p, 4, hipMemcpyDeviceToHost, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess) {
    L.poisoned = true;
    return IMIE_EARG;
  }
  if (stat) { L.poisoned = true; return 3; }
  return IMIE_OK;
}

int64_t imie_rmsnorm_eps(unsigned long long eps) { return eps > (unsigned long long)INT64_MAX ? -1 : (int64_t)eps; }

}  // namespace

extern "C" {

// nmc_qk_cuda.cu:1068 `qk_register_i64` (qk_cuda.py:285-303): dense int64 [rows, cols] (norm gains, router)
long long qk_register_i64(const int64_t* W, long long rows, long long cols) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  return imie_qk_register_i64(W, rows, cols);
}

// nmc_qk_cuda.cu:1116 `qk_rmsnorm_router` (qk_cuda.py:331-372): h = RMSNorm(x) with the resident gain, router
// logits, lowest-index top-`used` ids and their sigmoid gates. rc 3: an exact envelope rejection (the caller
// runs its host path); 1: bad arguments.
int qk_rmsnorm_router(long long gain_h, long long router_h, const int64_t* x, long long rows, int fa, int fw,
                      unsigned long long eps, int used, long long h_capacity, long long route_capacity,
                      int64_t* h_out, int* ids_out, int64_t* gates_out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  int64_t grows = 0, gcols = 0, rrows = 0, rcols = 0;
  int gq = -1, rq = -1;
  const uint8_t *gp = nullptr, *rp = nullptr;
  if (imie_qk_info(gain_h, &grows, &gcols, &gq, &gp) || imie_qk_info(router_h, &rrows, &rcols, &rq, &rp) || !x ||
      !h_out || !ids_out || !gates_out || rows <= 0 || used <= 0 || fa < 1 || fa > 29 || fw < 0 || fw > 62)
    return IMIE_EARG;
  const int64_t e = imie_rmsnorm_eps(eps);
  if (gq != 2 || rq != 2 || grows != 1 || rcols != gcols || rrows <= 0 || rrows > INT_MAX || used > rrows || e < 0 ||
      rows * gcols > h_capacity || rows * used > route_capacity)
    return IMIE_EARG;
  hipStream_t st = imie_stream();
  static DevBuf dx, dh, dl, di, dg, ds;
  const int64_t width = gcols;
  if (dx.ensure((size_t)(rows * width) * 8) || dh.ensure((size_t)(rows * width) * 8) ||
      dl.ensure((size_t)(rows * rrows) * 8) || di.ensure((size_t)(rows * used) * 4) ||
      dg.ensure((size_t)(rows * used) * 8) || ds.ensure(64))
    return IMIE_EARG;
  IMIE_HIP(hipMemcpyAsync(dx.p, x, (size_t)(rows * width) * 8, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemsetAsync(ds.p, 0, 4, st));
  int rc = imie_rmsnorm_launch((const int64_t*)dx.p, rows, width, fa, e, (const int64_t*)gp, (int64_t*)dh.p,
                               (int*)ds.p, st);
  if (rc) return rc;
  hipLaunchKernelGGL(nb_router_kernel, dim3((unsigned)rrows, (unsigned)rows), dim3(256), 0, st, (const int64_t*)dh.p,
                     width, (const int64_t*)rp, (int)rrows, fw, (int64_t*)dl.p, (int*)ds.p);
  hipLaunchKernelGGL(nb_topk_kernel, dim3((unsigned)((rows + 63) / 64)), dim3(64), 0, st, (const int64_t*)dl.p, rows,
                     (int)rrows, used, fa, (int*)di.p, (int64_t*)dg.p);
  IMIE_HIP(hipGetLastError());
  int stat = 0;
  IMIE_HIP(hipMemcpyAsync(&stat, ds.p, 4, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipStreamSynchronize(st));
  if (stat) return 3;
  IMIE_HIP(hipMemcpy(h_out, dh.p, (size_t)(rows * width) * 8, hipMemcpyDeviceToHost));
  IMIE_HIP(hipMemcpy(ids_out, di.p, (size_t)(rows * used) * 4, hipMemcpyDeviceToHost));
  IMIE_HIP(hipMemcpy(gates_out, dg.p, (size_t)(rows * used) * 8, hipMemcpyDeviceToHost));
  return IMIE_OK;
}

// nmc_qk_cuda.cu:877 `qk_attention_bank_create` (qk_cuda.py:486-519): handle >= 0 or -1
long long qk_attention_bank_create(int n_layers, long long max_length, long long d_model, int heads, int n_kv,
                                   int head_dim, int fa, const int64_t* cos, const int64_t* sin) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!cos || !sin || n_layers <= 0 || max_length <= 0 || d_model <= 0 || d_model % 256 || heads <= 0 || n_kv <= 0 ||
      heads % n_kv || head_dim <= 0 || head_dim % 2 || fa < 1 || fa > 29 || ((int64_t)heads * head_dim) % 256 ||
      imie_device_ready() != 0)
    return -1;
  auto& bs = banks();
  size_t slot = bs.size();
  for (size_t i = 0; i < bs.size(); ++i) if (!bs[i].live) { slot = i; break; }
  if (slot == bs.size()) bs.emplace_back();
  Bank& b = bs[slot];
  b = Bank();
  const size_t tb = (size_t)(max_length * (head_dim / 2)) * 8;
  if (b.cos.ensure(tb) || b.sin.ensure(tb) || hipMemcpy(b.cos.p, cos, tb, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(b.sin.p, sin, tb, hipMemcpyHostToDevice) != hipSuccess) {
    bank_release(b);
    return -1;
  }
  b.n_layers = n_layers; b.max_len = max_length; b.d_model = d_model; b.heads = heads; b.nkv = n_kv;
  b.hd = head_dim; b.fa = fa;
  b.layers.resize((size_t)n_layers);
  b.live = true;
  return (long long)slot;
}

// nmc_qk_cuda.cu:914 `qk_attention_bank_reset`
int qk_attention_bank_reset(long long h) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  Bank* b = bank_get(h);
  if (!b) return IMIE_EARG;
  for (Layer& L : b->layers) {
    L.length = 0;
    L.poisoned = false;
    L.pending_cold.clear();
    if (L.kvmax.p) IMIE_HIP(hipMemset(L.kvmax.p, 0, 16));
  }
  b->res_slot = 0; b->has_res = false; b->retained = -1; b->pending = false; b->pending_layer = -1;
  return IMIE_OK;
}

// nmc_qk_cuda.cu:927 `qk_attention_bank_destroy`
void qk_attention_bank_destroy(long long h) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  Bank* b = bank_get(h);
  if (b) bank_release(*b);
}

// nmc_qk_cuda.cu:1363 `qk_attention_bank_import` (qk_cuda.py:528-546): K/V [n_kv, length, head_dim] of a prefill
int qk_attention_bank_import(long long h, int layer, const int64_t* k, const int64_t* v, long long length) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  Bank* b = bank_get(h);
  if (!b || !k || !v || layer < 0 || layer >= b->n_layers || length < 0 || length > b->max_len) return IMIE_EARG;
  Layer& L = b->layers[(size_t)layer];
  if (L.poisoned || ensure_layer_kv(*b, L)) return IMIE_EARG;
  const size_t per = (size_t)(length * b->hd);
  std::vector<uint64_t> mx(2, 0);
  for (int hh = 0; hh < b->nkv; ++hh) {
    const size_t dst = (size_t)(hh * b->max_len * b->hd);
    if (per && (hipMemcpy((int64_t*)L.k.p + dst, k + hh * per, per * 8, hipMemcpyHostToDevice) != hipSuccess ||
                hipMemcpy((int64_t*)L.v.p + dst, v + hh * per, per * 8, hipMemcpyHostToDevice) != hipSuccess)) {
      L.poisoned = true;
      return IMIE_EARG;
    }
    for (size_t i = 0; i < per; ++i) {
      const int64_t a = k[hh * per + i], c = v[hh * per + i];
      const uint64_t ua = a < 0 ? 0 - (uint64_t)a : (uint64_t)a, uc = c < 0 ? 0 - (uint64_t)c : (uint64_t)c;
      mx[0] = ua > mx[0] ? ua : mx[0];
      mx[1] = uc > mx[1] ? uc : mx[1];
    }
  }
  IMIE_HIP(hipMemcpy(L.kvmax.p, mx.data(), 16, hipMemcpyHostToDevice));
  L.length = length;
  return IMIE_OK;
}

// nmc_qk_cuda.cu:1530 `qk_attention_bank_apply` (qk_cuda.py:548-572): the attention sublayer output (after O) of
// one normalized hidden row; rc 3 = an exact guard fired (the layer is poisoned).
int qk_attention_bank_apply(long long h, int layer, long long qh, long long kh, long long vh, long long oh,
                            const int64_t* x, int fw, int window, int rope, int64_t inv_sqrt,
                            long long output_capacity, int64_t* out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  Bank* b = bank_get(h);
  if (!b || !x || !out || output_capacity < b->d_model || fw < 0 || fw > 62) return IMIE_EARG;
  if (attention_preflight(*b, layer, qh, kh, vh, oh, window)) return IMIE_EARG;
  if (b->norm.ensure((size_t)b->d_model * 8)) return IMIE_EARG;
  hipStream_t st = imie_stream();
  Layer& L = b->layers[(size_t)layer];
  IMIE_HIP(hipMemcpyAsync(b->norm.p, x, (size_t)b->d_model * 8, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemsetAsync(b->status.p, 0, 4, st));
  int rc = attention_enqueue(*b, layer, qh, kh, vh, oh, (const int64_t*)b->norm.p, fw, window, rope, inv_sqrt, st);
  if (rc) { (void)hipStreamSynchronize(st); L.poisoned = true; return IMIE_EARG; }
  if ((rc = finish(*b, L, st))) return rc;
  IMIE_HIP(hipMemcpy(out, b->ao.p, (size_t)b->d_model * 8, hipMemcpyDeviceToHost));
  ++L.length;
  return IMIE_OK;
}

// nmc_qk_cuda.cu:935 `qk_attention_bank_moe_configure` (qk_cuda.py:574-595): per-layer expert metadata only
int qk_attention_bank_moe_configure(long long h, int layer, int experts, int used, long long d_model,
                                    long long expert_ffn) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  Bank* b = bank_get(h);
  if (!b || layer < 0 || experts <= 0 || used <= 0 || used > experts || d_model <= 0 || expert_ffn <= 0 ||
      d_model % 256 || expert_ffn % 256)
    return IMIE_EARG;
  if (layer >= b->n_layers || d_model != b->d_model || b->pending) return IMIE_EARG;
  Layer& L = b->layers[(size_t)layer];
  if (L.poisoned) return IMIE_EARG;
  if (L.experts)
    return (L.experts == experts && L.used == used && L.d_model == d_model && L.e_ffn == expert_ffn) ? IMIE_OK
                                                                                                     : IMIE_EARG;
  L.experts = experts; L.used = used; L.d_model = d_model; L.e_ffn = expert_ffn;
  L.bind.assign((size_t)experts, Binding());
  L.pending_cold.clear();
  return IMIE_OK;
}

// nmc_qk_cuda.cu:984 `qk_attention_bank_moe_bind` (qk_cuda.py:597-614): one resident expert triplet
int qk_attention_bank_moe_bind(long long h, int layer, int expert, long long gate_h, long long up_h,
                               long long down_h) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  Bank* b = bank_get(h);
  if (!b || layer < 0 || layer >= b->n_layers) return IMIE_EARG;
  Layer& L = b->layers[(size_t)layer];
  if (L.poisoned || expert < 0 || expert >= L.experts) return IMIE_EARG;
  int64_t gof, gnb, uof, unb, dof, dnb;
  if (!quant_handle(gate_h, &gof, &gnb) || !quant_handle(up_h, &uof, &unb) || !quant_handle(down_h, &dof, &dnb))
    return IMIE_EARG;
  if (gof != L.e_ffn || gnb != L.d_model / 256 || uof != L.e_ffn || unb != L.d_model / 256 || dof != L.d_model ||
      dnb != L.e_ffn / 256)
    return IMIE_EARG;
  Binding& bd = L.bind[(size_t)expert];
  if (bd.bound && (bd.g != gate_h || bd.u != up_h || bd.d != down_h)) return IMIE_EARG;
  bd.g = gate_h; bd.u = up_h; bd.d = down_h; bd.bound = true;
  if (b->pending && b->pending_layer == layer)
    for (size_t i = 0; i < L.pending_cold.size(); ++i)
      if (L.pending_cold[i] == expert) { L.pending_cold.erase(L.pending_cold.begin() + (long)i); break; }
  return IMIE_OK;
}

// nmc_qk_cuda.cu:1557 `qk_attention_bank_moe_begin` (qk_cuda.py:616-660): RMSNorm + router + top-k and the
// attention sublayer of one layer, retained on the device; returns the selected experts not yet bound (in
// selected order, without repeats). x is the host hidden row unless use_retained (the previous continuation's).
int qk_attention_bank_moe_begin(long long h, int layer, long long gain_h, long long router_h, long long qh,
                                long long kh, long long vh, long long oh, const int64_t* x, int use_retained, int fw,
                                unsigned long long eps, int window, int rope, int64_t inv_sqrt, int cold_capacity,
                                int* cold_count_out, int* cold_ids_out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  Bank* b = bank_get(h);
  if (!b || layer < 0 || !cold_count_out || !cold_ids_out || use_retained < 0 || use_retained > 1 || fw < 0 ||
      fw > 62 || window == 0 || window < -1)
    return IMIE_EARG;
  if (layer >= b->n_layers || b->pending) return IMIE_EARG;
  Layer& L = b->layers[(size_t)layer];
  int64_t grows, gcols, rrows, rcols;
  int gq = -1, rq = -1;
  const uint8_t *gp = nullptr, *rp = nullptr;
  if (imie_qk_info(gain_h, &grows, &gcols, &gq, &gp) || imie_qk_info(router_h, &rrows, &rcols, &rq, &rp))
    return IMIE_EARG;
  const int64_t e = imie_rmsnorm_eps(eps);
  if (L.poisoned || L.experts <= 0 || !L.pending_cold.empty() || cold_capacity < L.used || gq != 2 || rq != 2 ||
      grows != 1 || gcols != L.d_model || rrows != L.experts || rcols != L.d_model || e < 0)
    return IMIE_EARG;
  if ((!use_retained && !x) || (use_retained && (!b->has_res || b->retained + 1 != layer))) return IMIE_EARG;
  if (attention_preflight(*b, layer, qh, kh, vh, oh, window)) return IMIE_EARG;
  const size_t dm = (size_t)L.d_model;
  if (b->res[0].ensure(dm * 8) || b->res[1].ensure(dm * 8) || b->norm.ensure(dm * 8) ||
      b->logits.ensure((size_t)L.experts * 8) || b->ids.ensure((size_t)L.used * 4) ||
      b->gates.ensure((size_t)L.used * 8) || b->moe.ensure(dm * 8))
    return IMIE_EARG;
  hipStream_t st = imie_stream();
  if (!use_retained) {
    IMIE_HIP(hipMemcpyAsync(b->res[0].p, x, dm * 8, hipMemcpyHostToDevice, st));
    b->res_slot = 0;
  }
  const int64_t* resid = (const int64_t*)b->res[b->res_slot].p;
  int* status = (int*)b->status.p;
  IMIE_HIP(hipMemsetAsync(status, 0, 4, st));
  int rc = imie_rmsnorm_launch(resid, 1, L.d_model, b->fa, e, (const int64_t*)gp, (int64_t*)b->norm.p, status, st);
  if (rc) return rc;
  hipLaunchKernelGGL(nb_router_kernel, dim3((unsigned)L.experts, 1), dim3(256), 0, st, (const int64_t*)b->norm.p,
                     L.d_model, (const int64_t*)rp, L.experts, fw, (int64_t*)b->logits.p, status);
  hipLaunchKernelGGL(nb_topk_kernel, dim3(1), dim3(64), 0, st, (const int64_t*)b->logits.p, (int64_t)1, L.experts,
                     L.used, b->fa, (int*)b->ids.p, (int64_t*)b->gates.p);
  IMIE_HIP(hipGetLastError());
  rc = attention_enqueue(*b, layer, qh, kh, vh, oh, (const int64_t*)b->norm.p, fw, window, rope, inv_sqrt, st);
  if (rc) { (void)hipStreamSynchronize(st); L.poisoned = true; return IMIE_EARG; }
  b->route_ids.assign((size_t)L.used, -1);
  IMIE_HIP(hipMemcpyAsync(b->route_ids.data(), b->ids.p, (size_t)L.used * 4, hipMemcpyDeviceToHost, st));
  if ((rc = finish(*b, L, st))) return rc;
  std::vector<int> cold;
  for (int id : b->route_ids) {
    if (id < 0 || id >= L.experts) { L.poisoned = true; return 3; }
    if (L.bind[(size_t)id].bound) continue;
    bool dup = false;
    for (int c : cold) dup = dup || c == id;
    if (!dup) cold.push_back(id);
  }
  for (size_t i = 0; i < cold.size(); ++i) cold_ids_out[i] = cold[i];
  *cold_count_out = (int)cold.size();
  L.pending_cold = cold;
  ++L.length;
  b->has_res = true; b->pending = true; b->pending_layer = layer;
  return IMIE_OK;
}

// nmc_qk_cuda.cu:1658 `qk_attention_bank_moe_continue` (qk_cuda.py:662-686): the selected experts' MoE and the
// parallel residual x + attention + MoE, retained (publish = 0) or also copied out. rc 4: a selected expert is
// still unbound; rc 3: an envelope guard fired.
int qk_attention_bank_moe_continue(long long h, int layer, int fw, int publish, long long output_capacity,
                                   int64_t* out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  Bank* b = bank_get(h);
  if (!b || layer < 0 || fw < 0 || fw > 62 || publish < 0 || publish > 1 || (publish && (!out || output_capacity <= 0)))
    return IMIE_EARG;
  if (layer >= b->n_layers || !b->pending || b->pending_layer != layer) return IMIE_EARG;
  Layer& L = b->layers[(size_t)layer];
  if (L.poisoned || L.experts <= 0 || (publish && output_capacity < L.d_model)) return IMIE_EARG;
  if (!L.pending_cold.empty()) return 4;
  std::vector<long long> gh, uh, dh;
  for (int id : b->route_ids) {
    const Binding& bd = L.bind[(size_t)id];
    if (!bd.bound) return 4;
    gh.push_back(bd.g); uh.push_back(bd.u); dh.push_back(bd.d);
  }
  hipStream_t st = imie_stream();
  int rc = imie_qk_moe_dev(gh.data(), uh.data(), dh.data(), L.used, (const int64_t*)b->norm.p,
                           (const int64_t*)b->gates.p, L.d_model, L.e_ffn, b->fa, fw, (int64_t*)b->moe.p, st);
  if (rc == IMIE_EOVF) { L.poisoned = true; return 3; }
  if (rc) { L.poisoned = true; return IMIE_EARG; }
  const int next = b->res_slot ^ 1;
  hipLaunchKernelGGL(nb_add3_kernel, dim3((unsigned)((L.d_model + 255) / 256)), dim3(256), 0, st,
                     (const int64_t*)b->res[b->res_slot].p, (const int64_t*)b->ao.p, (const int64_t*)b->moe.p,
                     L.d_model, (int64_t*)b->res[next].p);
  IMIE_HIP(hipGetLastError());
  if (publish) IMIE_HIP(hipMemcpyAsync(out, b->res[next].p, (size_t)L.d_model * 8, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipStreamSynchronize(st));
  b->res_slot = next; b->has_res = true; b->retained = layer; b->pending = false; b->pending_layer = -1;
  return IMIE_OK;
}

// nmc_qk_cuda.cu:1748 `qk_attention_bank_moe_export` (qk_cuda.py:688-699): the retained residual row
int qk_attention_bank_moe_export(long long h, long long output_capacity, int64_t* out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  Bank* b = bank_get(h);
  if (!b || !out || b->pending || !b->has_res || b->retained < 0 || output_capacity < b->d_model) return IMIE_EARG;
  IMIE_HIP(hipMemcpy(out, b->res[b->res_slot].p, (size_t)b->d_model * 8, hipMemcpyDeviceToHost));
  return IMIE_OK;
}

// nmc_qk_cuda.cu:1765 `qk_attention_bank_workspace_bytes`: device bytes owned by the bank (2^64 - 1 if invalid)
unsigned long long qk_attention_bank_workspace_bytes(long long h) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  Bank* b = bank_get(h);
  return b ? (unsigned long long)bank_bytes(*b) : ~0ull;
}

}  // extern "C"
