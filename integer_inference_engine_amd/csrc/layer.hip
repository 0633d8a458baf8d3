// Resident Qwen3-dense (Bonsai) forward over packed Q1_0 weights: the per-layer pipeline, a paged integer KV
// cache, and the reference's monolith / decode-context ABIs on top of them.
//
// Per layer (reference_bonsai.py:941-966, :656-720, :603-615):
//   n1 = rmsnorm(x, n1g); q,k,v = Q1(n1); q,k = head-rmsnorm(q/k); q,k = rope(q/k, pos); cache <- (k, v)
//   x += Q1(attention(q, cache), wo); n2 = rmsnorm(x, n2g); x += Q1((silu(Q1(n2,w1)) * Q1(n2,wu)) >> f, w2)
// Residual adds are fused into the Q1 epilogue (accumulate mode). Positions of the B*M new rows are
// pos = start_b + m; the attention is causal over each sequence's cache.
//
// KV cache: per layer a pool of pages [page][Hkv][P][hd] (int32 or int64); page table [B][mp] shared by the
// layers. int32 storage is guarded: a value that does not fit sets status bit 2 (the caller re-runs with an
// int64 cache). A dense reference cache (B, Hkv, cap, hd) is the case P = cap, mp = 1.
#include "imie_common.h"
#include "imie_kernels.h"
#include <stdlib.h>
#include "imie_attention.h"
#include "imie_kvfmt.h"
#include <string.h>
#include <algorithm>

namespace {

// ---- device buffer registry (bonsai_buf_upload_i64) ---------------------------------------------------------
struct BufEntry {
  int64_t* p = nullptr;
  int64_t n = 0;
};
std::vector<BufEntry>& bufs() {
  static std::vector<BufEntry> b;
  return b;
}
const int64_t* buf_get(int64_t h, int64_t need) {
  if (h < 0 || h >= (int64_t)bufs().size() || !bufs()[(size_t)h].p) return nullptr;
  if (bufs()[(size_t)h].n < need) return nullptr;
  return bufs()[(size_t)h].p;
}

__global__ void fill_i64_kernel(int64_t* p, int64_t n, int64_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// Start of a single-token pass with matvec prologues: workgroup i < ng writes max |gain_i| (over cols) for the
// RMSNorm envelope check; every workgroup clears its share of the RoPE guards and of the zero list (the first
// layer's q, k, v, which its K-split matvec adds into).
__global__ __launch_bounds__(256) void pro_start_kernel(const int64_t* const* __restrict__ gains, int ng, int64_t cols,
                                                        uint64_t* __restrict__ gmax, int64_t* __restrict__ guard,
                                                        int64_t nguard, imie_q1::Q1Zero zero) {
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < nguard; e += (int64_t)gridDim.x * 256) guard[e] = 0;
  imie_q1::zero_share(zero, blockIdx.x, gridDim.x, threadIdx.x, 256);
  if ((int)blockIdx.x >= ng) return;
  const int64_t* g = gains[blockIdx.x];
  uint64_t m = 0;
  for (int64_t c0 = 0; c0 < cols; c0 += 16 * 256) {   // 16 loads in flight per thread
    int64_t v[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int64_t c = c0 + threadIdx.x + 256 * k;
      v[k] = g[c < cols ? c : 0];                      // unconditional: an in-range duplicate changes no maximum
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const uint64_t a = imie_absu64(v[k]);
      m = a > m ? a : m;
    }
  }
  m = imie_wave_max_u64(m);
  __shared__ uint64_t s_m[4];
  if ((threadIdx.x & 63) == 0) s_m[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) m = s_m[w] > m ? s_m[w] : m;
    gmax[blockIdx.x] = m;
  }
}

int fill_i64(int64_t* p, int64_t n, int64_t v, hipStream_t st) {
  if (n <= 0) return IMIE_OK;
  hipLaunchKernelGGL(fill_i64_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p, n, v);
  IMIE_HIP(hipGetLastError());
  return IMIE_OK;
}

// Seeded synthetic cache contents: element i (flattened (kv, j, c) of the (Hkv, len, hd) tensor of one layer,
// kind 0 = K / 1 = V, and sequence b) is uniform in [lo, lo + span) from the counter-based SplitMix64 stream keyed
// by (seed, 100000 + 1024 layer + 512 kind + sequence id) -- the same draw as the host generator's uniform_int.
__device__ inline uint64_t sm_mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void kv_fill_kernel(void* pool, const int64_t* __restrict__ pt, int64_t mp,
                                                      int64_t P, int pshift, int64_t Hkv, int64_t hd,
                                                      const int64_t* __restrict__ lens, const int64_t* __restrict__ sid,
                                                      uint64_t seed, int64_t layer, int kind, int64_t lo,
                                                      uint64_t span, int kv8, uint64_t* __restrict__ run) {
  const int64_t b = blockIdx.z, kv = blockIdx.y;
  const int64_t len = lens[b];
  const int64_t n = len * hd;
  const uint64_t tid = (uint64_t)(100000 + 1024 * layer + 512 * kind + sid[b]);
  const uint64_t key = sm_mix(seed * 0x100000001B3ull + tid * 0x9E3779B1ull + 0x632BE59BD9B4E019ull);
  uint64_t mx = 0;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    // K walks dims fastest and V slots fastest, so consecutive threads store consecutive bytes of a plane
    int64_t j, c;
    if (kind == 0 || !kv8) { j = e / hd; c = e - j * hd; }
    else { c = e / len; j = e - c * len; }
    const uint64_t i = (uint64_t)(kv * len * hd + j * hd + c);
    const int64_t v = (int64_t)(sm_mix(key + (i + 1) * 0x9E3779B97F4A7C15ull) % span) + lo;
    const uint64_t a = imie_absu64(v);
    mx = a > mx ? a : mx;
    const int64_t pg = pt[b * mp + (j >> pshift)], slot = j & (P - 1);
    if (kv8) {
      int8_t* blk = (int8_t*)pool + imie_kv8::block_base(pg, kv, Hkv, hd, P);
      const uint32_t w = imie_kv8::encode(v);
      for (int db = 0; db < 4; ++db) {
        const int64_t off = kind == 0 ? imie_kv8::k_off(slot, db, c, hd) : imie_kv8::v_off(slot, db, c, hd, P);
        blk[off] = (int8_t)(w >> (8 * db));
      }
    } else {
      ((int64_t*)pool)[pg * (Hkv * P * hd) + kv * P * hd + slot * hd + c] = v;
    }
  }
  mx = imie_wave_max_u64(mx);
  if (run && (threadIdx.x & 63) == 0 && mx) atomicMax((unsigned long long*)&run[b * Hkv + kv], (unsigned long long)mx);
}

struct LayerW {
  int64_t w[7];                       // wq, wk, wv, wo, w1, wu, w2 Q1 handles
  const int64_t *n1g, *n2g, *qng, *kng;
};

struct Net {
  int64_t B = 0, d = 0, H = 0, Hkv = 0, hd = 0, dff = 0, nl = 0, vocab = 0, frac = 16, eps = 1, inv_sqrt = 0;
  std::vector<LayerW> layers;
  const int64_t* finalg = nullptr;
  int64_t out_head = -1;
  const int64_t *cos = nullptr, *sin = nullptr;
  int64_t rope_rows = 0;              // positions the uploaded RoPE tables cover (rows of hd/2 entries)
  // KV
  int kv32 = 0;                       // 1: kv8 digit-plane cache (imie_kvfmt.h), 0: int64 rows
  int64_t P = 0, mp = 0, npages = 0;  // page size, page-table row length (max pages of a sequence), pool pages
  std::vector<int64_t> pg0, npg;      // per sequence: first pool page and page count (its pages are contiguous)
  std::vector<void*> kpool, vpool;    // per layer
  int64_t* pt = nullptr;              // device [B][mp]
  std::vector<int64_t> len;           // host lengths per sequence
  // workspace
  DevBuf n, q, k, v, qn, kn, att, gate, up, h, pos, starts, attn, guard, status, x, logits, ids, lastx, amx, stepc;
  DevBuf gtab, gmax;                  // device table of the 2 * nl RMSNorm gains (n1g, n2g per layer), their max |g|
  DevBuf kvrun;                       // kv8: running max|K|, max|V| per (layer, sequence, kv head): [nl][2][B*Hkv]
  DevBuf kvrow;                       // kv8: appended rows' maxima [2][rows*Hkv]
  DevBuf gpart;                       // many-row head stage: per-(row, head) RoPE envelope maxima [rows][H+Hkv][2]
  Q1Ws q1w;                           // this net's Q1 workspace (graph-stable addresses)
  // captured greedy decode step (imie_net_decode_dev): valid for the pointer key it was captured with
  hipGraphExec_t gexec = nullptr;
  const void* gkey[5] = {nullptr, nullptr, nullptr, nullptr, nullptr};
  uint64_t ggen = 0;                  // allocation generation (imie_alloc_gen) the graph was captured under
  bool live = false;
};

std::vector<Net*>& nets() {
  static std::vector<Net*> v;
  return v;
}

Net* net_get(int64_t h) {
  if (h < 0 || h >= (int64_t)nets().size()) return nullptr;
  Net* n = nets()[(size_t)h];
  return (n && n->live) ? n : nullptr;
}

void net_free_kv(Net& n) {
  for (auto p : n.kpool) if (p) imie_free(p);
  for (auto p : n.vpool) if (p) imie_free(p);
  n.kpool.clear();
  n.vpool.clear();
  if (n.pt) imie_free(n.pt);
  n.pt = nullptr;
}

void net_free(Net* n) {
  if (!n) return;
  (void)hipStreamSynchronize(imie_stream());
  net_free_kv(*n);
  if (n->gexec) { (void)hipGraphExecDestroy(n->gexec); n->gexec = nullptr; }
  DevBuf* bs[] = {&n->n, &n->q, &n->k, &n->v, &n->qn, &n->kn, &n->att, &n->gate, &n->up, &n->h, &n->pos,
                  &n->starts, &n->attn, &n->guard, &n->status, &n->x, &n->logits, &n->ids, &n->lastx, &n->amx,
                  &n->stepc, &n->q1w.xq, &n->q1w.totals, &n->q1w.lslab, &n->q1w.wide, &n->kvrun, &n->kvrow, &n->gpart,
                  &n->gtab, &n->gmax};
  for (auto b : bs) b->release();
  n->live = false;
}

// Allocate the paged cache: sequence b gets ceil(caps[b] / P) pages, contiguous in the pool; its page-table row
// (mp = the largest page count) lists them and repeats its first page past its own count (never addressed).
int net_alloc_kv(Net& n, const std::vector<int64_t>& caps, int64_t P, int kv32) {
  // kv8 MFMA steps take 64 slots of one page; its K pieces are 16 dims wide
  if (P <= 0 || (kv32 && (P % 64 != 0 || n.hd % 16 != 0))) return IMIE_EARG;
  n.kv32 = kv32;
  n.P = P;
  n.pg0.assign((size_t)n.B, 0);
  n.npg.assign((size_t)n.B, 0);
  int64_t tot = 0, mp = 1;
  for (int64_t b = 0; b < n.B; ++b) {
    if (caps[(size_t)b] <= 0) return IMIE_EARG;
    const int64_t np = (caps[(size_t)b] + P - 1) / P;
    n.pg0[(size_t)b] = tot;
    n.npg[(size_t)b] = np;
    tot += np;
    mp = np > mp ? np : mp;
  }
  n.mp = mp;
  n.npages = tot;
  const size_t esz = kv32 ? 4 : 8;
  const size_t bytes = (size_t)(n.npages * n.Hkv * P * n.hd) * esz;
  n.kpool.assign((size_t)n.nl, nullptr);
  n.vpool.assign((size_t)n.nl, nullptr);
  for (int64_t l = 0; l < n.nl; ++l) {
    if (hipMalloc(&n.kpool[(size_t)l], bytes) != hipSuccess) return IMIE_EARG;
    if (hipMalloc(&n.vpool[(size_t)l], bytes) != hipSuccess) return IMIE_EARG;
  }
  std::vector<int64_t> pt((size_t)(n.B * mp));
  for (int64_t b = 0; b < n.B; ++b)
    for (int64_t i = 0; i < mp; ++i)
      pt[(size_t)(b * mp + i)] = n.pg0[(size_t)b] + (i < n.npg[(size_t)b] ? i : 0);
  IMIE_HIP(hipMalloc((void**)&n.pt, pt.size() * 8));
  IMIE_HIP(hipMemcpy(n.pt, pt.data(), pt.size() * 8, hipMemcpyHostToDevice));
  n.len.assign((size_t)n.B, 0);
  if (kv32) {
    const size_t rb = (size_t)(n.nl * 2 * n.B * n.Hkv) * 8;
    if (n.kvrun.ensure(rb)) return IMIE_EARG;
    IMIE_HIP(hipMemset(n.kvrun.p, 0, rb));
  }
  return IMIE_OK;
}

int64_t seq_cap(const Net& n, int64_t b) { return n.npg[(size_t)b] * n.P; }
// Positions sequence b can hold: its pages, and no further than the RoPE tables reach (page rounding can give a
// sequence more slots than the tables have rows; a position past them would read beyond the uploaded table).
int64_t pos_cap(const Net& n, int64_t b) { return std::min(seq_cap(n, b), n.rope_rows); }

uint64_t* run_k(Net& n, int64_t l) { return (uint64_t*)n.kvrun.p + (l * 2) * n.B * n.Hkv; }
uint64_t* run_v(Net& n, int64_t l) { return (uint64_t*)n.kvrun.p + (l * 2 + 1) * n.B * n.Hkv; }

// Workspace for rows = B * M new rows attending over at most lmax keys.
int net_ensure(Net& n, int64_t M, int64_t lmax) {
  const int64_t rows = n.B * M;
  const int64_t qd = n.H * n.hd, kd = n.Hkv * n.hd;
  if (n.n.ensure((size_t)(rows * n.d) * 8) || n.q.ensure((size_t)(rows * qd) * 8) ||
      n.k.ensure((size_t)(rows * kd) * 8) || n.v.ensure((size_t)(rows * kd) * 8) ||
      n.qn.ensure((size_t)(rows * qd) * 8) || n.kn.ensure((size_t)(rows * kd) * 8) ||
      n.att.ensure((size_t)(rows * qd) * 8) || n.gate.ensure((size_t)(rows * n.dff) * 8) ||
      n.up.ensure((size_t)(rows * n.dff) * 8) || n.h.ensure((size_t)(rows * n.dff) * 8) ||
      n.pos.ensure((size_t)rows * 8) || n.starts.ensure((size_t)n.B * 8) || n.guard.ensure((size_t)n.nl * 32) ||
      n.status.ensure(64) || n.attn.ensure(imie_attn_scratch_bytes(n.B, n.H, n.Hkv, M, n.hd, lmax)) ||
      n.kvrow.ensure((size_t)(2 * rows * n.Hkv) * 8) ||
      (rows > 1 && n.gpart.ensure((size_t)(rows * (n.H + n.Hkv) * 2) * 8)))
    return IMIE_EARG;
  return IMIE_OK;
}

// RMSNorm of `rows` rows of x (gain g) into xn, then the matvec(s) `hs` of xn into outs. When d is a multiple of
// 128 up to 4096, the norm kernel also writes the matvec's digit table and clears its outputs (one kernel fewer).
int norm_into_matvec(Net& n, const int64_t* x, int64_t rows, const int64_t* g, int64_t* xn, const int64_t* hs,
                     int cnt, int64_t* const* outs, hipStream_t st) {
  int* status = (int*)n.status.p;
  if (n.d % 128 == 0 && n.d <= 4096 && rows < imie_q1::kGemmMinT) {
    imie_q1::Q1PrepOut po;
    int rc = imie_q1_prep_target(&n.q1w, n.d / 128, rows, &po);
    if (rc) return rc;
    imie_q1::Q1Zero z = {};
    z.cnt = cnt;
    for (int i = 0; i < cnt; ++i) {
      int64_t N = 0, nb = 0;
      if (imie_q1_dims(hs[i], &N, &nb)) return IMIE_EARG;
      z.p[i] = outs[i];
      z.n[i] = rows * N;
    }
    if ((rc = imie_rmsnorm_prep_launch(x, rows, n.d, n.frac, n.eps, g, xn, status, po, z, st))) return rc;
    return imie_q1_launch_multi(hs, cnt, xn, rows, n.frac, outs, 0, &n.q1w, st, 1);
  }
  if (n.d % 128 == 0 && n.d <= 4096) {                // GEMM: the norm writes the projections' digit table
    imie_q1::GemmPrepOut gp;
    int rc = imie_q1_gemm_target(&n.q1w, n.d / 128, rows, &gp);
    if (rc) return rc;
    imie_q1::Q1Zero z = {};
    for (int i = 0; i < cnt && imie_q1_gemm_splits(hs[i], rows); ++i) {   // K-split GEMMs add into cleared outputs
      int64_t N = 0, nb = 0;
      if (imie_q1_dims(hs[i], &N, &nb)) return IMIE_EARG;
      z.p[i] = outs[i];
      z.n[i] = rows * N;
      z.cnt = i + 1;
    }
    if (z.cnt != cnt) z.cnt = 0;                      // all or none: the GEMM is told the outputs are clear
    // the GEMM reads only the digit table: the normalised rows themselves are not written
    if ((rc = imie_rmsnorm_gemm_prep_launch(x, rows, n.d, n.frac, n.eps, g, nullptr, status, gp, z, st))) return rc;
    return imie_q1_launch_multi(hs, cnt, nullptr, rows, n.frac, outs, 0, &n.q1w, st, z.cnt ? 3 : 2);
  }
  int rc = imie_rmsnorm_launch(x, rows, n.d, n.frac, n.eps, g, xn, status, st);
  if (rc) return rc;
  return imie_q1_launch_multi(hs, cnt, xn, rows, n.frac, outs, 0, &n.q1w, st);
}

// Whether every projection of every layer takes the prologue matvec (int32 scales, RMSNorm rows <= 4096), and
// the device gain table is in place. IMIE_NO_PRO=1 keeps the separate producer kernels (comparison runs).
bool pro_path_ok(Net& n) {
  static const bool off = [] { const char* e = getenv("IMIE_NO_PRO"); return e && atoi(e) != 0; }();
  if (off || !n.gtab.p || !n.gmax.p) return false;
  const int64_t qd = n.H * n.hd;
  for (const LayerW& L : n.layers) {
    if (!imie_q1_pro_ok(L.w, 3, imie_q1::kProNorm, n.d) || !imie_q1_pro_ok(&L.w[3], 1, imie_q1::kProCopy, qd) ||
        !imie_q1_pro_ok(&L.w[4], 2, imie_q1::kProNorm, n.d) || !imie_q1_pro_ok(&L.w[6], 1, imie_q1::kProSiluMul, n.dff))
      return false;
  }
  return true;
}

// All layers over M new tokens per sequence; positions come from the device buffers n.pos (B*M) and n.starts
// (B), so the launch sequence is independent of the positions (graph-capturable). lmax bounds the keys any row
// sees and fixes the attention geometry. x: device (B*M, d), updated in place.
int net_run_core(Net& n, int64_t* x, int64_t M, int64_t lmax, hipStream_t st) {
  const int64_t rows = n.B * M;
  const int64_t qd = n.H * n.hd, kd = n.Hkv * n.hd;
  int rc = 0;
#define CK(call) do { rc = (call); if (rc) return rc; } while (0)
  int64_t *xn = (int64_t*)n.n.p, *q = (int64_t*)n.q.p, *k = (int64_t*)n.k.p, *v = (int64_t*)n.v.p;
  int64_t *qn = (int64_t*)n.qn.p, *kn = (int64_t*)n.kn.p, *att = (int64_t*)n.att.p;
  int64_t *gate = (int64_t*)n.gate.p, *up = (int64_t*)n.up.p, *hh = (int64_t*)n.h.p;
  const int64_t* posd = (const int64_t*)n.pos.p;
  uint64_t* guard = (uint64_t*)n.guard.p;
  int* status = (int*)n.status.p;
  // one token: the matvecs build their digit tables in their own prologue (RMSNorm, copy, SiLU * up) instead of
  // after a separate producer kernel; K-split outputs are cleared by the kernel before (q, k, v by the start
  // kernel and by each layer's gate / up matvec, gate / up by the q, k, v matvec)
  const bool pro = rows == 1 && pro_path_ok(n);
  int64_t log2e = 0, dclip = 0;
  imie_silu_consts(n.frac, &log2e, &dclip);
  imie_q1::Q1Zero zq = {}, zg = {};
  zq.cnt = 3; zq.p[0] = q; zq.p[1] = k; zq.p[2] = v; zq.n[0] = rows * qd; zq.n[1] = rows * kd; zq.n[2] = rows * kd;
  zg.cnt = 2; zg.p[0] = gate; zg.p[1] = up; zg.n[0] = rows * n.dff; zg.n[1] = rows * n.dff;
  if (pro) {
    hipLaunchKernelGGL(pro_start_kernel, dim3((unsigned)(2 * n.nl)), dim3(256), 0, st,
                       (const int64_t* const*)n.gtab.p, (int)(2 * n.nl), n.d, (uint64_t*)n.gmax.p, (int64_t*)guard,
                       4 * n.nl, zq);
    IMIE_HIP(hipGetLastError());
  } else {
    CK(fill_i64((int64_t*)guard, 4 * n.nl, 0, st));   // per-layer RoPE envelope maxima
  }
  auto pro_in = [&](const int64_t* a, const int64_t* b, const int64_t* g, int64_t cols, int gi,
                    const imie_q1::Q1Zero& z) {
    imie_q1::Q1Pro p = {};
    p.x = a; p.x2 = b; p.gain = g; p.cols = cols; p.frac = (int)n.frac; p.eps = n.eps; p.status = status;
    p.gmax = gi >= 0 ? (const uint64_t*)n.gmax.p + gi : nullptr;
    p.log2e = log2e; p.dclip = dclip;
    p.zero = z;
    return p;
  };
  for (int64_t l = 0; l < n.nl; ++l) {
    const LayerW& L = n.layers[(size_t)l];
    if (pro) {
      int64_t* outs[3] = {q, k, v};
      const imie_q1::Q1Pro p = pro_in(x, nullptr, L.n1g, n.d, (int)(2 * l), zg);
      CK(imie_q1_launch_pro(L.w, 3, p, imie_q1::kProNorm, n.frac, outs, 0, st));
    } else {
      int64_t* outs[3] = {q, k, v};
      CK(norm_into_matvec(n, x, rows, L.n1g, xn, L.w, 3, outs, st));
    }
    AttnDesc d = {};
    d.B = n.B; d.H = n.H; d.Hkv = n.Hkv; d.hd = n.hd; d.M = M;
    d.qsb = M * qd; d.qsh = n.hd; d.qsm = qd;
    d.q = qn; d.K = n.kpool[(size_t)l]; d.V = n.vpool[(size_t)l]; d.kv32 = n.kv32;
    d.pt = n.pt; d.P = n.P; d.mp = n.mp;
    d.starts = (const int64_t*)n.starts.p; d.lengths = nullptr;
    d.Lmax = lmax; d.frac = (int)n.frac; d.inv_sqrt = n.inv_sqrt;
    d.out = att; d.status = status; d.rope_guard = guard + 4 * l;
    if (n.kv32) { d.run_k = run_k(n, l); d.run_v = run_v(n, l); }
    imie_attn_bind_scratch(d, n.attn.p);
    if (n.kv32 && M == 1) imie_attn_qdigit_scratch(d, (int8_t**)&d.qd, (int**)&d.qlimbs);
    {
      QkHeadArgs a = {};
      a.q = q; a.k = k; a.v = v; a.qo = qn;
      a.qng = L.qng; a.kng = L.kng; a.pos = posd; a.cos = n.cos; a.sin = n.sin;
      a.rows = rows; a.H = n.H; a.Hkv = n.Hkv; a.hd = n.hd; a.M = M; a.eps = n.eps; a.frac = (int)n.frac;
      a.pt = n.pt; a.P = n.P; a.mp = n.mp; a.kpool = n.kpool[(size_t)l]; a.vpool = n.vpool[(size_t)l];
      a.guard = guard + 4 * l; a.status = status;
      if (n.kv32) {
        a.rowk = (uint64_t*)n.kvrow.p; a.rowv = (uint64_t*)n.kvrow.p + rows * n.Hkv;
        a.run_k = run_k(n, l); a.run_v = run_v(n, l);
      }
      if (d.qd) { a.qd = (int8_t*)d.qd; a.qlimbs = (int*)d.qlimbs; a.qmax = d.maxq; }
      if (rows > 1) a.gpart = (uint64_t*)n.gpart.p;   // several rows: no same-address atomics on the guard
      CK(imie_qk_head_launch(a, n.kv32, st));
      CK(imie_qk_head_finish_launch(a, n.kv32, st));
    }
    CK(imie_attention_launch(d, st));
    if (pro) {
      const imie_q1::Q1Zero none = {};
      const imie_q1::Q1Pro po = pro_in(att, nullptr, nullptr, qd, -1, none);
      CK(imie_q1_launch_pro(&L.w[3], 1, po, imie_q1::kProCopy, n.frac, &x, 1, st));
      int64_t* outs[2] = {gate, up};
      const imie_q1::Q1Pro pn = pro_in(x, nullptr, L.n2g, n.d, (int)(2 * l + 1), zq);
      CK(imie_q1_launch_pro(&L.w[4], 2, pn, imie_q1::kProNorm, n.frac, outs, 0, st));
      const imie_q1::Q1Pro ps = pro_in(gate, up, nullptr, n.dff, -1, none);
      CK(imie_q1_launch_pro(&L.w[6], 1, ps, imie_q1::kProSiluMul, n.frac, &x, 1, st));
      continue;
    }
    CK(imie_q1_launch_multi(&L.w[3], 1, att, rows, n.frac, &x, 1, &n.q1w, st));
    {
      int64_t* outs[2] = {gate, up};
      CK(norm_into_matvec(n, x, rows, L.n2g, xn, &L.w[4], 2, outs, st));
    }
    if (n.dff % 128 == 0 && rows < imie_q1::kGemmMinT) {
      imie_q1::Q1PrepOut po;
      CK(imie_q1_prep_target(&n.q1w, n.dff / 128, rows, &po));
      CK(imie_silu_mul_prep_launch(gate, up, rows, n.dff, n.frac, hh, po, st));
      CK(imie_q1_launch_multi(&L.w[6], 1, hh, rows, n.frac, &x, 1, &n.q1w, st, 1));
    } else if (n.dff % 128 == 0) {                 // GEMM: SiLU * up writes the down projection's digit table
      imie_q1::GemmPrepOut gp;
      CK(imie_q1_gemm_target(&n.q1w, n.dff / 128, rows, &gp));
      CK(imie_silu_mul_gemm_prep_launch(gate, up, rows, n.dff, n.frac, gp, st));
      CK(imie_q1_launch_multi(&L.w[6], 1, nullptr, rows, n.frac, &x, 1, &n.q1w, st, 2));
    } else {
      CK(imie_silu_mul_launch(gate, up, rows * n.dff, n.frac, hh, st));
      CK(imie_q1_launch_multi(&L.w[6], 1, hh, rows, n.frac, &x, 1, &n.q1w, st));
    }
  }
#undef CK
  return IMIE_OK;
}

// Run all layers over M new tokens for each of the B sequences. x: device (B*M, d), updated in place.
// starts: host (B), the first new position per sequence (== its current cache length).
int net_run(Net& n, int64_t* x, const int64_t* starts, int64_t M, hipStream_t st) {
  const int64_t rows = n.B * M;
  int64_t lmax = 0;
  for (int64_t b = 0; b < n.B; ++b) {
    if (starts[b] < 0 || starts[b] + M > pos_cap(n, b)) return IMIE_EARG;
    lmax = starts[b] + M > lmax ? starts[b] + M : lmax;
  }
  if (net_ensure(n, M, lmax)) return IMIE_EARG;
  std::vector<int64_t> pos((size_t)rows);
  for (int64_t r = 0; r < rows; ++r) pos[(size_t)r] = starts[r / M] + r % M;
  IMIE_HIP(hipMemcpyAsync(n.pos.p, pos.data(), (size_t)rows * 8, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemcpyAsync(n.starts.p, starts, (size_t)n.B * 8, hipMemcpyHostToDevice, st));
  const int rc = net_run_core(n, x, M, lmax, st);
  if (rc) return rc;
  for (int64_t b = 0; b < n.B; ++b) n.len[(size_t)b] = starts[b] + M;
  return IMIE_OK;
}

// After a greedy step: hist[step * B + b] = ids[b]; every sequence advances one position (starts, pos); step++.
__global__ void decode_advance_kernel(const int64_t* __restrict__ ids, int64_t* __restrict__ hist,
                                      int64_t* __restrict__ stepc, int64_t* __restrict__ starts,
                                      int64_t* __restrict__ pos, int64_t B) {
  const int64_t s = *stepc;
  for (int64_t b = threadIdx.x; b < B; b += blockDim.x) {
    if (hist) hist[s * B + b] = ids[b];
    const int64_t p = starts[b] + 1;
    starts[b] = p;
    pos[b] = p;
  }
  __syncthreads();
  if (threadIdx.x == 0) *stepc = s + 1;
}

// After a sampled step: the token joins its sequence's history row (hist[b * hld + len]), len++ (the next draw
// key), and every sequence advances one position.
__global__ void decode_advance_sampled_kernel(const int64_t* __restrict__ ids, int64_t* __restrict__ hist, int64_t hld,
                                              int64_t* __restrict__ hlen, int64_t* __restrict__ starts,
                                              int64_t* __restrict__ pos, int64_t B) {
  for (int64_t b = threadIdx.x; b < B; b += blockDim.x) {
    const int64_t L = hlen[b];
    if (L >= 0 && L < hld) hist[b * hld + L] = ids[b];
    hlen[b] = L + 1;
    const int64_t p = starts[b] + 1;
    starts[b] = p;
    pos[b] = p;
  }
}

// final norm of selected rows + output head (+ argmax). rows_idx: host list of row indices into x.
int net_head(Net& n, const int64_t* x, const std::vector<int64_t>& rows_idx, int64_t* logits, int64_t* ids,
             hipStream_t st) {
  const int64_t R = (int64_t)rows_idx.size();
  if (n.out_head < 0 || R == 0) return IMIE_EARG;
  if (n.lastx.ensure((size_t)(R * n.d) * 8) || n.n.ensure((size_t)(R * n.d) * 8)) return IMIE_EARG;
  bool ident = true;
  for (int64_t i = 0; i < R; ++i) ident = ident && rows_idx[(size_t)i] == i;
  const int64_t* src = x;
  if (!ident) {
    for (int64_t i = 0; i < R; ++i)
      IMIE_HIP(hipMemcpyAsync((int64_t*)n.lastx.p + i * n.d, x + rows_idx[(size_t)i] * n.d, (size_t)n.d * 8,
                              hipMemcpyDeviceToDevice, st));
    src = (const int64_t*)n.lastx.p;
  }
  int rc = norm_into_matvec(n, src, R, n.finalg, (int64_t*)n.n.p, &n.out_head, 1, &logits, st);
  if (rc) return rc;
  if (ids) {
    if (n.amx.ensure(imie_argmax_scratch_bytes(R))) return IMIE_EARG;
    rc = imie_argmax_launch(logits, R, n.vocab, ids, (int64_t*)n.amx.p, st);
  }
  return rc;
}

int read_status(Net& n, hipStream_t st, int* stat) {
  IMIE_HIP(hipMemcpyAsync(stat, n.status.p, 4, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipStreamSynchronize(st));
  return IMIE_OK;
}

int64_t net_create(int64_t B, int64_t n_layers, int64_t H, int64_t Hkv, int64_t hd, int64_t d, int64_t dff,
                   int64_t cap, int64_t vocab, int64_t frac, int64_t eps, int64_t inv_sqrt, const int64_t* wq,
                   const int64_t* wk, const int64_t* wv, const int64_t* wo, const int64_t* w1, const int64_t* wu,
                   const int64_t* w2, const int64_t* n1g, const int64_t* n2g, const int64_t* qng, const int64_t* kng,
                   int64_t finalg, int64_t out_head, int64_t cos_h, int64_t sin_h, int64_t page, int kv32) {
  if (B <= 0 || n_layers <= 0 || H <= 0 || Hkv <= 0 || H % Hkv || hd <= 0 || hd > 128 || (hd & 1) || d <= 0 ||
      dff <= 0 || cap <= 0 || frac < 1 || frac > 29 || eps < 0 || imie_device_ready() != 0)
    return -1;
  Net* n = new Net();
  n->B = B; n->d = d; n->H = H; n->Hkv = Hkv; n->hd = hd; n->dff = dff; n->nl = n_layers; n->vocab = vocab;
  n->frac = frac; n->eps = eps; n->inv_sqrt = inv_sqrt;
  const int64_t* arrs[] = {wq, wk, wv, wo, w1, wu, w2};
  for (int64_t l = 0; l < n_layers; ++l) {
    LayerW L;
    for (int i = 0; i < 7; ++i) L.w[i] = arrs[i][l];
    // shape checks: q (H*hd, d), k/v (Hkv*hd, d), o (d, H*hd), w1/wu (dff, d), w2 (d, dff)
    const int64_t want[7][2] = {{H * hd, d}, {Hkv * hd, d}, {Hkv * hd, d}, {d, H * hd}, {dff, d}, {dff, d}, {d, dff}};
    for (int i = 0; i < 7; ++i) {
      int64_t N = 0, nb = 0;
      if (imie_q1_dims(L.w[i], &N, &nb) || N != want[i][0] || nb * 128 != want[i][1]) { delete n; return -1; }
    }
    L.n1g = buf_get(n1g[l], d); L.n2g = buf_get(n2g[l], d); L.qng = buf_get(qng[l], hd); L.kng = buf_get(kng[l], hd);
    if (!L.n1g || !L.n2g || !L.qng || !L.kng) { delete n; return -1; }
    n->layers.push_back(L);
  }
  n->finalg = finalg >= 0 ? buf_get(finalg, d) : nullptr;
  n->out_head = out_head;
  if (out_head >= 0) {
    int64_t N = 0, nb = 0;
    if (imie_q1_dims(out_head, &N, &nb) || nb * 128 != d || (vocab > 0 && N != vocab) || !n->finalg) { delete n; return -1; }
    n->vocab = N;
  }
  n->cos = buf_get(cos_h, cap * (hd / 2));
  n->sin = buf_get(sin_h, cap * (hd / 2));
  if (!n->cos || !n->sin) { delete n; return -1; }
  n->rope_rows = std::min(bufs()[(size_t)cos_h].n, bufs()[(size_t)sin_h].n) / (hd / 2);
  {
    std::vector<const int64_t*> gt;
    for (const LayerW& L : n->layers) { gt.push_back(L.n1g); gt.push_back(L.n2g); }
    if (n->gtab.ensure(gt.size() * sizeof(void*)) || n->gmax.ensure(gt.size() * 8) ||
        hipMemcpy(n->gtab.p, gt.data(), gt.size() * sizeof(void*), hipMemcpyHostToDevice) != hipSuccess) {
      n->gtab.release(); n->gmax.release(); delete n; return -1;
    }
  }
  n->live = true;
  if (net_alloc_kv(*n, std::vector<int64_t>((size_t)B, cap), page, kv32)) { net_free(n); delete n; return -1; }
  nets().push_back(n);
  return (int64_t)nets().size() - 1;
}

}  // namespace

extern "C" {

// gpu_native.py:549-556 / bonsai_q1_gpu.cu `bonsai_buf_upload_i64`: upload an int64 array once -> handle.
int64_t bonsai_buf_upload_i64(const int64_t* host, int64_t n) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!host || n <= 0 || imie_device_ready() != 0) return -1;
  BufEntry e;
  if (hipMalloc((void**)&e.p, (size_t)n * 8) != hipSuccess) return -1;
  if (hipMemcpy(e.p, host, (size_t)n * 8, hipMemcpyHostToDevice) != hipSuccess) { imie_free(e.p); return -1; }
  e.n = n;
  bufs().push_back(e);
  return (int64_t)bufs().size() - 1;
}

// Device address of an uploaded buffer (device-pointer pipelines).
const int64_t* imie_buf_device_ptr(int64_t handle) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  return buf_get(handle, 0);
}

void imie_buf_free_all(void) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  (void)hipStreamSynchronize(imie_stream());
  for (auto& e : bufs()) if (e.p) imie_free(e.p);
  bufs().clear();
}

// gpu_native.py:559-595 / bonsai_q1_gpu.cu:3694-3819 `bonsai_prefill_forward_gpu`: whole prefill on the device,
// last-row logits (vocab,) out; optional KV export (n_layers, Hkv, T, hd) int64 (post-RoPE K, raw V).
int bonsai_prefill_forward_gpu(const int64_t* x_embed, int64_t T, int64_t d, int64_t n_layers, int64_t H, int64_t Hkv,
                               int64_t hd, int64_t dff, int64_t frac, int64_t eps, int64_t inv_sqrt,
                               const int64_t* wq, const int64_t* wk, const int64_t* wv, const int64_t* wo,
                               const int64_t* w1, const int64_t* wu, const int64_t* w2, const int64_t* n1g,
                               const int64_t* n2g, const int64_t* qng, const int64_t* kng, int64_t finalg,
                               int64_t out_head, int64_t cos_h, int64_t sin_h, int64_t* out_logits, int64_t* out_k,
                               int64_t* out_v) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!x_embed || !out_logits || T <= 0 || !wq || !wk || !wv || !wo || !w1 || !wu || !w2 || !n1g || !n2g || !qng ||
      !kng)
    return IMIE_EARG;
  const int64_t h = net_create(1, n_layers, H, Hkv, hd, d, dff, T, 0, frac, eps, inv_sqrt, wq, wk, wv, wo, w1, wu,
                               w2, n1g, n2g, qng, kng, finalg, out_head, cos_h, sin_h, T, 0);
  if (h < 0) return IMIE_EARG;
  Net& n = *nets()[(size_t)h];
  hipStream_t st = imie_stream();
  int rc = IMIE_OK;
  do {
    if (n.x.ensure((size_t)(T * d) * 8) || n.logits.ensure((size_t)n.vocab * 8)) { rc = IMIE_EARG; break; }
    if (hipMemcpyAsync(n.x.p, x_embed, (size_t)(T * d) * 8, hipMemcpyHostToDevice, st) != hipSuccess) { rc = IMIE_EARG; break; }
    if (n.status.ensure(64) || fill_i64((int64_t*)n.status.p, 1, 0, st)) { rc = IMIE_EARG; break; }
    const int64_t start = 0;
    if ((rc = net_run(n, (int64_t*)n.x.p, &start, T, st))) break;
    if ((rc = net_head(n, (const int64_t*)n.x.p, {T - 1}, (int64_t*)n.logits.p, nullptr, st))) break;
    int stat = 0;
    if ((rc = read_status(n, st, &stat))) break;
    if (stat) { rc = stat & IMIE_ERMS ? IMIE_ERMS : IMIE_EOVF; break; }
    if (hipMemcpy(out_logits, n.logits.p, (size_t)n.vocab * 8, hipMemcpyDeviceToHost) != hipSuccess) { rc = IMIE_EARG; break; }
    if (out_k && out_v) {
      // dense int64 cache with P = T: layer pool is exactly (Hkv, T, hd)
      const size_t lb = (size_t)(Hkv * T * hd) * 8;
      for (int64_t l = 0; l < n_layers; ++l) {
        if (hipMemcpy((char*)out_k + l * lb, n.kpool[(size_t)l], lb, hipMemcpyDeviceToHost) != hipSuccess ||
            hipMemcpy((char*)out_v + l * lb, n.vpool[(size_t)l], lb, hipMemcpyDeviceToHost) != hipSuccess) {
          rc = IMIE_EARG;
          break;
        }
      }
    }
  } while (0);
  net_free(&n);
  delete nets()[(size_t)h];
  nets()[(size_t)h] = nullptr;
  return rc;
}

// gpu_native.py:483-506 / bonsai_q1_gpu.cu:3517-3562 `bonsai_decode_ctx_create`: B sequences, int64 cache of
// capacity cap per sequence. Returns a context handle >= 0 or -1.
int64_t bonsai_decode_ctx_create(int64_t B, int64_t n_layers, int64_t H, int64_t Hkv, int64_t hd, int64_t d,
                                 int64_t dff, int64_t cap, int64_t vocab, int64_t frac, int64_t eps, int64_t inv_sqrt,
                                 const int64_t* wq, const int64_t* wk, const int64_t* wv, const int64_t* wo,
                                 const int64_t* w1, const int64_t* wu, const int64_t* w2, const int64_t* n1g,
                                 const int64_t* n2g, const int64_t* qng, const int64_t* kng, int64_t finalg,
                                 int64_t out_head, int64_t cos_h, int64_t sin_h) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!wq || !wk || !wv || !wo || !w1 || !wu || !w2 || !n1g || !n2g || !qng || !kng) return -1;
  return net_create(B, n_layers, H, Hkv, hd, d, dff, cap, vocab, frac, eps, inv_sqrt, wq, wk, wv, wo, w1, wu, w2, n1g,
                    n2g, qng, kng, finalg, out_head, cos_h, sin_h, cap, 0);
}

// Extended context (no reference counterpart): int32 (kv32 = 1, guarded) or int64 paged cache with `page`
// tokens per page; out_head < 0 builds a layers-only context.
int64_t imie_net_create(int64_t B, int64_t n_layers, int64_t H, int64_t Hkv, int64_t hd, int64_t d, int64_t dff,
                        int64_t cap, int64_t frac, int64_t eps, int64_t inv_sqrt, const int64_t* wq, const int64_t* wk,
                        const int64_t* wv, const int64_t* wo, const int64_t* w1, const int64_t* wu, const int64_t* w2,
                        const int64_t* n1g, const int64_t* n2g, const int64_t* qng, const int64_t* kng,
                        int64_t finalg, int64_t out_head, int64_t cos_h, int64_t sin_h, int64_t page, int kv32) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!wq || !wk || !wv || !wo || !w1 || !wu || !w2 || !n1g || !n2g || !qng || !kng || page <= 0) return -1;
  return net_create(B, n_layers, H, Hkv, hd, d, dff, cap, 0, frac, eps, inv_sqrt, wq, wk, wv, wo, w1, wu, w2, n1g,
                    n2g, qng, kng, finalg, out_head, cos_h, sin_h, page, kv32);
}

// gpu_native.py:509-521 / bonsai_q1_gpu.cu:3565-3584 `bonsai_decode_ctx_seed_seq`: k/v (n_layers, Hkv, Lb, hd).
int bonsai_decode_ctx_seed_seq(int64_t ctx, int64_t b, const int64_t* k, const int64_t* v, int64_t Lb) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  Net* n = net_get(ctx);
  if (!n || !k || !v || b < 0 || b >= n->B || Lb < 0 || Lb > pos_cap(*n, b)) return IMIE_EARG;
  const size_t esz = n->kv32 ? 4 : 8;
  std::vector<char> kb((size_t)(n->npg[(size_t)b] * n->Hkv * n->P * n->hd) * esz), vb(kb.size());
  std::vector<uint64_t> mk((size_t)(n->nl * n->Hkv), 0), mv(mk.size(), 0);
  for (int64_t l = 0; l < n->nl && n->kv32; ++l)   // transactional: check every value before writing any
    for (int64_t kv = 0; kv < n->Hkv; ++kv)
      for (int64_t j = 0; j < Lb; ++j)
        for (int64_t c = 0; c < n->hd; ++c) {
          const int64_t src = ((l * n->Hkv + kv) * Lb + j) * n->hd + c;
          if (!imie_kv8::fits(k[src]) || !imie_kv8::fits(v[src])) return IMIE_EOVF;
          const uint64_t ak = k[src] < 0 ? (uint64_t)0 - (uint64_t)k[src] : (uint64_t)k[src];
          const uint64_t av = v[src] < 0 ? (uint64_t)0 - (uint64_t)v[src] : (uint64_t)v[src];
          uint64_t& a1 = mk[(size_t)(l * n->Hkv + kv)];
          uint64_t& a2 = mv[(size_t)(l * n->Hkv + kv)];
          a1 = ak > a1 ? ak : a1;
          a2 = av > a2 ? av : a2;
        }
  for (int64_t l = 0; l < n->nl; ++l) {
    memset(kb.data(), 0, kb.size());
    memset(vb.data(), 0, vb.size());
    for (int64_t kv = 0; kv < n->Hkv; ++kv)
      for (int64_t j = 0; j < Lb; ++j)
        for (int64_t c = 0; c < n->hd; ++c) {
          const int64_t src = ((l * n->Hkv + kv) * Lb + j) * n->hd + c;
          const int64_t pgl = j / n->P, slot = j % n->P;     // page within sequence b (identity page table)
          if (n->kv32) {
            const int64_t base = imie_kv8::block_base(pgl, kv, n->Hkv, n->hd, n->P);
            const uint32_t wk = imie_kv8::encode(k[src]), wv = imie_kv8::encode(v[src]);
            for (int db = 0; db < 4; ++db) {
              kb[(size_t)(base + imie_kv8::k_off(slot, db, c, n->hd))] = (char)(wk >> (8 * db));
              vb[(size_t)(base + imie_kv8::v_off(slot, db, c, n->hd, n->P))] = (char)(wv >> (8 * db));
            }
          } else {
            const int64_t dst = pgl * (n->Hkv * n->P * n->hd) + kv * n->P * n->hd + slot * n->hd + c;
            ((int64_t*)kb.data())[dst] = k[src];
            ((int64_t*)vb.data())[dst] = v[src];
          }
        }
    const size_t off = (size_t)(n->pg0[(size_t)b] * n->Hkv * n->P * n->hd) * esz;
    IMIE_HIP(hipMemcpy((char*)n->kpool[(size_t)l] + off, kb.data(), kb.size(), hipMemcpyHostToDevice));
    IMIE_HIP(hipMemcpy((char*)n->vpool[(size_t)l] + off, vb.data(), vb.size(), hipMemcpyHostToDevice));
    if (n->kv32) {
      IMIE_HIP(hipMemcpy(run_k(*n, l) + b * n->Hkv, &mk[(size_t)(l * n->Hkv)], (size_t)n->Hkv * 8,
                         hipMemcpyHostToDevice));
      IMIE_HIP(hipMemcpy(run_v(*n, l) + b * n->Hkv, &mv[(size_t)(l * n->Hkv)], (size_t)n->Hkv * 8,
                         hipMemcpyHostToDevice));
    }
  }
  n->len[(size_t)b] = Lb;
  return IMIE_OK;
}

// gpu_native.py:524-538 / bonsai_q1_gpu.cu:3588-3647 `bonsai_decode_step`: x_in (B, d) new-token residuals, pos (B,)
// absolute positions; out (B, vocab) logits. Host pointers, synchronous.
int bonsai_decode_step(int64_t ctx, const int64_t* x_in, const int64_t* pos, int64_t* out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  Net* n = net_get(ctx);
  if (!n || !x_in || !pos || !out || n->out_head < 0) return IMIE_EARG;
  hipStream_t st = imie_stream();
  const size_t xb = (size_t)(n->B * n->d) * 8;
  if (n->x.ensure(xb) || n->logits.ensure((size_t)(n->B * n->vocab) * 8) || n->status.ensure(64)) return IMIE_EARG;
  IMIE_HIP(hipMemcpyAsync(n->x.p, x_in, xb, hipMemcpyHostToDevice, st));
  int rc = fill_i64((int64_t*)n->status.p, 1, 0, st);
  if (rc) return rc;
  if ((rc = net_run(*n, (int64_t*)n->x.p, pos, 1, st))) return rc;
  std::vector<int64_t> rows((size_t)n->B);
  for (int64_t b = 0; b < n->B; ++b) rows[(size_t)b] = b;
  if ((rc = net_head(*n, (const int64_t*)n->x.p, rows, (int64_t*)n->logits.p, nullptr, st))) return rc;
  int stat = 0;
  if ((rc = read_status(*n, st, &stat))) return rc;
  if (stat) return stat & IMIE_ERMS ? IMIE_ERMS : IMIE_EOVF;
  IMIE_HIP(hipMemcpy(out, n->logits.p, (size_t)(n->B * n->vocab) * 8, hipMemcpyDeviceToHost));
  return IMIE_OK;
}

void bonsai_decode_ctx_free(int64_t ctx) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  Net* n = net_get(ctx);
  if (!n) return;
  net_free(n);
  delete n;
  nets()[(size_t)ctx] = nullptr;
}

// Device-pointer forward (no reference counterpart): x_dev (B*M, d) updated in place through all layers for M new
// tokens per sequence at positions starts[b] .. starts[b] + M - 1 (host array). Asynchronous on `stream`;
// the status word (imie_net_status) reports envelope refusals.
int imie_net_forward_dev(int64_t ctx, int64_t* x_dev, const int64_t* starts, int64_t M, void* stream) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  Net* n = net_get(ctx);
  if (!n || !x_dev || !starts || M <= 0) return IMIE_EARG;
  return net_run(*n, x_dev, starts, M, (hipStream_t)stream);
}

// Final norm + output head (+ lowest-index argmax when ids_dev != NULL) for rows [0, rows) of x_dev.
int imie_net_head_dev(int64_t ctx, const int64_t* x_dev, int64_t rows, int64_t* logits_dev, int64_t* ids_dev,
                      void* stream) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  Net* n = net_get(ctx);
  if (!n || !x_dev || !logits_dev || rows <= 0) return IMIE_EARG;
  std::vector<int64_t> r((size_t)rows);
  for (int64_t i = 0; i < rows; ++i) r[(size_t)i] = i;
  return net_head(*n, x_dev, r, logits_dev, ids_dev, (hipStream_t)stream);
}

// Greedy decode on the device (no reference counterpart; the reference's decode loop drives
// bonsai_decode_step from the host, reference_bonsai.py:1200-1310): `steps` times, embed ids_dev (B) from the
// natural-layout Q1 embedding (ebits, escale), run every layer at the sequences' current lengths, final norm +
// LM head into logits_dev (B, vocab), lowest-index argmax back into ids_dev, and hist_dev[step * B + b] (when
// non-null) records the token. use_graph != 0 runs the first step eagerly and replays a captured HIP graph of
// one step for the rest (the graph is kept for the same pointer set). Asynchronous on `stream`; envelope
// refusals set the status word (imie_net_status).
int imie_net_decode_dev(int64_t ctx, const uint8_t* ebits, const int64_t* escale, int64_t* ids_dev,
                        int64_t* logits_dev, int64_t* hist_dev, int64_t steps, int use_graph, void* stream) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  Net* n = net_get(ctx);
  if (!n || !ebits || !escale || !ids_dev || !logits_dev || steps <= 0 || n->out_head < 0) return IMIE_EARG;
  const int64_t cap = n->mp * n->P;
  for (int64_t b = 0; b < n->B; ++b)
    if (n->len[(size_t)b] + steps > pos_cap(*n, b)) return IMIE_EARG;
  hipStream_t st = (hipStream_t)stream;
  if (net_ensure(*n, 1, cap) || n->amx.ensure(imie_argmax_scratch_bytes(n->B)) || n->stepc.ensure(64) ||
      n->lastx.ensure((size_t)(n->B * n->d) * 8))
    return IMIE_EARG;
  IMIE_HIP(hipMemcpyAsync(n->starts.p, n->len.data(), (size_t)n->B * 8, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemcpyAsync(n->pos.p, n->len.data(), (size_t)n->B * 8, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipStreamSynchronize(st));                 // the host length vector is read by the copies above
  if (fill_i64((int64_t*)n->stepc.p, 1, 0, st)) return IMIE_EARG;
  std::vector<int64_t> rows((size_t)n->B);
  for (int64_t b = 0; b < n->B; ++b) rows[(size_t)b] = b;
  auto step = [&]() -> int {
    int rc = imie_embed_launch(ebits, escale, n->d / 128, ids_dev, n->B, (int64_t*)n->x.p, st);
    if (rc) return rc;
    if ((rc = net_run_core(*n, (int64_t*)n->x.p, 1, cap, st))) return rc;
    if ((rc = net_head(*n, (const int64_t*)n->x.p, rows, logits_dev, ids_dev, st))) return rc;
    hipLaunchKernelGGL(decode_advance_kernel, dim3(1), dim3(256), 0, st, ids_dev, hist_dev, (int64_t*)n->stepc.p,
                       (int64_t*)n->starts.p, (int64_t*)n->pos.p, n->B);
    IMIE_HIP(hipGetLastError());
    return IMIE_OK;
  };
  if (n->x.ensure((size_t)(n->B * n->d) * 8)) return IMIE_EARG;
  int rc = step();                                    // eager: also sizes every workspace the graph will use
  if (rc) return rc;
  if (steps > 1) {
    if (!use_graph) {
      for (int64_t s = 1; s < steps && !rc; ++s) rc = step();
      if (rc) return rc;
    } else {
      const void* key[5] = {ebits, escale, ids_dev, logits_dev, hist_dev};
      // The graph also holds this net's workspaces, pools and the weights' addresses: any device free since
      // the capture (a larger prefill regrowing a workspace, a weight freed) invalidates it.
      if (n->gexec && (memcmp(key, n->gkey, sizeof(key)) != 0 || n->ggen != imie_alloc_gen())) {
        (void)hipGraphExecDestroy(n->gexec);
        n->gexec = nullptr;
      }
      if (!n->gexec) {
        const bool prof = imie_prof_suspend(true);
        hipGraph_t g = nullptr;
        IMIE_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        rc = step();
        const hipError_t ec = hipStreamEndCapture(st, &g);
        imie_prof_suspend(prof);
        if (rc || ec != hipSuccess || !g) { if (g) (void)hipGraphDestroy(g); return rc ? rc : IMIE_EARG; }
        const hipError_t ei = hipGraphInstantiate(&n->gexec, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (ei != hipSuccess) { n->gexec = nullptr; return IMIE_EARG; }
        memcpy(n->gkey, key, sizeof(key));
        n->ggen = imie_alloc_gen();
      }
      for (int64_t s = 1; s < steps; ++s) IMIE_HIP(hipGraphLaunch(n->gexec, st));
    }
  }
  for (int64_t b = 0; b < n->B; ++b) n->len[(size_t)b] += steps;
  return IMIE_OK;
}

// Sampled decode on the device (no reference counterpart for the fused loop; each token equals
// sample_token(logits_row, cfg, len(ids), frac, ids), sampler.py:403-437, as the reference generate loops call it,
// reference_bonsai.py:1110-1146 / :1260-1310): per step embed -> layers -> head -> imie_sample_launch over the B
// logits rows with history rows hist_dev[b * hist_ld + i] (i < hist_len_dev[b]: prompt + generated tokens) and
// draw key hist_len_dev[b]; the token is appended and hist_len_dev[b] advances. One step is captured as a graph.
int imie_net_decode_sampled_dev(int64_t ctx, const uint8_t* ebits, const int64_t* escale, int64_t* ids_dev,
                                int64_t* logits_dev, const ImieSamplerConfig* cfg, int64_t* hist_dev, int64_t hist_ld,
                                int64_t* hist_len_dev, int64_t steps, int use_graph, void* stream) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  Net* n = net_get(ctx);
  if (!n || !ebits || !escale || !ids_dev || !logits_dev || !cfg || !hist_dev || !hist_len_dev || hist_ld <= 0 ||
      steps <= 0 || n->out_head < 0 || cfg->frac != n->frac)
    return IMIE_EARG;
  const int64_t cap = n->mp * n->P;
  for (int64_t b = 0; b < n->B; ++b)
    if (n->len[(size_t)b] + steps > pos_cap(*n, b)) return IMIE_EARG;
  hipStream_t st = (hipStream_t)stream;
  if (net_ensure(*n, 1, cap) || n->stepc.ensure(64) || n->lastx.ensure((size_t)(n->B * n->d) * 8)) return IMIE_EARG;
  std::vector<int64_t> hl((size_t)n->B);
  IMIE_HIP(hipMemcpyAsync(hl.data(), hist_len_dev, (size_t)n->B * 8, hipMemcpyDeviceToHost, st));
  IMIE_HIP(hipMemcpyAsync(n->starts.p, n->len.data(), (size_t)n->B * 8, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipMemcpyAsync(n->pos.p, n->len.data(), (size_t)n->B * 8, hipMemcpyHostToDevice, st));
  IMIE_HIP(hipStreamSynchronize(st));
  for (int64_t b = 0; b < n->B; ++b)                  // every drawn token must fit its history row
    if (hl[(size_t)b] < 0 || hl[(size_t)b] + steps > hist_ld) return IMIE_EARG;
  std::vector<int64_t> rows((size_t)n->B);
  for (int64_t b = 0; b < n->B; ++b) rows[(size_t)b] = b;
  const ImieSamplerConfig c = *cfg;
  auto step = [&]() -> int {
    int rc = imie_embed_launch(ebits, escale, n->d / 128, ids_dev, n->B, (int64_t*)n->x.p, st);
    if (rc) return rc;
    if ((rc = net_run_core(*n, (int64_t*)n->x.p, 1, cap, st))) return rc;
    if ((rc = net_head(*n, (const int64_t*)n->x.p, rows, logits_dev, nullptr, st))) return rc;
    if ((rc = imie_sample_launch(logits_dev, n->B, n->vocab, n->vocab, c, hist_dev, hist_ld, hist_len_dev,
                                 hist_len_dev, ids_dev, (int*)n->status.p, st)))
      return rc;
    hipLaunchKernelGGL(decode_advance_sampled_kernel, dim3(1), dim3(256), 0, st, ids_dev, hist_dev, hist_ld,
                       hist_len_dev, (int64_t*)n->starts.p, (int64_t*)n->pos.p, n->B);
    IMIE_HIP(hipGetLastError());
    return IMIE_OK;
  };
  if (n->x.ensure((size_t)(n->B * n->d) * 8)) return IMIE_EARG;
  int rc = step();                                    // eager: also sizes every workspace the graph will use
  if (rc) return rc;
  if (steps > 1) {
    if (!use_graph) {
      for (int64_t s = 1; s < steps && !rc; ++s) rc = step();
      if (rc) return rc;
    } else {
      const bool prof = imie_prof_suspend(true);
      hipGraph_t g = nullptr;
      hipGraphExec_t ge = nullptr;
      IMIE_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
      rc = step();
      const hipError_t ec = hipStreamEndCapture(st, &g);
      imie_prof_suspend(prof);
      if (rc || ec != hipSuccess || !g) { if (g) (void)hipGraphDestroy(g); return rc ? rc : IMIE_EARG; }
      const hipError_t ei = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
      (void)hipGraphDestroy(g);
      if (ei != hipSuccess) return IMIE_EARG;
      for (int64_t s = 1; s < steps && !rc; ++s)
        if (hipGraphLaunch(ge, st) != hipSuccess) rc = IMIE_EARG;
      (void)hipStreamSynchronize(st);
      (void)hipGraphExecDestroy(ge);
      if (rc) return rc;
    }
  }
  for (int64_t b = 0; b < n->B; ++b) n->len[(size_t)b] += steps;
  return IMIE_OK;
}

// Ragged page allocation (no reference counterpart): sequence b gets room for caps[b] positions. Replaces the
// cache (its contents are discarded and every sequence length restarts at 0).
int imie_net_set_caps(int64_t ctx, const int64_t* caps) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  Net* n = net_get(ctx);
  if (!n || !caps) return IMIE_EARG;
  for (int64_t b = 0; b < n->B; ++b)                  // no position beyond the RoPE tables is ever usable
    if (caps[b] <= 0 || caps[b] > n->rope_rows) return IMIE_EARG;
  IMIE_HIP(hipDeviceSynchronize());
  if (n->gexec) { (void)hipGraphExecDestroy(n->gexec); n->gexec = nullptr; }
  net_free_kv(*n);
  return net_alloc_kv(*n, std::vector<int64_t>(caps, caps + n->B), n->P, n->kv32);
}

// Restart every sequence at length 0, keeping the allocated pools and page tables (no reference counterpart; the
// receipt verifier's repeated prefills of one context). Clears the kv8 running maxima. Synchronous.
int imie_net_reset(int64_t ctx) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  Net* n = net_get(ctx);
  if (!n) return IMIE_EARG;
  IMIE_HIP(hipDeviceSynchronize());
  n->len.assign((size_t)n->B, 0);
  if (n->kv32 && n->kvrun.p) IMIE_HIP(hipMemset(n->kvrun.p, 0, (size_t)(n->nl * 2 * n->B * n->Hkv) * 8));
  return IMIE_OK;
}

// Fill every layer's cache with seeded synthetic K / V for lens[b] positions per sequence, on the device (no
// reference counterpart; the workload generator of the benchmark and the large-context tests). Values are
// uniform in [lo, hi); see kv_fill_kernel for the stream; seq_ids[b] (0..511, nullptr: b) keys sequence b's
// draw, so one sequence can be regenerated alone in another context. Sets the sequence lengths.
int imie_net_fill_kv(int64_t ctx, uint64_t seed, const int64_t* lens, const int64_t* seq_ids, int64_t lo,
                     int64_t hi) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  Net* n = net_get(ctx);
  if (!n || !lens || hi <= lo || (n->P & (n->P - 1)) != 0) return IMIE_EARG;
  if (n->kv32 && (!imie_kv8::fits(lo) || !imie_kv8::fits(hi - 1))) return IMIE_EOVF;
  int64_t lmax = 0;
  for (int64_t b = 0; b < n->B; ++b) {
    if (lens[b] < 0 || lens[b] > pos_cap(*n, b)) return IMIE_EARG;
    lmax = lens[b] > lmax ? lens[b] : lmax;
  }
  hipStream_t st = imie_stream();
  std::vector<int64_t> ls((size_t)(2 * n->B));
  for (int64_t b = 0; b < n->B; ++b) {
    ls[(size_t)b] = lens[b];
    ls[(size_t)(n->B + b)] = seq_ids ? seq_ids[b] : b;
    if (ls[(size_t)(n->B + b)] < 0 || ls[(size_t)(n->B + b)] >= 512) return IMIE_EARG;
  }
  DevBuf dl;
  if (dl.ensure((size_t)n->B * 16)) return IMIE_EARG;
  IMIE_HIP(hipMemcpy(dl.p, ls.data(), (size_t)n->B * 16, hipMemcpyHostToDevice));
  int pshift = 0;
  while (((int64_t)1 << pshift) < n->P) ++pshift;
  const unsigned gx = (unsigned)std::min<int64_t>(1024, (lmax * n->hd + 255) / 256 + 1);
  for (int64_t l = 0; l < n->nl; ++l)
    for (int kind = 0; kind < 2; ++kind) {
      uint64_t* run = n->kv32 ? (kind == 0 ? run_k(*n, l) : run_v(*n, l)) : nullptr;
      hipLaunchKernelGGL(kv_fill_kernel, dim3(gx, (unsigned)n->Hkv, (unsigned)n->B), dim3(256), 0, st,
                         kind == 0 ? n->kpool[(size_t)l] : n->vpool[(size_t)l], (const int64_t*)n->pt, n->mp, n->P,
                         pshift, n->Hkv, n->hd, (const int64_t*)dl.p, (const int64_t*)dl.p + n->B, seed, l, kind, lo,
                         (uint64_t)(hi - lo),
                         n->kv32, run);
      IMIE_HIP(hipGetLastError());
    }
  IMIE_HIP(hipStreamSynchronize(st));
  dl.release();
  for (int64_t b = 0; b < n->B; ++b) n->len[(size_t)b] = lens[b];
  return IMIE_OK;
}

// Clear (0) or read the context status word: 0 ok, bit 2 attention / RoPE / int32-KV envelope, bit 4 RMSNorm.
int imie_net_status(int64_t ctx, int clear, void* stream) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  Net* n = net_get(ctx);
  if (!n || n->status.ensure(64)) return -1;
  hipStream_t st = (hipStream_t)stream;
  if (clear) return fill_i64((int64_t*)n->status.p, 1, 0, st) ? -1 : 0;
  int stat = 0;
  if (read_status(*n, st, &stat)) return -1;
  return stat;
}

// Copy sequence b's cached K/V of `layer` for positions [0, count) to host (Hkv, count, hd) int64.
int imie_net_export_kv(int64_t ctx, int64_t layer, int64_t b, int64_t count, int64_t* k_out, int64_t* v_out) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  Net* n = net_get(ctx);
  if (!n || !k_out || !v_out || layer < 0 || layer >= n->nl || b < 0 || b >= n->B || count < 0 ||
      count > seq_cap(*n, b))
    return IMIE_EARG;
  IMIE_HIP(hipStreamSynchronize(imie_stream()));
  IMIE_HIP(hipDeviceSynchronize());
  const size_t esz = n->kv32 ? 4 : 8;
  const size_t seq = (size_t)(n->npg[(size_t)b] * n->Hkv * n->P * n->hd);
  std::vector<char> kb(seq * esz), vb(seq * esz);
  const size_t off = (size_t)n->pg0[(size_t)b] * n->Hkv * n->P * n->hd * esz;
  IMIE_HIP(hipMemcpy(kb.data(), (char*)n->kpool[(size_t)layer] + off, kb.size(), hipMemcpyDeviceToHost));
  IMIE_HIP(hipMemcpy(vb.data(), (char*)n->vpool[(size_t)layer] + off, vb.size(), hipMemcpyDeviceToHost));
  for (int64_t kv = 0; kv < n->Hkv; ++kv)
    for (int64_t j = 0; j < count; ++j)
      for (int64_t c = 0; c < n->hd; ++c) {
        const int64_t pgl = j / n->P, slot = j % n->P;
        const size_t dst = (size_t)((kv * count + j) * n->hd + c);
        if (n->kv32) {
          const int64_t base = imie_kv8::block_base(pgl, kv, n->Hkv, n->hd, n->P);
          int8_t kd[4], vd[4];
          for (int db = 0; db < 4; ++db) {
            kd[db] = (int8_t)kb[(size_t)(base + imie_kv8::k_off(slot, db, c, n->hd))];
            vd[db] = (int8_t)vb[(size_t)(base + imie_kv8::v_off(slot, db, c, n->hd, n->P))];
          }
          k_out[dst] = imie_kv8::decode4(kd[0], kd[1], kd[2], kd[3]);
          v_out[dst] = imie_kv8::decode4(vd[0], vd[1], vd[2], vd[3]);
        } else {
          const size_t src = (size_t)(pgl * (n->Hkv * n->P * n->hd) + kv * n->P * n->hd + slot * n->hd + c);
          k_out[dst] = ((int64_t*)kb.data())[src];
          v_out[dst] = ((int64_t*)vb.data())[src];
        }
      }
  return IMIE_OK;
}

// Q1 embedding rows on the device: out (T, nb*128) = sign * scale of rows ids (device int64) of a natural-layout
// table (bits (V, nb, 16), scale (V, nb) int64, both device pointers).
int imie_embed_dev(const uint8_t* bits, const int64_t* scale, int64_t nb, const int64_t* ids, int64_t T, int64_t* out,
                   void* stream) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!bits || !scale || !ids || !out || nb <= 0 || T < 0) return IMIE_EARG;
  return imie_embed_launch(bits, scale, nb, ids, T, out, (hipStream_t)stream);
}

}  // extern "C"
