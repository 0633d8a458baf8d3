// Internal launchers shared by the C-ABI files (device pointers, asynchronous on `st`).
#pragma once
#include "imie_common.h"
#include "imie_q1prep.h"

// status word bits (device int, OR-ed by kernels): IMIE_EOVF (2) attention / RoPE / int32-KV envelope,
// IMIE_ERMS (4) RMSNorm envelope.

int imie_rmsnorm_launch(const int64_t* x, int64_t rows, int64_t cols, int64_t frac, int64_t eps,
                        const int64_t* gain, int64_t* out, int* status, hipStream_t st);

// Q1 apply on a registered handle. accumulate != 0 adds the result into out (residual add fused).
int imie_q1_launch(int64_t handle, const int64_t* x, int64_t T, int64_t frac, int64_t* out, int accumulate,
                   hipStream_t st);
int imie_q1_dims(int64_t handle, int64_t* N, int64_t* nb);
// Per-caller Q1 activation workspace (digit table, block totals, limb counts). A caller that captures its launches
// into a graph owns one, so no other call can reallocate the buffers the graph points at.
struct Q1Ws {
  DevBuf xq, totals, lslab;
  DevBuf wide;                     // GEMM: per 64-token tile, whether any slab needs more than 3 limbs
};
// Up to 3 weights with the same n_blocks applied to the same x in one prep + one matvec launch (wk == nullptr:
// the library's shared workspace).
// prepped != 0: the digit table is already in wk (written by a fused producer through imie_q1_prep_target) and
// the non-accumulated outputs are already zero.
int imie_q1_launch_multi(const int64_t* handles, int cnt, const int64_t* x, int64_t T, int64_t frac,
                         int64_t* const* outs, int accumulate, Q1Ws* wk, hipStream_t st, int prepped = 0);
// Size wk for T tokens of nb blocks and describe it for a producer that writes the digit table itself.
int imie_q1_prep_target(Q1Ws* wk, int64_t nb, int64_t T, imie_q1::Q1PrepOut* po);
// RMSNorm rows of cols = nb * 128 (<= 4096) that also write the Q1 digit table of the output (po) and clear
// the zero list, for a following matvec launched with prepped = 1.
int imie_rmsnorm_prep_launch(const int64_t* x, int64_t rows, int64_t cols, int64_t frac, int64_t eps,
                             const int64_t* gain, int64_t* out, int* status, const imie_q1::Q1PrepOut& po,
                             const imie_q1::Q1Zero& zero, hipStream_t st);
// h = silu(gate) * up >> frac (as imie_silu_mul_launch) for T rows of n = nb * 128 that also writes the digit
// table of h (po).
int imie_silu_mul_prep_launch(const int64_t* gate, const int64_t* up, int64_t T, int64_t n, int64_t frac,
                              int64_t* out, const imie_q1::Q1PrepOut& po, hipStream_t st);

// The SiLU constants for frac fraction bits (log2(e) in fixed point and the exponent clip).
void imie_silu_consts(int64_t frac, int64_t* log2e, int64_t* dclip);
// Single-token matvec whose workgroups derive the digit table of their slab range from the producer's inputs
// (imie_q1::Q1Pro, kind kProCopy / kProSiluMul / kProNorm) in place of a prep kernel; pro.zero is cleared on the
// way. K-split outputs are added into: with accumulate == 0 they must be clear before the launch.
// imie_q1_pro_ok: whether the weights (same n_blocks, int32 scales, K == pro.cols) take this path.
int imie_q1_pro_ok(const int64_t* handles, int cnt, int kind, int64_t cols);
int imie_q1_launch_pro(const int64_t* handles, int cnt, const imie_q1::Q1Pro& pro, int kind, int64_t frac,
                       int64_t* const* outs, int accumulate, hipStream_t st);

// NeoX RoPE on rows x (rows, nh, hd); row r uses table row pos[r] (pos == nullptr: pos0 + r).
// The fail-loud envelope 2*max|x|*max|cos,sin| <= INT64_MAX is checked exactly via `guard` scratch
// (2 x uint64, zeroed by the caller) and reported in `status` by imie_rope_guard_check.
int imie_rope_launch(const int64_t* x, int64_t rows, int64_t nh, int64_t hd, const int64_t* pos, int64_t pos0,
                     const int64_t* cos, const int64_t* sin, int64_t frac, int64_t* out, uint64_t* guard,
                     hipStream_t st);
int imie_rope_guard_check(const uint64_t* guard, int* status, hipStream_t st);

// h = ((silu(gate) * up) >> frac) with the bonsai wrap semantics (reference_bonsai.py:245-264, 611-614)
// The GEMM digit table (T >= kGemmMinT) of wk for weights of nb blocks; a producer that writes it passes
// prepped = 2 to imie_q1_launch_multi.
int imie_q1_gemm_target(Q1Ws* wk, int64_t nb, int64_t T, imie_q1::GemmPrepOut* gp);
// h = silu(gate) * up >> frac for T >= kGemmMinT rows of n = nb * 128 straight into the GEMM digit table gp (h
// itself is not stored): SiLU * up fused with the prep of the next GEMM.
// RMSNorm of rows >= kGemmMinT rows (cols = nb * 128 <= 4096) that also writes the next GEMM's digit table gp
// and clears the outputs in `zero` (for a K-split GEMM, which then adds into them: prepped = 3)
int imie_rmsnorm_gemm_prep_launch(const int64_t* x, int64_t rows, int64_t cols, int64_t frac, int64_t eps,
                                  const int64_t* gain, int64_t* out, int* status, const imie_q1::GemmPrepOut& gp,
                                  const imie_q1::Q1Zero& zero, hipStream_t st);
// Whether the GEMM of weight `handle` over T tokens is expected to split K (its outputs are then worth clearing
// in the producer); a wrong guess costs a redundant clear or a separate one, never a wrong result
int imie_q1_gemm_splits(int64_t handle, int64_t T);
int imie_silu_mul_gemm_prep_launch(const int64_t* gate, const int64_t* up, int64_t T, int64_t n, int64_t frac,
                                   const imie_q1::GemmPrepOut& gp, hipStream_t st);
int imie_silu_mul_launch(const int64_t* gate, const int64_t* up, int64_t n, int64_t frac, int64_t* out,
                         hipStream_t st);
int imie_silu_launch(const int64_t* x, int64_t n, int64_t frac, int64_t* out, hipStream_t st);
int imie_add_launch(int64_t* x, const int64_t* y, int64_t n, hipStream_t st);
// embedding rows: out[t] = sign(bits[ids[t]]) * scale[ids[t]] (no frac shift), natural Q1 layout
int imie_embed_launch(const uint8_t* bits, const int64_t* scale, int64_t nb, const int64_t* ids, int64_t T,
                      int64_t* out, hipStream_t st);
// lowest-index argmax per row of (rows, cols) int64
// scratch: device buffer of imie_argmax_scratch_bytes(rows) bytes (two-stage reduction partials)
constexpr int kArgmaxParts = 256;
inline size_t imie_argmax_scratch_bytes(int64_t rows) { return (size_t)rows * kArgmaxParts * 16; }
int imie_argmax_launch(const int64_t* logits, int64_t rows, int64_t cols, int64_t* ids, int64_t* scratch,
                       hipStream_t st);

// Fused head RMSNorm + RoPE + KV-cache append for rows = B * M new rows (see qkhead.hip). q, k, v: projection
// outputs (rows, H|Hkv, hd); qo receives the rotated q; k (rotated) and v go to the paged cache at pos[row].
struct QkHeadArgs {
  const int64_t *q, *k, *v;
  int64_t* qo;
  const int64_t *qng, *kng, *pos, *cos, *sin;
  int64_t rows, H, Hkv, hd, M, eps;
  int frac;
  const int64_t* pt;
  int64_t P, mp;
  void *kpool, *vpool;
  uint64_t* guard;                 // 4 x u64, zeroed before the launch (RoPE envelope maxima)
  int* status;
  // kv8 cache only: max|k|, max|v| of the appended rows per (row, kv head) [rows][Hkv] (M > 1), or folded
  // straight into the running per-(sequence, kv head) maxima run_k / run_v [B][Hkv] (M == 1)
  uint64_t *rowk, *rowv, *run_k, *run_v;
  // kv8 decode (optional): rotated q as 8 balanced digit planes qd[row * H + h][8][hd], max|q| and limb count per
  // (row, head), consumed directly as MFMA A operands by the decode attention
  int8_t* qd;
  uint64_t* qmax;
  int* qlimbs;
  // several rows: per-workgroup RoPE envelope maxima gpart[(row * (H + Hkv) + head) * 2 + {0, 1}] instead of
  // same-address atomics from every workgroup (reduced into guard by imie_qk_head_finish_launch); with M > 1 the
  // kv8 V planes are also appended by that launch's coalesced kernel instead of per-element byte scatters
  uint64_t* gpart;
};
// kv8 = 1: the digit-plane cache of imie_kvfmt.h; 0: int64 rows
int imie_qk_head_launch(const QkHeadArgs& a, int kv8, hipStream_t st);
// after imie_qk_head_launch with gpart set: guard <- max over gpart; kv8 with M > 1: the V digit planes of the new
// rows, and their maxima (rowk / rowv) folded into run_k / run_v
int imie_qk_head_finish_launch(const QkHeadArgs& a, int kv8, hipStream_t st);

// Integer sampler config (committed fixed-point settings; layout shared with include/imie_bonsai.h).
// mode: 0 greedy, 1 temp, 2 top_k, 3 top_p, 4 min_p (the reference ABI's numbering, bonsai_q1_gpu.cu:905-910)
struct ImieSamplerConfig {
  int64_t mode, frac, inv_temp, top_k, top_p, min_p, rep_penalty, no_repeat_ngram, seed;
};
// tokens of `rows` logits rows (stride ld) into token[r]; per-row history / positions on the device.
// Single-stream: the flag, probability, key and sort scratch is one library-wide set, so two calls in flight on
// different streams at once race on it (the library lock serialises the enqueues, not the kernels).
int imie_sample_launch(const int64_t* logits, int64_t rows, int64_t V, int64_t ld, const ImieSamplerConfig& c,
                       const int64_t* hist, int64_t hld, const int64_t* hlen, const int64_t* pos, int64_t* token,
                       int* status, hipStream_t st);
