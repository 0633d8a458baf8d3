/* imie — gfx950 producer C-ABI, Bonsai (Qwen3-dense, packed Q1_0) half.
 *
 * Conventions (reference: bonsai/src/trinote/infer_int/gpu_native.py:34-185 and bonsai/tools/bonsai_q1_gpu.cu):
 *   all scalars int64; host pointers are C-contiguous buffers owned by the caller; calls are synchronous;
 *   rc 0 ok, 1 bad args / runtime failure, 2 attention overflow, 4 RMSNorm overflow. Handles index
 *   process-global registries that live until the matching *_free call. Not reentrant (one caller at a time;
 *   entry points serialize on a process lock).
 * Entry points prefixed imie_ have no counterpart in the reference: they take DEVICE pointers and an optional
 * hipStream_t (as void*; NULL is HIP's null stream) and are asynchronous.
 */
#ifndef IMIE_BONSAI_H
#define IMIE_BONSAI_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ---- runtime ---------------------------------------------------------------------------------------- */
/* bonsai_q1_gpu.cu `bonsai_gpu_available` (bound at gpu_native.py:174-184): 0 iff a gfx950 device is usable. */
int bonsai_gpu_available(void);
/* bonsai_q1_gpu.cu `bonsai_gpu_mem_info` (gpu_native.py:107-115, 309-331). */
int bonsai_gpu_mem_info(uint64_t *free_bytes, uint64_t *total_bytes);
/* bonsai_q1_gpu.cu:1970-1972 `bonsai_gpu_abi_version`: the bonsai_* ABI generation mirrored here (3). */
int bonsai_gpu_abi_version(void);
/* bonsai_q1_gpu.cu:1974-1980 `bonsai_gpu_last_error_code` / `bonsai_gpu_last_error` (read by gpu_bonsai35.py:52-58):
 * the last HIP error any entry point noted (number, text). */
int bonsai_gpu_last_error_code(void);
const char *bonsai_gpu_last_error(void);
int imie_abi_version(void);
const char *imie_last_error(void);
void *imie_default_stream(void);
int imie_synchronize(void);
/* per-kernel HIP-event timing on the stream each kernel runs on (kernel ids: 0 q1 prep, 1 q1 matvec,
 * 2 q1 GEMM, 3 attention, 4 Q4_K/Q6_K linear); read synchronizes. */
void imie_profile_begin(void);
int imie_profile_read(int kernel, double *total_ms, int64_t *count);
/* Executed int8 MFMA ops of the Q1 GEMM launches (prefill) recorded while profiling is on, counted on the device
 * from the limb tables (synchronizes); reset != 0 clears the counter. No reference counterpart (measurement). */
int imie_profile_gemm_ops(unsigned long long *ops, int reset);
void imie_profile_end(void);
/* one int8 MFMA over per-lane operands (A, B: 64x16 int8, D: 64x4 int32); pins the lane mapping in tests. */
int imie_probe_mfma(const int8_t *a, const int8_t *b, int32_t *d);
/* Sustained int8 MFMA throughput of the device in ops/s (8 independent 16x16x64 chains per wave, 4 waves per
 * SIMD, HIP events). No reference counterpart (measurement: the measured peak the prefill GEMM is quoted against). */
int imie_mfma_peak(double *ops_per_s);
/* Sustained HBM read bandwidth in bytes/s over a `bytes` (>= 16 MiB) device buffer: nontemporal 16-byte loads from
 * 16 workgroups per CU, best of three timed launches. No reference counterpart (measurement: the practical read
 * ceiling the Q1 matvec is quoted against beside the published 8 TB/s). */
int imie_hbm_read_peak(int64_t bytes, double *bytes_per_s);

/* ---- packed Q1_0 linear: out[t,o] = sum_b ((sum_i sign*x) * scale[o,b]) >> frac, mod 2^64 ----------- */
/* bonsai_q1_gpu.cu:2200-2241 `bonsai_q1_linear_gpu` (bound at gpu_native.py:44-52, called :212-217). */
int bonsai_q1_linear_gpu(const int64_t *x, const uint8_t *bits, const int64_t *scale, int64_t tokens,
                         int64_t out_features, int64_t n_blocks, int64_t frac, int64_t *out);
/* bonsai_q1_gpu.cu `bonsai_q1_register_weight` (gpu_native.py:73-74, 270-306): handle >= 0 or -1. */
int64_t bonsai_q1_register_weight(const uint8_t *bits, const int64_t *scale, int64_t out_features, int64_t n_blocks);
/* bonsai_q1_gpu.cu `bonsai_q1_register_weight_i32` (gpu_native.py:79-87). */
int64_t bonsai_q1_register_weight_i32(const uint8_t *bits, const int32_t *scale, int64_t out_features,
                                      int64_t n_blocks);
/* bonsai_q1_gpu.cu:2350-2366 `bonsai_q1_register_weight_i32_gpu_layout` (gpu_native.py:89-96, 286-306): the
 * reference's coalesced runtime layout; every registration here is already the gfx950 tile-major layout. */
int64_t bonsai_q1_register_weight_i32_gpu_layout(const uint8_t *bits, const int32_t *scale, int64_t out_features,
                                                 int64_t n_blocks);
/* bonsai_q1_gpu.cu:2368-2385 `bonsai_q1_register_weight_i32_bmma` (gpu_native.py:98-105, 286-306): -1 unless
 * out_features % 8 == 0, as there; stored in the same tile-major layout. */
int64_t bonsai_q1_register_weight_i32_bmma(const uint8_t *bits, const int32_t *scale, int64_t out_features,
                                           int64_t n_blocks);
/* bonsai_q1_gpu.cu:2245-2300 `bonsai_q1_linear_dp4a_gpu` (bound at gpu_native.py:55-64, called :235-261): the Q1
 * linear of x taken as L balanced base-256 digits (|L| in 1..8, L < 0 the reference's warp variant, same bytes).
 * rc 0; 1 bad arguments; 4 when |L| == 4 and some |x| > 2,139,062,143 (nothing computed). x needing more than L
 * digits is truncated to its low L digits (mod 2^64) as the reference's digit kernel does. */
int bonsai_q1_linear_dp4a_gpu(const int64_t *x, const uint8_t *bits, const int64_t *scale, int64_t tokens,
                              int64_t out_features, int64_t n_blocks, int64_t frac, int L, int64_t *out);
/* bonsai_q1_gpu.cu:2388-2423 `bonsai_q1_apply_resident` (gpu_native.py:75-76, 364-380). */
int bonsai_q1_apply_resident(int64_t handle, const int64_t *x, int64_t tokens, int64_t frac, int64_t *out);
/* bonsai_q1_gpu.cu `bonsai_q1_free_weights` (gpu_native.py:77-78, 383-387). */
void bonsai_q1_free_weights(void);
/* bonsai_q1_gpu.cu `bonsai_q1_resident_weight_bytes` (gpu_native.py:108-115). */
uint64_t bonsai_q1_resident_weight_bytes(void);
/* host-side tile repack used at registration (exposed for CPU tests). */
int imie_q1_repack_host(const uint8_t *bits, const int64_t *scale, int64_t N, int64_t n_blocks, int scale64,
                        uint8_t *bits_tiled, void *scale_tiled);
/* device-pointer resident apply, asynchronous on `stream`. */
int imie_q1_apply_dev(int64_t handle, const int64_t *x_dev, int64_t tokens, int64_t frac, int64_t *out_dev,
                      void *stream);
/* No reference counterpart: imie_q1_apply_dev for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc). Same arguments and results; the digit-table workspace
 * is a fixed 1.8 MiB device array held per device for the life of the process. tokens <= 7 and n_blocks <= 256
 * (K <= 32768), else rc 1 (reason in imie_last_error). Calls overlapping on one device race on that array. */
int imie_q1_apply_dev_noalloc(int64_t handle, const int64_t *x_dev, int64_t tokens, int64_t frac, int64_t *out_dev,
                              void *stream);
int imie_q1_weight_info(int64_t handle, int64_t *out_features, int64_t *n_blocks, int64_t *scale_bytes);
/* exact thread-per-output kernel over natural-layout device buffers (cross-check path). */
int imie_q1_linear_simple_dev(const int64_t *x_dev, const uint8_t *bits_dev, const int64_t *scale_dev,
                              int64_t tokens, int64_t out_features, int64_t n_blocks, int64_t frac,
                              int64_t *out_dev, void *stream);

/* ---- integer RMSNorm / element-wise ---------------------------------------------------------------- */
/* bonsai_q1_gpu.cu:625-670 `bonsai_rmsnorm_gpu` (gpu_native.py:129-138, 390-415): rc 4 on the 128-bit / gain envelope. */
int bonsai_rmsnorm_gpu(const int64_t *x, int64_t rows, int64_t cols, int64_t frac, int64_t eps, const int64_t *gain,
                       int64_t *out);
/* The fused RMSNorm producer of the resident decode (it also writes the next Q1 matvec's digit table, kept in
 * a workspace here) with the host contract of bonsai_rmsnorm_gpu; cols a multiple of 128, at most 4096. No
 * reference counterpart: it exposes the fused kernel to the parity tests. */
int imie_rmsnorm_fused_gpu(const int64_t *x, int64_t rows, int64_t cols, int64_t frac, int64_t eps,
                           const int64_t *gain, int64_t *out);
int imie_rmsnorm_dev(const int64_t *x, int64_t rows, int64_t cols, int64_t frac, int64_t eps, const int64_t *gain,
                     int64_t *out, int *status, void *stream);
/* bonsai_q1_kernel.c:1729-1767 `bonsai_silu_i64` (q1_native.py:1895 `silu_native`) on the GPU: (x*sigmoid(x))>>frac. */
int bonsai_silu_gpu(const int64_t *x, int64_t n, int64_t frac, int64_t *out);
/* rope_v2.py:92-117 NeoX apply (bonsai_q1_gpu.cu:812-827 / :1746-1761 `rope_kernel` / `rope_decode_kernel`);
 * row r uses table row pos[r]; rc 2 where the oracle raises (rope.py:26-39). */
int imie_rope_neox_gpu(const int64_t *x, int64_t rows, int64_t nh, int64_t hd, const int64_t *pos, const int64_t *cos,
                       const int64_t *sin, int64_t n_pos, int64_t frac, int64_t *out);
/* lowest-index argmax (reference_bonsai.py:812-827; bonsai_q1_kernel.c:468-543 merge rule). */
int imie_argmax_gpu(const int64_t *logits, int64_t rows, int64_t cols, int64_t *ids);

/* ---- fixed-point attention -------------------------------------------------------------------------- */
/* bonsai_q1_gpu.cu:731-797 `bonsai_attention_prefill_gpu` (gpu_native.py:139-151, 418-446). */
int bonsai_attention_prefill_gpu(const int64_t *q, const int64_t *k, const int64_t *v, int64_t H, int64_t Hkv,
                                 int64_t hd, int64_t M, int64_t L, int64_t start, int64_t frac, int64_t inv_sqrt,
                                 int64_t *out);
/* bonsai_q1_gpu.cu:1409-1470 `bonsai_attention_decode_batched_gpu` (gpu_native.py:449-468). */
int bonsai_attention_decode_batched_gpu(const int64_t *q, const int64_t *K, const int64_t *V, const int64_t *lengths,
                                        int64_t B, int64_t H, int64_t Hkv, int64_t hd, int64_t cap, int64_t frac,
                                        int64_t inv_sqrt, int64_t *out);

/* stage probe (tests): runs the causal pipeline with V = K up to `stage` (1 scores, 2 softmax, 3 PV) and returns
 * the score/probability rows (H*M, L), the row maxima (H*M) and, at stage 3, the int64 PV accumulator (H*M, hd). */
int imie_attention_scores_probe(const int64_t *q, const int64_t *k, int64_t H, int64_t Hkv, int64_t hd, int64_t M,
                                int64_t L, int64_t start, int64_t frac, int64_t inv_sqrt, int64_t *scores,
                                int64_t *rowmax, int stage, int64_t *acc_out);

/* ---- resident model: monolith prefill and decode context -------------------------------------------- */
/* bonsai_q1_gpu.cu `bonsai_buf_upload_i64` (gpu_native.py:154-160, 549-556): handle >= 0 or -1. */
int64_t bonsai_buf_upload_i64(const int64_t *host, int64_t n);
const int64_t *imie_buf_device_ptr(int64_t handle);
void imie_buf_free_all(void);
/* bonsai_q1_gpu.cu:3694-3819 `bonsai_prefill_forward_gpu` (gpu_native.py:161-172, 559-595). */
int bonsai_prefill_forward_gpu(const int64_t *x_embed, int64_t T, int64_t d, int64_t n_layers, int64_t H, int64_t Hkv,
                               int64_t hd, int64_t dff, int64_t frac, int64_t eps, int64_t inv_sqrt,
                               const int64_t *wq, const int64_t *wk, const int64_t *wv, const int64_t *wo,
                               const int64_t *w1, const int64_t *wu, const int64_t *w2, const int64_t *n1g,
                               const int64_t *n2g, const int64_t *qng, const int64_t *kng, int64_t finalg,
                               int64_t out_head, int64_t cos_h, int64_t sin_h, int64_t *out_logits, int64_t *out_k,
                               int64_t *out_v);
/* bonsai_q1_gpu.cu:3517-3562 `bonsai_decode_ctx_create` (gpu_native.py:483-506). */
int64_t bonsai_decode_ctx_create(int64_t B, int64_t n_layers, int64_t H, int64_t Hkv, int64_t hd, int64_t d,
                                 int64_t dff, int64_t cap, int64_t vocab, int64_t frac, int64_t eps, int64_t inv_sqrt,
                                 const int64_t *wq, const int64_t *wk, const int64_t *wv, const int64_t *wo,
                                 const int64_t *w1, const int64_t *wu, const int64_t *w2, const int64_t *n1g,
                                 const int64_t *n2g, const int64_t *qng, const int64_t *kng, int64_t finalg,
                                 int64_t out_head, int64_t cos_h, int64_t sin_h);
/* paged int32 (guarded) / int64 context; out_head < 0 = layers only. */
int64_t imie_net_create(int64_t B, int64_t n_layers, int64_t H, int64_t Hkv, int64_t hd, int64_t d, int64_t dff,
                        int64_t cap, int64_t frac, int64_t eps, int64_t inv_sqrt, const int64_t *wq, const int64_t *wk,
                        const int64_t *wv, const int64_t *wo, const int64_t *w1, const int64_t *wu, const int64_t *w2,
                        const int64_t *n1g, const int64_t *n2g, const int64_t *qng, const int64_t *kng,
                        int64_t finalg, int64_t out_head, int64_t cos_h, int64_t sin_h, int64_t page, int kv32);
/* bonsai_q1_gpu.cu:3565-3584 `bonsai_decode_ctx_seed_seq` (gpu_native.py:509-521). */
int bonsai_decode_ctx_seed_seq(int64_t ctx, int64_t b, const int64_t *k, const int64_t *v, int64_t Lb);
/* bonsai_q1_gpu.cu:3588-3647 `bonsai_decode_step` (gpu_native.py:524-538). */
int bonsai_decode_step(int64_t ctx, const int64_t *x_in, const int64_t *pos, int64_t *out);
/* bonsai_q1_gpu.cu `bonsai_decode_ctx_free` (gpu_native.py:541-546). */
void bonsai_decode_ctx_free(int64_t ctx);
int imie_net_forward_dev(int64_t ctx, int64_t *x_dev, const int64_t *starts, int64_t M, void *stream);
int imie_net_head_dev(int64_t ctx, const int64_t *x_dev, int64_t rows, int64_t *logits_dev, int64_t *ids_dev,
                      void *stream);
int imie_net_status(int64_t ctx, int clear, void *stream);
int imie_net_export_kv(int64_t ctx, int64_t layer, int64_t b, int64_t count, int64_t *k_out, int64_t *v_out);
/* Greedy decode of `steps` tokens on the device: embed -> all layers -> final norm + LM head -> lowest-index
 * argmax, per step (the host-driven loop of reference_bonsai.py:1200-1310 moved onto the GPU; no single
 * reference entry point). ids_dev (B) in/out, logits_dev (B, vocab) = last step's logits, hist_dev (steps, B)
 * optional; use_graph replays a captured HIP graph of one step after the first. */
int imie_net_decode_dev(int64_t ctx, const uint8_t *ebits, const int64_t *escale, int64_t *ids_dev,
                        int64_t *logits_dev, int64_t *hist_dev, int64_t steps, int use_graph, void *stream);
/* Ragged paged cache: sequence b gets room for caps[b] positions; the cache is replaced (lengths restart at 0).
 * No reference counterpart (the reference decode context is dense). */
int imie_net_set_caps(int64_t ctx, const int64_t *caps);
/* Every sequence back to length 0 with the pools kept (no reference counterpart: the receipt verifier's repeated
   prefills). Synchronous. */
int imie_net_reset(int64_t ctx);
/* gpu_native.py:334-361 / bonsai_q1_gpu.cu:2160-2197 `bonsai_gpu_reservation_create` / `_free`: reserve several
   exact device allocations as one failure-atomic probe (returns the handle and the bytes taken, or -1 with nothing
   left allocated); freeing twice is a no-op. */
int64_t bonsai_gpu_reservation_create(const uint64_t *sizes, int64_t count, uint64_t *allocated);
void bonsai_gpu_reservation_free(int64_t handle);
/* Seeded synthetic K/V for lens[b] positions per sequence, generated on the device (benchmark / large-context
 * test workloads; no reference counterpart). Values uniform in [lo, hi); seq_ids (nullable) keys each
 * sequence's draw. */
int imie_net_fill_kv(int64_t ctx, uint64_t seed, const int64_t *lens, const int64_t *seq_ids, int64_t lo,
                     int64_t hi);
/* CPU test hooks for the exact RMSNorm arithmetic (no reference counterpart): floor(sqrt(hi*2^64 + lo)),
 * floor((2^64 - 1) / d), low 64 bits of floor((hi*2^64 + lo) / d). */
uint64_t imie_fx_isqrt_u128(uint64_t hi, uint64_t lo);
uint64_t imie_fx_recip_u64(uint64_t d);
uint64_t imie_fx_div_u128(uint64_t hi, uint64_t lo, uint32_t d);
/* CPU test hooks for the short paths of the single-token matvec prologue (no reference counterpart): the
 * double-precision isqrt below 2^52; n = floor((x << frac) / rms) in double precision (returns 1 when that path
 * applies, 0 when the integer routine would be taken); (silu(g) * u) >> frac by the two-exponential form
 * (fast = 0) or the one-exponential form (fast = 1). */
uint64_t imie_fx_isqrt_fast(uint64_t hi, uint64_t lo);
int imie_fx_norm_f64(int64_t x, int frac, uint64_t rms, int64_t *out);
int64_t imie_silu_mul_host(int64_t g, int64_t u, int64_t frac, int fast);
/* The softmax short paths (no reference counterpart; CPU tests pin them): exp2_neg_fixed((d * log2e) >> frac) of a
   clipped difference (fast != 0: the 32-bit form when the constants allow), and floor((e << frac) / z). */
int64_t imie_exp_clipped_host(int64_t d, int64_t frac, int fast);
int64_t imie_prob_div_host(int64_t e, int64_t frac, uint64_t z);
/* Q1 embedding rows sign*scale (reference_bonsai.py:138-146) from device tables. */
int imie_embed_dev(const uint8_t *bits, const int64_t *scale, int64_t nb, const int64_t *ids, int64_t T, int64_t *out,
                   void *stream);

/* ---- host (CPU) re-execution for receipt verification (bonsai/src/trinote/infer_int/verify.py:156-272: the
 * reference verifier re-derives turns on its CPU reference engine; this is that role, independent of the GPU). ---- */
/* A host model over the caller's arrays (borrowed): 7 Q1_0 projections per layer (wq, wk, wv, wo, w1, wu, w2) as
 * bits (out, in/128, 16) / int64 scales (out, in/128), 4 int64 gains per layer (n1, n2, q-norm, k-norm), the Q1_0
 * embedding and output head, the final gain and the RoPE tables (rope_rows, hd/2). Handle >= 0 or -1. */
int64_t imie_cpu_model_create(int64_t n_layers, int64_t H, int64_t Hkv, int64_t hd, int64_t d, int64_t dff,
                              int64_t vocab, int64_t frac, int64_t eps, int64_t inv_sqrt,
                              const uint8_t *const *w_bits, const int64_t *const *w_scale,
                              const int64_t *const *gains, const uint8_t *embed_bits, const int64_t *embed_scale,
                              const uint8_t *out_bits, const int64_t *out_scale, const int64_t *final_gain,
                              const int64_t *cos, const int64_t *sin, int64_t rope_rows);
void imie_cpu_model_free(int64_t model);
/* worker threads of the host forward (0: the machine's hardware threads) */
void imie_cpu_set_threads(int threads);
/* ReferenceModelV2.forward (reference_bonsai.py:941-966, 790-827) of ids at positions 0..T-1 on the host: logits
 * (T, vocab) or the last row only. rc 0; 1 bad arguments; 2 an attention / RoPE envelope the reference raises on;
 * 4 RMSNorm (128-bit sum of squares exceeded, or the gain envelope). */
int imie_cpu_forward(int64_t model, const int64_t *ids, int64_t T, int last_only, int64_t *logits);
/* sample_token (sampler.py:403-437) on the host: cfg is an ImieSamplerConfig. rc 0; 1 bad arguments or a history
 * id outside the vocabulary; 2 the temperature envelope. */
int imie_cpu_sample_token(const int64_t *logits, int64_t vocab, const void *cfg, const int64_t *history,
                          int64_t hist_len, int64_t position, int64_t *token);

/* ---- integer samplers (bonsai/src/trinote/infer_int/sampler.py) ------------------------------------------ */
/* Committed fixed-point sampler settings. mode 0 greedy, 1 temp, 2 top_k, 3 top_p, 4 min_p; inv_temp =
 * round(2^frac / T), top_p / min_p in 2^frac units (sampler.py:214-258); the field order and mode numbering follow
 * the reference sampler ABI struct `Bonsai35SamplerConfig` (bonsai/tools/bonsai_q1_gpu.cu:905-910) plus the seed. */
typedef struct ImieSamplerConfig {
  int64_t mode, frac, inv_temp, top_k, top_p, min_p, rep_penalty, no_repeat_ngram, seed;
} ImieSamplerConfig;
/* sample_token (sampler.py:403-437) for one host logits row: replaces the host sampler call at
 * reference_bonsai.py:1110-1146 / :1260-1310 and the device pair bonsai35_sample_prepare / bonsai35_sample_select
 * (bonsai_q1_gpu.cu:3342-3418; the SHA-256 Lemire draw runs on the device here). rc 0, 1 bad arguments or a
 * history token outside the vocabulary, 2 temperature overflow (the reference raises OverflowError). */
int imie_sample_token(const int64_t *logits, int64_t vocab, const ImieSamplerConfig *cfg, const int64_t *history,
                      int64_t history_n, int64_t position, int64_t *token);
/* Device rows (no reference counterpart: the sampled decode step without a logits row on the host): token_dev[r]
 * for logits_dev[r * ld ...], history hist_dev[r * hist_ld + i] (i < hist_len_dev[r]), draw key pos_dev[r].
 * Asynchronous on `stream` (null: the default stream); *status_dev |= 2 on the temperature guard, |= 1 on a bad history token. The first
 * call for a shape sizes the workspace (synchronous); later calls only launch kernels.
 * Single-stream: the sampler's scratch is shared library-wide, so calls overlapping on two streams race. */
int imie_sample_dev(const int64_t *logits_dev, int64_t rows, int64_t vocab, int64_t ld, const ImieSamplerConfig *cfg,
                    const int64_t *hist_dev, int64_t hist_ld, const int64_t *hist_len_dev, const int64_t *pos_dev,
                    int64_t *token_dev, int *status_dev, void *stream);
/* Sampled decode on the device (no reference counterpart for the fused loop): per step embed -> layers -> head
 * -> sampler over the B rows, each token equal to sample_token(row, cfg, len(ids), frac, ids) (sampler.py:403-437)
 * as the reference generate loops call it (reference_bonsai.py:1110-1146, :1260-1310). hist_dev (B, hist_ld)
 * row-major holds every sequence's tokens so far (hist_len_dev[b] of them; the draw key), the drawn token is
 * appended. ids_dev holds the step's input tokens and receives the drawn ones. One step is captured as a graph. */
int imie_net_decode_sampled_dev(int64_t ctx, const uint8_t *ebits, const int64_t *escale, int64_t *ids_dev,
                                int64_t *logits_dev, const ImieSamplerConfig *cfg, int64_t *hist_dev,
                                int64_t hist_ld, int64_t *hist_len_dev, int64_t steps, int use_graph, void *stream);
/* Test hook (no reference counterpart): the device SHA-256 counter word 0 and the Lemire value for
 * (total, seed, position) (sampler.py:283-315). */
int imie_sample_draw_probe(int64_t total, int64_t seed, int64_t position, uint64_t *word0, int64_t *target);
/* logits_digest (sampler.py:421-425) on the device: digest_dev (rows, 32) = SHA-256 of each row's little-endian
   int64 bytes (row stride ld). Used by the receipt re-execution (verify.py:156-235) to commit every row without a
   device-to-host copy of the logits. Asynchronous on `stream` (null: the default stream). */
int imie_logits_digest_dev(const int64_t *logits_dev, int64_t rows, int64_t vocab, int64_t ld, uint8_t *digest_dev,
                           void *stream);

#ifdef __cplusplus
}
#endif
#endif
