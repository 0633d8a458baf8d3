/* imie — gfx950 producer C-ABI, north-mini-code (Q4_K / Q6_K) half.
 *
 * Conventions (reference: north-mini-code/src/nmc/qk_cuda.py:107-223 and tools/nmc_qk_cuda.cu): handles are
 * `long long`, fw / qtype / limb counts `int`; host pointers; synchronous; rc 0 ok, 1 bad args / runtime failure,
 * 2 an int64 result envelope miss (where the big-int oracle's int64 conversion raises). qtype 0 = Q4_K (144-byte
 * blocks), 1 = Q6_K (210-byte blocks); weights are raw GGUF block rows (out_f rows x n_blocks blocks).
 * Entry points prefixed imie_ have no reference counterpart (device pointers, asynchronous on `stream`).
 */
#ifndef IMIE_NMC_H
#define IMIE_NMC_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* nmc_qk_cuda.cu:755 (qk_cuda.py:22, 83-92): the bridge requires 5. */
int qk_cuda_abi_version(void);
/* nmc_qk_cuda.cu `qk_cuda_available` (qk_cuda.py:120): 0 iff usable. */
int qk_cuda_available(void);
/* nmc_qk_cuda.cu:720 `qk_linear_cuda` (qk_cuda.py:116-117, 230-244). */
int qk_linear_cuda(const uint8_t *W, const int64_t *x, long long T, long long out_f, long long n_blocks, int fw,
                   int qtype, int64_t *out);
/* nmc_qk_cuda.cu:1046 `qk_register_weight` (qk_cuda.py:252-270): handle >= 0 or -1. */
long long qk_register_weight(const uint8_t *W, long long out_f, long long n_blocks, int qtype);
/* nmc_qk_cuda.cu:1040 `qk_resident_reserve` (qk_cuda.py:928-937). */
int qk_resident_reserve(long long count);
/* nmc_qk_cuda.cu:1252 `qk_apply_resident` (qk_cuda.py:387-397). */
int qk_apply_resident(long long h, const int64_t *x, long long T, int fw, int64_t *out);
/* nmc_qk_cuda.cu:1284 `qk_apply_resident_grouped` (qk_cuda.py:405-442). */
int qk_apply_resident_grouped(const long long *handles, const int *phase_ids, int count, const int64_t *x,
                              long long rows, int fw, long long total, int64_t *out);
/* nmc_qk_cuda.cu:2003 / :1932 DP4A applies (qk_cuda.py:1029-1050). */
int qk_apply_resident_q4k_dp4a(long long h, const int64_t *x, long long T, int fw, int Ln, int64_t *out);
int qk_apply_resident_q6k_dp4a(long long h, const int64_t *x, long long T, int fw, int Ln, int64_t *out);
/* nmc_qk_cuda.cu:2203-2254 `qk_moe_ffn_batched` (qk_cuda.py:1073-1101). */
int qk_moe_ffn_batched(const long long *gate_h, const long long *up_h, const long long *down_h, int m, int k,
                       const int64_t *h, const int64_t *gates, long long d_model, long long e_ffn, int fa, int fw,
                       int64_t *out);
/* nmc_qk_cuda.cu:2261 `qk_moe_ffn_batched_dp4a` (qk_cuda.py:1094-1098). */
int qk_moe_ffn_batched_dp4a(const long long *gate_h, const long long *up_h, const long long *down_h, int m, int k,
                            const int64_t *h, const int64_t *gates, long long d_model, long long e_ffn, int fa, int fw,
                            int64_t *out);
/* nmc_qk_cuda.cu:1816 `qk_moe_ffn` / :2110 `qk_moe_ffn_dp4a` (qk_cuda.py:1104-1124). */
int qk_moe_ffn(const long long *gate_h, const long long *up_h, const long long *down_h, int n_e, const int64_t *h,
               const int64_t *gates, long long d_model, long long e_ffn, int fa, int fw, int64_t *out);
int qk_moe_ffn_dp4a(const long long *gate_h, const long long *up_h, const long long *down_h, int n_e,
                    const int64_t *h, const int64_t *gates, long long d_model, long long e_ffn, int fa, int fw,
                    int64_t *out);
/* device-pointer batched MoE and its status word (bit 2: int64 envelope miss). */
int imie_moe_ffn_batched_dev(const long long *gate_h, const long long *up_h, const long long *down_h, int m, int k,
                             const int64_t *h_dev, const int64_t *gates_dev, long long d_model, long long e_ffn,
                             int fa, int fw, int64_t *out_dev, void *stream);
int imie_moe_status(int clear, void *stream);
/* fp16 -> round-half-even(h * 2^fw) as the Q4_K / Q6_K kernels compute it, over n host values (synchronous). No
 * reference counterpart: a test hook for the exhaustive check against the integer rule (nmc_qk_kernel.c:16-39). */
int imie_fp16_fixed_probe(const uint16_t *h, int64_t n, int fw, int64_t *out);
/* registry / workspace / profiling (nmc_qk_cuda.cu:82-90, 1783-1815; qk_cuda.py:870-965). */
void qk_free_all(void);
long long qk_resident_count(void);
long long qk_resident_capacity(void);
long long qk_moe_workspace_allocations(void);
unsigned long long qk_moe_workspace_bytes(void);
void qk_moe_workspace_release(void);
void qk_profile_reset(void);
void qk_profile_set_enabled(int enabled);
int qk_profile_snapshot(unsigned long long *out, int capacity);

/* ---- resident preprocessing and attention bank (the steps either side of the MoE block) ------------------ */
/* nmc_qk_cuda.cu:1068 `qk_register_i64` (qk_cuda.py:285-303): dense int64 [rows, cols] (gains, router). */
long long qk_register_i64(const int64_t *W, long long rows, long long cols);
/* nmc_qk_cuda.cu:1116 `qk_rmsnorm_router` (qk_cuda.py:331-372): RMSNorm + router + lowest-index top-k + sigmoid
 * gates; rc 3 = exact envelope rejection. */
int qk_rmsnorm_router(long long gain_h, long long router_h, const int64_t *x, long long rows, int fa, int fw,
                      unsigned long long eps, int used, long long h_capacity, long long route_capacity,
                      int64_t *h_out, int *ids_out, int64_t *gates_out);
/* nmc_qk_cuda.cu:877-933, :1363-1780 attention bank (qk_cuda.py:476-715 `ResidentAttentionCache`). */
long long qk_attention_bank_create(int n_layers, long long max_length, long long d_model, int heads, int n_kv,
                                   int head_dim, int fa, const int64_t *cos, const int64_t *sin);
int qk_attention_bank_import(long long h, int layer, const int64_t *k, const int64_t *v, long long length);
int qk_attention_bank_apply(long long h, int layer, long long qh, long long kh, long long vh, long long oh,
                            const int64_t *x, int fw, int window, int rope, int64_t inv_sqrt,
                            long long output_capacity, int64_t *out);
int qk_attention_bank_moe_configure(long long h, int layer, int experts, int used, long long d_model,
                                    long long expert_ffn);
int qk_attention_bank_moe_bind(long long h, int layer, int expert, long long gate_h, long long up_h,
                               long long down_h);
int qk_attention_bank_moe_begin(long long h, int layer, long long gain_h, long long router_h, long long qh,
                                long long kh, long long vh, long long oh, const int64_t *x, int use_retained, int fw,
                                unsigned long long eps, int window, int rope, int64_t inv_sqrt, int cold_capacity,
                                int *cold_count_out, int *cold_ids_out);
int qk_attention_bank_moe_continue(long long h, int layer, int fw, int publish, long long output_capacity,
                                   int64_t *out);
int qk_attention_bank_moe_export(long long h, long long output_capacity, int64_t *out);
unsigned long long qk_attention_bank_workspace_bytes(long long h);
int qk_attention_bank_reset(long long h);
void qk_attention_bank_destroy(long long h);

#ifdef __cplusplus
}
#endif
#endif
