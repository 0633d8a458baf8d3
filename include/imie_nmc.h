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

#ifdef __cplusplus
}
#endif
#endif
