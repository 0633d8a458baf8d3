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
int imie_abi_version(void);
const char *imie_last_error(void);
void *imie_default_stream(void);
int imie_synchronize(void);
/* per-kernel HIP-event timing on the stream each kernel runs on (kernel ids: 0 q1 prep, 1 q1 matvec,
 * 2 q1 GEMM, 3 attention, 4 Q4_K/Q6_K linear); read synchronizes. */
void imie_profile_begin(void);
int imie_profile_read(int kernel, double *total_ms, int64_t *count);
void imie_profile_end(void);
/* one int8 MFMA over per-lane operands (A, B: 64x16 int8, D: 64x4 int32); pins the lane mapping in tests. */
int imie_probe_mfma(const int8_t *a, const int8_t *b, int32_t *d);

/* ---- packed Q1_0 linear: out[t,o] = sum_b ((sum_i sign*x) * scale[o,b]) >> frac, mod 2^64 ----------- */
/* bonsai_q1_gpu.cu:2200-2241 `bonsai_q1_linear_gpu` (bound at gpu_native.py:44-52, called :212-217). */
int bonsai_q1_linear_gpu(const int64_t *x, const uint8_t *bits, const int64_t *scale, int64_t tokens,
                         int64_t out_features, int64_t n_blocks, int64_t frac, int64_t *out);
/* bonsai_q1_gpu.cu `bonsai_q1_register_weight` (gpu_native.py:73-74, 270-306): handle >= 0 or -1. */
int64_t bonsai_q1_register_weight(const uint8_t *bits, const int64_t *scale, int64_t out_features, int64_t n_blocks);
/* bonsai_q1_gpu.cu `bonsai_q1_register_weight_i32` (gpu_native.py:79-87). */
int64_t bonsai_q1_register_weight_i32(const uint8_t *bits, const int32_t *scale, int64_t out_features,
                                      int64_t n_blocks);
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
int imie_q1_weight_info(int64_t handle, int64_t *out_features, int64_t *n_blocks, int64_t *scale_bytes);
/* exact thread-per-output kernel over natural-layout device buffers (cross-check path). */
int imie_q1_linear_simple_dev(const int64_t *x_dev, const uint8_t *bits_dev, const int64_t *scale_dev,
                              int64_t tokens, int64_t out_features, int64_t n_blocks, int64_t frac,
                              int64_t *out_dev, void *stream);

#ifdef __cplusplus
}
#endif
#endif
