// imie — integer inference engine producer for MI355X (gfx950 / CDNA4).
// Shared device helpers and the process-global runtime state behind the C-ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <mutex>
#include <vector>

// Return codes of the reference producers (bonsai/tools/bonsai_q1_gpu.cu, nmc_qk_cuda.cu):
// 0 ok, 1 bad args / runtime failure, 2 attention overflow (or DP4A envelope miss), 4 RMSNorm overflow.
enum { IMIE_OK = 0, IMIE_EARG = 1, IMIE_EOVF = 2, IMIE_ERMS = 4 };

#define IMIE_HIP(call)                                   \
  do {                                                   \
    hipError_t e_ = (call);                              \
    if (e_ != hipSuccess) { imie_note_error(e_, #call); return IMIE_EARG; } \
  } while (0)

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

void imie_note_error(hipError_t e, const char* what);
hipStream_t imie_stream();                 // the library's default stream (created on first use)
std::recursive_mutex& imie_lock();         // the library is single-caller; ABI entry points take this lock
int imie_device_ready();                   // 0 when a gfx9xx device is usable

// Grow-only device workspace owned by the library (host-pointer ABI staging buffers).
struct DevBuf {
  void* p = nullptr;
  size_t cap = 0;
  int ensure(size_t bytes);
  void release();
};

// ---------------------------------------------------------------------------------------------------------
// Device integer helpers (numpy int64 semantics: wrap mod 2^64, floor shifts).
// ---------------------------------------------------------------------------------------------------------
__device__ __forceinline__ int64_t imie_floor_shift(int64_t v, int s) {
  // numpy `v >> s` for 0 <= s; counts >= 63 give the sign (-1 / 0), which `>> 63` already does.
  return v >> (s > 63 ? 63 : s);
}

// quotient / remainder of non-negative values below 2^32 (32-bit hardware-friendly division)
__device__ __forceinline__ int64_t imie_udiv32(int64_t a, int64_t b) { return (int64_t)((uint32_t)a / (uint32_t)b); }
__device__ __forceinline__ int64_t imie_umod32(int64_t a, int64_t b) { return (int64_t)((uint32_t)a % (uint32_t)b); }

__device__ __forceinline__ uint64_t imie_absu64(int64_t v) {
  return v < 0 ? (uint64_t)0 - (uint64_t)v : (uint64_t)v;
}

// Largest |x| exactly representable by L balanced base-256 digits (each in [-128, 127]): 127*(256^L-1)/255.
__host__ __device__ __forceinline__ uint64_t imie_balanced_cap(int L) {
  uint64_t c = 0;
  for (int i = 0; i < L; ++i) c = c * 256u + 127u;
  return c;
}

__host__ __device__ __forceinline__ int imie_limbs_needed(uint64_t maxabs) {
  int L = 1;
  while (L < 8 && maxabs > imie_balanced_cap(L)) ++L;
  return L;
}

__device__ __forceinline__ uint64_t imie_wave_max_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    uint64_t w = __shfl_xor(v, o, 64);
    v = w > v ? w : v;
  }
  return v;
}

__device__ __forceinline__ int64_t imie_wave_sum_i64(int64_t v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = (int64_t)((uint64_t)v + (uint64_t)__shfl_xor(v, o, 64));
  return v;
}

// ---------------------------------------------------------------------------------------------------------
// Per-kernel HIP-event timing (enabled by imie_profile_begin; used by the benchmark to time the dominant
// kernel on the stream it runs on). Kernel ids below.
// ---------------------------------------------------------------------------------------------------------
enum { IMIE_K_Q1_PREP = 0, IMIE_K_Q1_GEMV = 1, IMIE_K_Q1_GEMM = 2, IMIE_K_ATTN = 3, IMIE_K_QK = 4,
       IMIE_K_COUNT = 16 };
bool imie_prof_on();
bool imie_prof_suspend(bool off);
void imie_prof_mark(int kernel, hipStream_t st, bool begin);
