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
void imie_note_message(const char* msg);        // a refusal's reason for imie_last_error (no HIP error)
hipStream_t imie_stream();                 // the library's default stream (created on first use)
std::recursive_mutex& imie_lock();         // the library is single-caller; ABI entry points take this lock
int imie_device_ready();                   // 0 when a gfx9xx device is usable

// Every device free in the library goes through imie_free, which advances a process-wide allocation generation.
// A captured HIP graph records raw device addresses; its owner compares the generation it was captured under with
// the current one and re-captures when any block may have been freed (and its address handed out again).
void imie_free(void* p);
uint64_t imie_alloc_gen();

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

__host__ __device__ __forceinline__ uint64_t imie_absu64(int64_t v) {
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
// Whole-wave reductions over DPP lane moves (VALU only, no LDS crossbar): xor 1 and xor 2 (quad_perm), the
// half-row and row mirrors reduce each 16-lane row, row_bcast15 / row_bcast31 fold the four rows into lane
// 63, which readlane broadcasts as a wave-uniform value. Every lane of the wave must be active, and 0 must be
// the identity of the operation for the values reduced (sums, unsigned maxima, signed maxima / minima of sets
// that contain 0): lanes outside a row-masked step contribute 0.
// ---------------------------------------------------------------------------------------------------------
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ uint64_t imie_dpp64(uint64_t v) {
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, ROWS, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, ROWS, 0xF, false);
  return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}

__device__ __forceinline__ uint64_t imie_readlane_u64(uint64_t v, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), lane);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t imie_readlane63(uint64_t v) { return imie_readlane_u64(v, 63); }

template <typename Op>
__device__ __forceinline__ uint64_t imie_wave_reduce_full(uint64_t v, Op op) {
  v = op(v, imie_dpp64<0xB1>(v));        // quad_perm [1,0,3,2]
  v = op(v, imie_dpp64<0x4E>(v));        // quad_perm [2,3,0,1]
  v = op(v, imie_dpp64<0x141>(v));       // row_half_mirror
  v = op(v, imie_dpp64<0x140>(v));       // row_mirror: every lane holds its row's result
  v = op(v, imie_dpp64<0x142, 0xA>(v));  // row_bcast15 into rows 1 and 3
  v = op(v, imie_dpp64<0x143, 0xC>(v));  // row_bcast31 into rows 2 and 3: lane 63 holds the wave's result
  return imie_readlane63(v);
}

// sum over each 16-lane row (every lane of the row receives it); every lane of the wave must be active
__device__ __forceinline__ uint64_t imie_row_sum_u64_full(uint64_t v) {
  v += imie_dpp64<0xB1>(v);
  v += imie_dpp64<0x4E>(v);
  v += imie_dpp64<0x141>(v);
  v += imie_dpp64<0x140>(v);
  return v;
}

__device__ __forceinline__ uint64_t imie_wave_max_u64_full(uint64_t v) {
  return imie_wave_reduce_full(v, [](uint64_t a, uint64_t b) { return a > b ? a : b; });
}
__device__ __forceinline__ uint64_t imie_wave_sum_u64_full(uint64_t v) {
  return imie_wave_reduce_full(v, [](uint64_t a, uint64_t b) { return a + b; });
}
// signed maximum / minimum of sets that contain 0
__device__ __forceinline__ int64_t imie_wave_max0_i64_full(int64_t v) {
  return (int64_t)imie_wave_reduce_full((uint64_t)v, [](uint64_t a, uint64_t b) {
    return (int64_t)a > (int64_t)b ? a : b; });
}
__device__ __forceinline__ int64_t imie_wave_min0_i64_full(int64_t v) {
  return (int64_t)imie_wave_reduce_full((uint64_t)v, [](uint64_t a, uint64_t b) {
    return (int64_t)a < (int64_t)b ? a : b; });
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
