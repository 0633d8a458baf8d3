// Process-global runtime: device probe, default stream, error notes, workspace buffers, memory info.
#include "imie_common.h"
#include <vector>
#include <stdio.h>
#include <string.h>

static hipStream_t g_stream = nullptr;
static int g_ready = -1;
static char g_last_error[256];
static int g_last_error_code = 0;

std::recursive_mutex& imie_lock() {
  static std::recursive_mutex m;
  return m;
}

void imie_note_error(hipError_t e, const char* what) {
  g_last_error_code = (int)e;
  snprintf(g_last_error, sizeof(g_last_error), "%s: %s", what, hipGetErrorString(e));
}

void imie_note_message(const char* msg) {
  g_last_error_code = 0;
  snprintf(g_last_error, sizeof(g_last_error), "%s", msg);
}

int imie_device_ready() {
  if (g_ready >= 0) return g_ready == 1 ? 0 : 1;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) { g_ready = 0; return 1; }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, 0) != hipSuccess) { g_ready = 0; return 1; }
  // The kernels are built for gfx950 only; refuse any other architecture loudly (rc != 0).
  g_ready = (strncmp(prop.gcnArchName, "gfx950", 6) == 0) ? 1 : 0;
  if (!g_ready) snprintf(g_last_error, sizeof(g_last_error), "device %s is not gfx950", prop.gcnArchName);
  return g_ready == 1 ? 0 : 1;
}

hipStream_t imie_stream() {
  if (!g_stream) {
    if (hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking) != hipSuccess) g_stream = nullptr;
  }
  return g_stream;
}

static uint64_t g_alloc_gen = 1;

void imie_free(void* p) {
  if (!p) return;
  (void)hipFree(p);
  ++g_alloc_gen;
}

uint64_t imie_alloc_gen() { return g_alloc_gen; }

int DevBuf::ensure(size_t bytes) {
  if (bytes <= cap && p) return 0;
  if (p) { imie_free(p); p = nullptr; cap = 0; }
  size_t want = bytes < 256 ? 256 : bytes;
  if (hipMalloc(&p, want) != hipSuccess) { p = nullptr; return 1; }
  cap = want;
  return 0;
}

void DevBuf::release() {
  if (p) imie_free(p);
  p = nullptr;
  cap = 0;
}

extern "C" {

// 0 iff a usable gfx950 device is present (bonsai_q1_gpu.cu `bonsai_gpu_available` contract).
int bonsai_gpu_available(void) {
  std::lock_guard<std::recursive_mutex> g(imie_lock());
  return imie_device_ready();
}

int imie_abi_version(void) { return 1; }

// bonsai_q1_gpu.cu:1970-1980 `bonsai_gpu_abi_version` / `bonsai_gpu_last_error_code` / `bonsai_gpu_last_error`:
// the generation of the bonsai_* entry points this library mirrors (3), and the last runtime error noted by any
// entry point (HIP error number and text; 0 / empty when none).
int bonsai_gpu_abi_version(void) { return 3; }

int bonsai_gpu_last_error_code(void) { return g_last_error_code; }

const char* bonsai_gpu_last_error(void) { return g_last_error; }

const char* imie_last_error(void) { return g_last_error; }

int bonsai_gpu_mem_info(uint64_t* free_b, uint64_t* total_b) {
  std::lock_guard<std::recursive_mutex> g(imie_lock());
  if (!free_b || !total_b || imie_device_ready() != 0) return IMIE_EARG;
  size_t f = 0, t = 0;
  IMIE_HIP(hipMemGetInfo(&f, &t));
  *free_b = f;
  *total_b = t;
  return IMIE_OK;
}

// Library stream as an opaque handle so a host runtime can order its own work around the library.
void* imie_default_stream(void) {
  std::lock_guard<std::recursive_mutex> g(imie_lock());
  return (void*)imie_stream();
}

int imie_synchronize(void) {
  std::lock_guard<std::recursive_mutex> g(imie_lock());
  IMIE_HIP(hipStreamSynchronize(imie_stream()));
  return IMIE_OK;
}

}  // extern "C"

// One v_mfma_i32_16x16x64_i8 over caller-provided per-lane operands (A, B: 64 lanes x 16 int8; D: 64 lanes x 4
// int32). Lets the tests pin the operand / accumulator lane mapping the Q1 kernels rely on.
__global__ void imie_probe_mfma_kernel(const v4i* a, const v4i* b, v4i* d) {
  const int l = threadIdx.x;
  v4i acc = {0, 0, 0, 0};
  d[l] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[l], b[l], acc, 0, 0, 0);
}

extern "C" int imie_probe_mfma(const int8_t* a_host, const int8_t* b_host, int32_t* d_host) {
  std::lock_guard<std::recursive_mutex> g(imie_lock());
  if (!a_host || !b_host || !d_host || imie_device_ready() != 0) return IMIE_EARG;
  void *a = nullptr, *b = nullptr, *d = nullptr;
  IMIE_HIP(hipMalloc(&a, 1024));
  IMIE_HIP(hipMalloc(&b, 1024));
  IMIE_HIP(hipMalloc(&d, 1024));
  IMIE_HIP(hipMemcpy(a, a_host, 1024, hipMemcpyHostToDevice));
  IMIE_HIP(hipMemcpy(b, b_host, 1024, hipMemcpyHostToDevice));
  hipLaunchKernelGGL(imie_probe_mfma_kernel, dim3(1), dim3(64), 0, 0, (const v4i*)a, (const v4i*)b, (v4i*)d);
  IMIE_HIP(hipGetLastError());
  IMIE_HIP(hipMemcpy(d_host, d, 1024, hipMemcpyDeviceToHost));
  imie_free(a); imie_free(b); imie_free(d);
  return IMIE_OK;
}

// Sustained int8 MFMA throughput of this device: every SIMD runs waves of 8 independent
// v_mfma_i32_16x16x64_i8 accumulator chains (no memory traffic in the loop), timed with HIP events. The bench
// quotes the prefill GEMM's MFMA utilisation against this as well as against the published dense peak.
__global__ __launch_bounds__(256) void imie_mfma_peak_kernel(int iters, int seed, int32_t* sink) {
  const v4i a = {seed, seed + 1, seed + 2, (int)threadIdx.x}, b = {seed + 3, seed, (int)threadIdx.x, 7};
  v4i c[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) c[i] = v4i{i, 0, 0, 0};
  for (int it = 0; it < iters; ++it)
#pragma unroll
    for (int i = 0; i < 8; ++i) c[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c[i], 0, 0, 0);
  int32_t v = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) v ^= c[i][0] ^ c[i][3];
  if (v == 0x7F3A5C11) sink[threadIdx.x] = v;        // keeps the chains live; practically never taken
}

extern "C" int imie_mfma_peak(double* ops_per_s) {
  std::lock_guard<std::recursive_mutex> g(imie_lock());
  if (!ops_per_s || imie_device_ready() != 0) return IMIE_EARG;
  int dev = 0, cus = 0;
  IMIE_HIP(hipGetDevice(&dev));
  IMIE_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  void* sink = nullptr;
  IMIE_HIP(hipMalloc(&sink, 1024));
  hipEvent_t e0, e1;
  IMIE_HIP(hipEventCreate(&e0));
  IMIE_HIP(hipEventCreate(&e1));
  const int wgs = cus * 4, iters = 2000;               // 4 workgroups of 4 waves per CU: 4 waves per SIMD
  float ms = 0.f;
  for (int rep = 0; rep < 2; ++rep) {                 // the first launch warms up clocks and code
    IMIE_HIP(hipEventRecord(e0, 0));
    hipLaunchKernelGGL(imie_mfma_peak_kernel, dim3((unsigned)wgs), dim3(256), 0, 0, iters, 1, (int32_t*)sink);
    IMIE_HIP(hipEventRecord(e1, 0));
    IMIE_HIP(hipEventSynchronize(e1));
    IMIE_HIP(hipEventElapsedTime(&ms, e0, e1));
  }
  (void)hipEventDestroy(e0); (void)hipEventDestroy(e1); imie_free(sink);
  const double mfmas = (double)wgs * 4 * iters * 8;   // waves x iterations x chains
  *ops_per_s = mfmas * (2.0 * 16 * 16 * 64) / (ms * 1e-3);
  return IMIE_OK;
}

// Sustained HBM read bandwidth of this device: a streaming kernel over `bytes` of device memory (16 CU-filling
// workgroups per CU, four independent 16-byte nontemporal loads per thread per iteration, XOR-reduced), timed with
// HIP events, best of three launches after a warm-up. The bench quotes the Q1 matvec against it as well as against
// the published 8 TB/s.
__global__ __launch_bounds__(256) void imie_read_peak_kernel(const v4i* __restrict__ p, size_t n, int32_t* sink) {
  size_t i = (size_t)blockIdx.x * 1024 + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * 1024;
  v4i acc = {0, 0, 0, 0};
  for (; i + 768 < n; i += stride) {
    v4i v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = __builtin_nontemporal_load(p + i + 256 * u);
#pragma unroll
    for (int u = 0; u < 4; ++u) acc ^= v[u];
  }
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x7F3A5C11) sink[threadIdx.x] = 1;   // keeps the loads live
}

extern "C" int imie_hbm_read_peak(int64_t bytes, double* bytes_per_s) {
  std::lock_guard<std::recursive_mutex> g(imie_lock());
  if (!bytes_per_s || bytes < (1 << 24) || imie_device_ready() != 0) return IMIE_EARG;
  int dev = 0, cus = 0;
  IMIE_HIP(hipGetDevice(&dev));
  IMIE_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  const size_t n = (size_t)bytes / 16;
  void *buf = nullptr, *sink = nullptr;
  IMIE_HIP(hipMalloc(&buf, n * 16));
  if (hipMalloc(&sink, 1024) != hipSuccess) { imie_free(buf); return IMIE_EARG; }
  IMIE_HIP(hipMemset(buf, 0x5A, n * 16));
  hipEvent_t e0, e1;
  IMIE_HIP(hipEventCreate(&e0));
  IMIE_HIP(hipEventCreate(&e1));
  float best = 0.f;
  for (int rep = 0; rep < 4; ++rep) {                 // the first launch warms up clocks and code
    float ms = 0.f;
    IMIE_HIP(hipEventRecord(e0, 0));
    hipLaunchKernelGGL(imie_read_peak_kernel, dim3((unsigned)(cus * 16)), dim3(256), 0, 0, (const v4i*)buf, n,
                       (int32_t*)sink);
    IMIE_HIP(hipEventRecord(e1, 0));
    IMIE_HIP(hipEventSynchronize(e1));
    IMIE_HIP(hipEventElapsedTime(&ms, e0, e1));
    if (rep > 0 && (best == 0.f || ms < best)) best = ms;
  }
  (void)hipEventDestroy(e0); (void)hipEventDestroy(e1); imie_free(buf); imie_free(sink);
  *bytes_per_s = (double)(n * 16) / (best * 1e-3);
  return IMIE_OK;
}

// ---- per-kernel event profiler ---------------------------------------------------------------------------
namespace {
struct ProfSlot {
  std::vector<hipEvent_t> ev;   // begin/end pairs
  size_t used = 0;
};
bool g_prof = false;
bool g_prof_suspended = false;     // set while a launch sequence is being captured into a graph
ProfSlot g_slots[IMIE_K_COUNT];
}  // namespace

bool imie_prof_on() { return g_prof; }
bool imie_prof_suspend(bool off) {   // returns the previous state; no events are recorded while suspended
  const bool prev = g_prof_suspended;
  g_prof_suspended = off;
  return prev;
}

void imie_prof_mark(int kernel, hipStream_t st, bool begin) {
  if (!g_prof || g_prof_suspended || kernel < 0 || kernel >= IMIE_K_COUNT) return;
  ProfSlot& s = g_slots[kernel];
  if (begin && s.used + 2 > s.ev.size()) {
    hipEvent_t a, b;
    if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) return;
    s.ev.push_back(a);
    s.ev.push_back(b);
  }
  if (begin) {
    (void)hipEventRecord(s.ev[s.used], st);
  } else {
    (void)hipEventRecord(s.ev[s.used + 1], st);
    s.used += 2;
  }
}

extern "C" {

void imie_profile_begin(void) {
  std::lock_guard<std::recursive_mutex> g(imie_lock());
  g_prof = true;
  for (auto& s : g_slots) s.used = 0;
}

// Total milliseconds and launch count recorded for `kernel` since imie_profile_begin (synchronizes).
int imie_profile_read(int kernel, double* total_ms, int64_t* count) {
  std::lock_guard<std::recursive_mutex> g(imie_lock());
  if (kernel < 0 || kernel >= IMIE_K_COUNT || !total_ms || !count) return IMIE_EARG;
  ProfSlot& s = g_slots[kernel];
  double tot = 0;
  for (size_t i = 0; i < s.used; i += 2) {
    IMIE_HIP(hipEventSynchronize(s.ev[i + 1]));
    float ms = 0;
    IMIE_HIP(hipEventElapsedTime(&ms, s.ev[i], s.ev[i + 1]));
    tot += ms;
  }
  *total_ms = tot;
  *count = (int64_t)(s.used / 2);
  return IMIE_OK;
}

void imie_profile_end(void) {
  std::lock_guard<std::recursive_mutex> g(imie_lock());
  g_prof = false;
}

}  // extern "C"

// Failure-atomic device reservations (gpu_native.py:334-361 / bonsai_q1_gpu.cu:2160-2197): a memory-feasibility
// probe that takes several exact allocations at once; a failed reservation frees what it took and returns -1.
namespace {
std::vector<std::vector<void*>>& reservations() {
  static std::vector<std::vector<void*>> r;
  return r;
}
}  // namespace

extern "C" int64_t bonsai_gpu_reservation_create(const uint64_t* sizes, int64_t count, uint64_t* allocated) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (!sizes || count <= 0 || !allocated || imie_device_ready() != 0) return -1;
  std::vector<void*> taken;
  uint64_t total = 0;
  for (int64_t i = 0; i < count; ++i) {
    void* p = nullptr;
    if (sizes[i] == 0 || hipMalloc(&p, (size_t)sizes[i]) != hipSuccess) {
      (void)hipGetLastError();
      for (void* q : taken) imie_free(q);
      return -1;
    }
    taken.push_back(p);
    total += sizes[i];
  }
  reservations().push_back(std::move(taken));
  *allocated = total;
  return (int64_t)reservations().size() - 1;
}

extern "C" void bonsai_gpu_reservation_free(int64_t handle) {
  std::lock_guard<std::recursive_mutex> lk(imie_lock());
  if (handle < 0 || handle >= (int64_t)reservations().size()) return;
  for (void* p : reservations()[(size_t)handle]) imie_free(p);
  reservations()[(size_t)handle].clear();            // a second free is a no-op
}
