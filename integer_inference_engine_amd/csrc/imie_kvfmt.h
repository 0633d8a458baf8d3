// "kv8x4" cache format: each cached K / V element is stored as 4 balanced base-256 digits (bytes in [-128, 127],
// value = d0 + 256 d1 + 65536 d2 + 2^24 d3), so the attention's dot products run as int8 MFMAs on the stored
// bytes directly. 4 bytes per element, like an int32 cache; representable values are |v| <= 2139062143
// (= 127 * (256^4 - 1) / 255), anything larger is refused (status bit 2) and needs the int64 cache.
//
// Per (page, kv head) block of P slots (P a multiple of 64, hd a multiple of 16), 4 * hd * P bytes:
//   K: [slot tile j / 16][digit b][dim group c / 16][slot j % 16][dim c % 16] -- the 16-byte pieces of one
//      (digit, dim group) for 16 consecutive slots are contiguous, so the 64 lanes of one MFMA operand load
//      (16 keys x 4 dim groups) read 1 KB contiguous
//   V: [digit b][dim c][slot j]   -- for one (digit, dim), the P slots are contiguous (keys on the MFMA K axis)
#pragma once
#include "imie_common.h"

namespace imie_kv8 {

constexpr int64_t kCap = 2139062143;

__host__ __device__ inline bool fits(int64_t v) { return v >= -kCap && v <= kCap; }

// balanced digits of v (|v| <= kCap), packed little-endian into a 32-bit word
__host__ __device__ inline uint32_t encode(int64_t v) {
  uint32_t w = 0;
  for (int b = 0; b < 4; ++b) {
    const int64_t d = ((v + 128) & 255) - 128;
    v = (v - d) >> 8;
    w |= (uint32_t)(d & 0xFF) << (8 * b);
  }
  return w;
}

__host__ __device__ inline int64_t digit(uint32_t w, int b) { return (int64_t)(int8_t)(uint8_t)(w >> (8 * b)); }

__host__ __device__ inline int64_t decode4(int8_t d0, int8_t d1, int8_t d2, int8_t d3) {
  return (int64_t)d0 + 256 * (int64_t)d1 + 65536 * (int64_t)d2 + 16777216 * (int64_t)d3;
}

__host__ __device__ inline int64_t block_base(int64_t pg, int64_t kv, int64_t Hkv, int64_t hd, int64_t P) {
  return (pg * Hkv + kv) * 4 * hd * P;
}
__host__ __device__ inline int64_t k_off(int64_t j, int b, int64_t c, int64_t hd) {
  return (((j >> 4) * 4 + b) * (hd >> 4) + (c >> 4)) * 256 + (j & 15) * 16 + (c & 15);
}
// offset of the 16-byte piece (digit b, dims c .. c + 15; c a multiple of 16) of slot j from k_off(j, 0, 0, hd)
__host__ __device__ inline int64_t k_piece(int b, int64_t c, int64_t hd) { return ((int64_t)b * hd + c) * 16; }
__host__ __device__ inline int64_t v_off(int64_t j, int b, int64_t c, int64_t hd, int64_t P) {
  return ((int64_t)b * hd + c) * P + j;
}

}  // namespace imie_kv8
