// Internal helpers shared by the libsnnk HIP sources (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "snnk.h"

#define SNNK_VERSION 100  // 0.1.0

namespace snnk {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// Status of the most recent launch on this thread, folded into the ABI code.
inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? SNNK_OK : static_cast<int>(e);
}

inline bool aligned(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

// Unsigned 32-bit division by a run-time invariant divisor d >= 1
// (round-up multiplier method, Granlund & Montgomery 1994):
//   s = ceil(log2 d),  m = floor(2^32 (2^s - d) / d) + 1,
//   n / d = (mulhi(n, m) + n) >> s       (sum taken in 64 bits).
struct FastDiv {
  uint32_t d, m, s;
};

inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d;
  uint32_t s = 0;
  while ((uint64_t(1) << s) < d) ++s;
  f.s = s;
  f.m = static_cast<uint32_t>(((uint64_t(1) << 32) * ((uint64_t(1) << s) - d)) / d + 1);
  return f;
}

__host__ __device__ __forceinline__ uint32_t fdiv(uint32_t n, FastDiv f) {
  uint32_t hi = static_cast<uint32_t>((static_cast<uint64_t>(n) * f.m) >> 32);
  return static_cast<uint32_t>((static_cast<uint64_t>(hi) + n) >> f.s);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

}  // namespace snnk
