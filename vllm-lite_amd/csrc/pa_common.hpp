// Shared helpers for the paged-attention kernels and their C entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/pa.h"

namespace pa {

constexpr int kBlock = PA_BLOCK_SIZE;  // tokens per cache block

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

// bf16 <-> f32 on raw 16-bit patterns (round to nearest even, NaN kept quiet).
__host__ __device__ inline float bf16_bits_to_f32(uint16_t h) {
  return __builtin_bit_cast(float, (uint32_t)h << 16);
}
__host__ __device__ inline uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Element access for the two storage types.
template <typename T>
struct Elem;
template <>
struct Elem<float> {
  __device__ static inline float load(const float* p) { return *p; }
  __device__ static inline void store(float* p, float x) { *p = x; }
};
template <>
struct Elem<uint16_t> {
  __device__ static inline float load(const uint16_t* p) { return bf16_bits_to_f32(*p); }
  __device__ static inline void store(uint16_t* p, float x) { *p = f32_to_bf16_bits(x); }
};

// Thread-local last-error message behind pa_last_error().
void set_error(const char* fmt, ...);
void clear_error();

inline size_t dtype_size(int32_t dtype) { return dtype == PA_DTYPE_BF16 ? 2 : 4; }
inline bool dtype_ok(int32_t dtype) { return dtype == PA_DTYPE_F32 || dtype == PA_DTYPE_BF16; }

// Checks the launch that was just enqueued.
inline int32_t check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return PA_ERR_HIP;
  }
  return PA_OK;
}

}  // namespace pa

#define PA_REQUIRE(cond, code, ...) \
  do {                              \
    if (!(cond)) {                  \
      ::pa::set_error(__VA_ARGS__); \
      return (code);                \
    }                               \
  } while (0)
