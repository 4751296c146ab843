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

// FP8-E4M3 codes in the reference's convention
// (crates/model/src/components/kv_cache_fp8.rs:188-212) to bf16.
//
// fp8x8_to_bf16 converts eight codes (little-endian bytes of lo, hi) with
// the hardware's unscaled conversion, which reads OCP E4M3.  That agrees
// with the reference's decode on every code except those with exponent
// field 0 and a nonzero byte (0x80 is NaN there, 0x01-0x07 / 0x81-0x87 read
// 2^-7 (1 + m/8), not OCP subnormals) and those with exponent field 15
// (0x7C / 0xFC are +-inf there, 0x7F / 0xFF read +-480, not NaN; the rest
// agree).  Kernels OR fp8_exotic_bits over the words they convert and take
// fp8x8_to_bf16_exact, the reference's decode, when bit 7 of any byte is set.
__device__ inline bf16x8 fp8x8_to_bf16(uint32_t lo, uint32_t hi) {
  const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
  const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
  const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
  const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
  return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// Bit 7 of each byte of the result is set where the hardware conversion
// differs (or may differ) from the reference: exponent field 15, or
// exponent field 0 with a nonzero byte.  The other bits are garbage, so
// callers OR the results and test them against 0x80808080.  Per byte, with
// y = b & 0x7F: y + 0x08 reaches bit 7 iff y >= 0x78 (exponent 15);
// y + 0x78 iff y >= 8 (exponent above 0); y + 0x7F iff y >= 1.  No sum
// carries into the next byte.
__host__ __device__ inline uint32_t fp8_exotic_bits(uint32_t w) {
  const uint32_t y = w & 0x7F7F7F7Fu;
  const uint32_t e15 = y + 0x08080808u;
  const uint32_t e_pos = y + 0x78787878u;
  const uint32_t y_pos = y + 0x7F7F7F7Fu;
  return e15 | (~e_pos & (y_pos | w));
}

// Two codes held in the low bytes of the 16-bit halves of x (bits 8-15 and
// 24-31 zero) to two bf16s with the reference's decode, integer arithmetic
// only: sign and (e, m) move into place with the exponent rebiased by
// 127 - 7 = 120 (every such value is a bf16 value); (e, m) = 0 gives a
// signed zero, except 0x80 which is NaN; 0x7C / 0xFC are +-inf.
__host__ __device__ inline uint32_t fp8x2_ref_bf16x2(uint32_t x) {
  const uint32_t lane1 = 0x00010001u;
  const uint32_t m = x & 0x007F007Fu;
  const uint32_t sgn = (x & 0x00800080u) << 8;
  const uint32_t nz = ((m + 0x007F007Fu) >> 7) & lane1;               // m != 0
  const uint32_t inf = (~((m ^ 0x007C007Cu) + 0x007F007Fu) >> 7) & lane1;  // m == 0x7C
  const uint32_t nan = ~nz & (x >> 7) & lane1;                         // x == 0x80
  uint32_t v = (((m << 4) + 0x3C003C00u) & (nz * 0xFFFFu)) | sgn;
  v = (v & ~(inf * 0xFFFFu)) | ((sgn | 0x7F807F80u) & (inf * 0xFFFFu));
  v = (v & ~(nan * 0xFFFFu)) | (0x7FC07FC0u & (nan * 0xFFFFu));
  return v;
}

__device__ inline bf16x8 fp8x8_to_bf16_exact(uint32_t lo, uint32_t hi) {
  typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4_t;
  const u32x4_t r = {fp8x2_ref_bf16x2(__builtin_amdgcn_perm(0u, lo, 0x0C010C00u)),
                     fp8x2_ref_bf16x2(__builtin_amdgcn_perm(0u, lo, 0x0C030C02u)),
                     fp8x2_ref_bf16x2(__builtin_amdgcn_perm(0u, hi, 0x0C010C00u)),
                     fp8x2_ref_bf16x2(__builtin_amdgcn_perm(0u, hi, 0x0C030C02u))};
  return __builtin_bit_cast(bf16x8, r);
}

// Block content hash of the reference (layout.rs:51-58):
//   fold(0, |acc, x| acc * 31 + (|x| * 1000) as u64)  (wrapping u64)
// over the block's K values in [head][token][dim] order, i.e.
//   sum_i term(x_i) * 31^(n-1-i) mod 2^64.  term: Rust's saturating float ->
// u64 cast (NaN and +0 -> 0, >= 2^64 -> u64::MAX).
__host__ __device__ inline uint64_t hash_term(float x) {
  const float y = fabsf(x) * 1000.0f;
  if (!(y > 0.0f)) return 0;  // NaN, +0
  if (y >= 18446744073709551616.0f) return ~0ull;
  return (uint64_t)y;
}
__host__ __device__ inline uint64_t pow_u64(uint64_t b, uint64_t e) {
  uint64_t r = 1;
  while (e) {
    if (e & 1) r *= b;
    b *= b;
    e >>= 1;
  }
  return r;
}
// The hash of n values val(0) .. val(n-1) by a workgroup of 256 threads:
// thread t sums term(val(e)) * 31^(n-1-e) over e = t, t + 256, ...; the
// partial sums are added through `red` (256 entries).  Every thread returns
// the hash; ends with a barrier (red may be reused).
template <typename F>
__device__ inline uint64_t workgroup_block_hash(int n, F val, uint64_t* red) {
  const int t = threadIdx.x;
  uint64_t acc = 0;
  if (t < n) {
    const int last = (n - 1 - t) / 256;  // this thread's last element t + 256 last
    uint64_t p = pow_u64(31u, (uint64_t)(n - 1 - (t + 256 * last)));
    const uint64_t step = pow_u64(31u, 256u);
    for (int k = last; k >= 0; --k) {
      acc += hash_term(val(t + 256 * k)) * p;
      p *= step;
    }
  }
  red[t] = acc;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (t < s) red[t] += red[t + s];
    __syncthreads();
  }
  const uint64_t h = red[0];
  __syncthreads();
  return h;
}

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

// FP8 E4M3 in the reference's convention
// (crates/model/src/components/kv_cache_fp8.rs:143-212): bias 7, normals
// only, NaN -> 0x80, +-inf -> 0x7C / 0xFC, |v| < 2^-6 -> +0, the significand
// rounded to 3 bits half-up, a biased exponent above 14 (before or after
// rounding) saturating to 0x7B / 0xFB (+-352).  Integer arithmetic only, so
// host and device agree bit for bit.
__host__ __device__ inline uint8_t fp8_encode(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const uint32_t sign = u >> 31, a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return 0x80;
  if (a == 0x7f800000u) return sign ? 0xFC : 0x7C;
  int be = (int)(a >> 23) - 127 + 7;  // f32 subnormals land far below 1
  if (a == 0 || be <= 0) return 0;
  const uint8_t sat = sign ? 0xFB : 0x7B;
  if (be > 14) return sat;
  // floor(f * 8 + 0.5) - 8 for the significand f = 1 + mant / 2^23
  uint32_t r = ((a & 0x7fffffu) + (1u << 19)) >> 20;
  if (r >= 8) {
    ++be;
    r = 0;
  }
  if (be > 14) return sat;
  return (uint8_t)((sign << 7) | ((uint32_t)be << 3) | r);
}
// The f32 value of the reference's f16 decode: 0x80 -> NaN, 0x7C / 0xFC ->
// +-inf, exponent and mantissa 0 -> +-0, else (-1)^s 2^(e-7) (1 + m/8).
__host__ __device__ inline float fp8_decode(uint32_t b) {
  if (b == 0x80) return __builtin_nanf("");
  if (b == 0x7C) return __builtin_inff();
  if (b == 0xFC) return -__builtin_inff();
  const uint32_t sign = (b >> 7) & 1, e = (b >> 3) & 15, m = b & 7;
  if (e == 0 && m == 0) return __builtin_bit_cast(float, sign << 31);
  return __builtin_bit_cast(float, (sign << 31) | ((e + 120) << 23) | (m << 20));
}
// FP8 cache element (one byte).
struct Fp8 {
  uint8_t bits;
};
template <>
struct Elem<Fp8> {
  __device__ static inline float load(const Fp8* p) { return fp8_decode(p->bits); }
  __device__ static inline void store(Fp8* p, float x) { p->bits = fp8_encode(x); }
};

// Thread-local last-error message behind pa_last_error().
void set_error(const char* fmt, ...);
void clear_error();

inline size_t dtype_size(int32_t dtype) {
  return dtype == PA_DTYPE_BF16 ? 2 : dtype == PA_DTYPE_FP8_E4M3 ? 1 : 4;
}
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
