// Fused rotary position embedding + KV-cache write (pa_rope_reshape_and_cache)
// and the host inverse-frequency table (pa_rope_inv_freq).
//
// The reference applies RoPE to Q and K, then writes the expanded K/V into
// the cache token by token (crates/model/src/components/attention/
// rope_gqa.rs:283-302 -> paged_gqa.rs:29-63).  Here one kernel reads each
// token's Q, K and V once: Q is rotated in place, K is rotated on the way
// into the K cache, V is copied into the token-minor V cache.
#include <cmath>

#include "pa_common.hpp"

namespace pa {
namespace {

// One workgroup per token.  Thread i of a head handles the pair
// (x[i], x[i + D/2]); heads are strided over the workgroup.
template <typename T>
__global__ __launch_bounds__(256) void rope_cache_kernel(
    T* __restrict__ q, int64_t q_stride, const T* __restrict__ key, int64_t key_stride,
    const T* __restrict__ value, int64_t value_stride, T* __restrict__ k_cache,
    T* __restrict__ v_cache, const int64_t* __restrict__ slots,
    const int64_t* __restrict__ positions, const float* __restrict__ inv_freq, int Hq, int Hkv,
    int D, int64_t num_slots) {
  const int t = blockIdx.x;
  const int half = D / 2;
  const float pos = (float)positions[t];
  const int64_t slot = slots[t];
  const bool write = slot >= 0 && slot < num_slots;
  const int64_t blk = write ? slot / kBlock : 0;
  const int off = write ? (int)(slot % kBlock) : 0;
  // Q rotation, all query heads.
  for (int e = threadIdx.x; e < Hq * half; e += blockDim.x) {
    const int h = e / half, i = e % half;
    float s, c;
    sincosf(pos * inv_freq[i], &s, &c);
    T* row = q + t * q_stride + (int64_t)h * D;
    const float x1 = Elem<T>::load(row + i), x2 = Elem<T>::load(row + half + i);
    Elem<T>::store(row + i, x1 * c - x2 * s);
    Elem<T>::store(row + half + i, x2 * c + x1 * s);
  }
  if (!write) return;
  // K rotation into the cache, V copy into the token-minor V cache.
  for (int e = threadIdx.x; e < Hkv * half; e += blockDim.x) {
    const int h = e / half, i = e % half;
    float s, c;
    sincosf(pos * inv_freq[i], &s, &c);
    const T* krow = key + t * key_stride + (int64_t)h * D;
    const float x1 = Elem<T>::load(krow + i), x2 = Elem<T>::load(krow + half + i);
    T* kd = k_cache + ((blk * Hkv + h) * kBlock + off) * (int64_t)D;
    Elem<T>::store(kd + i, x1 * c - x2 * s);
    Elem<T>::store(kd + half + i, x2 * c + x1 * s);
    const T* vrow = value + t * value_stride + (int64_t)h * D;
    T* vd = v_cache + ((blk * Hkv + h) * (int64_t)D) * kBlock + off;
    vd[(int64_t)i * kBlock] = vrow[i];
    vd[(int64_t)(half + i) * kBlock] = vrow[half + i];
  }
}

}  // namespace
}  // namespace pa

using namespace pa;

extern "C" int32_t pa_rope_inv_freq(int32_t head_dim, float theta, int32_t rope_type,
                                    float factor, int32_t original_max_position,
                                    int32_t cur_seq_len, const float* short_factor,
                                    const float* long_factor, float* out) {
  clear_error();
  PA_REQUIRE(head_dim > 0 && head_dim % 2 == 0, PA_ERR_INVALID_ARG,
             "pa_rope_inv_freq: head_dim %d must be even and positive", head_dim);
  PA_REQUIRE(rope_type >= PA_ROPE_DEFAULT && rope_type <= PA_ROPE_SU, PA_ERR_INVALID_ARG,
             "pa_rope_inv_freq: unknown rope type %d", rope_type);
  PA_REQUIRE(out, PA_ERR_INVALID_ARG, "pa_rope_inv_freq: null output");
  const int half = head_dim / 2;
  const bool near_one = std::fabs(factor - 1.0f) < 1.1920929e-07f;  // f32 epsilon
  const float d = (float)head_dim;
  float th = theta;
  if (rope_type == PA_ROPE_YARN && !near_one) {
    th = theta * std::pow(factor, d / (d - 2.0f));
  } else if (rope_type == PA_ROPE_DYNAMIC && original_max_position > 0 &&
             cur_seq_len > original_max_position && !near_one) {
    const float scale =
        std::fma(factor, (float)cur_seq_len / (float)original_max_position, -(factor - 1.0f));
    th = theta * std::pow(scale, d / (d - 2.0f));
  }
  for (int i = 0; i < half; ++i) out[i] = std::pow(th, -2.0f * (float)i / d);
  if (rope_type == PA_ROPE_LINEAR && !near_one)
    for (int i = 0; i < half; ++i) out[i] = out[i] / factor;
  if (rope_type == PA_ROPE_SU && original_max_position > 0) {
    int boundary = half;
    for (int i = 0; i < half; ++i)
      if (2.0f * 3.14159265358979323846f / out[i] > (float)original_max_position) {
        boundary = i;
        break;
      }
    for (int i = 0; i < half; ++i) {
      const float* f = i < boundary ? short_factor : long_factor;
      out[i] = out[i] / (f ? f[i] : 1.0f);
    }
  }
  return PA_OK;
}

extern "C" int32_t pa_rope_reshape_and_cache(void* q, int64_t q_stride, const void* key,
                                             int64_t key_stride, const void* value,
                                             int64_t value_stride, void* k_cache, void* v_cache,
                                             const int64_t* slot_mapping, const int64_t* positions,
                                             const float* inv_freq, int32_t num_tokens,
                                             int32_t num_heads, int32_t num_kv_heads,
                                             int32_t head_dim, int32_t num_blocks, int32_t dtype,
                                             pa_stream_t stream) {
  clear_error();
  PA_REQUIRE(dtype_ok(dtype), PA_ERR_INVALID_ARG, "pa_rope_reshape_and_cache: unknown dtype %d",
             dtype);
  PA_REQUIRE(num_tokens >= 0 && num_heads > 0 && num_kv_heads > 0 && head_dim > 0 &&
                 head_dim % 2 == 0 && num_blocks > 0,
             PA_ERR_INVALID_ARG, "pa_rope_reshape_and_cache: bad sizes");
  if (num_tokens == 0) return PA_OK;
  PA_REQUIRE(q && key && value && k_cache && v_cache && slot_mapping && positions && inv_freq,
             PA_ERR_INVALID_ARG, "pa_rope_reshape_and_cache: null pointer");
  if (q_stride == 0) q_stride = (int64_t)num_heads * head_dim;
  if (key_stride == 0) key_stride = (int64_t)num_kv_heads * head_dim;
  if (value_stride == 0) value_stride = (int64_t)num_kv_heads * head_dim;
  PA_REQUIRE(q_stride >= (int64_t)num_heads * head_dim &&
                 key_stride >= (int64_t)num_kv_heads * head_dim &&
                 value_stride >= (int64_t)num_kv_heads * head_dim,
             PA_ERR_INVALID_ARG, "pa_rope_reshape_and_cache: token stride too small");
  const int64_t num_slots = (int64_t)num_blocks * kBlock;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == PA_DTYPE_BF16)
    rope_cache_kernel<uint16_t><<<num_tokens, 256, 0, s>>>(
        (uint16_t*)q, q_stride, (const uint16_t*)key, key_stride, (const uint16_t*)value,
        value_stride, (uint16_t*)k_cache, (uint16_t*)v_cache, slot_mapping, positions, inv_freq,
        num_heads, num_kv_heads, head_dim, num_slots);
  else
    rope_cache_kernel<float><<<num_tokens, 256, 0, s>>>(
        (float*)q, q_stride, (const float*)key, key_stride, (const float*)value, value_stride,
        (float*)k_cache, (float*)v_cache, slot_mapping, positions, inv_freq, num_heads,
        num_kv_heads, head_dim, num_slots);
  return check_launch("pa_rope_reshape_and_cache");
}
