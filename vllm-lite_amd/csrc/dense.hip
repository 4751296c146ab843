// Dense-side kernels of an end-to-end decoder step (pa_dense.h): residual
// add + RMSNorm or LayerNorm, and the SwiGLU activation.  All are HBM-bound
// row passes.
#include "pa_common.hpp"
#include "../../include/pa_dense.h"

namespace pa {
namespace {

// One workgroup per row: optional residual add, sum of squares reduced over
// the workgroup, then the scaled write.
template <typename T>
__global__ __launch_bounds__(256) void rms_norm_kernel(T* __restrict__ out, T* __restrict__ res,
                                                       const T* __restrict__ add,
                                                       const T* __restrict__ w, int hidden,
                                                       float eps) {
  __shared__ float red[256];
  const int64_t row = blockIdx.x;
  T* x = res + row * hidden;
  const T* a = add ? add + row * hidden : nullptr;
  float ss = 0.f;
  for (int i = threadIdx.x; i < hidden; i += blockDim.x) {
    float v = Elem<T>::load(x + i);
    if (a) {
      // the residual is kept in the storage dtype, as the sum tensor would be
      Elem<T>::store(x + i, v + Elem<T>::load(a + i));
      v = Elem<T>::load(x + i);
    }
    ss += v * v;
  }
  red[threadIdx.x] = ss;
  __syncthreads();
  for (int s = blockDim.x / 2; s > 0; s >>= 1) {
    if (threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
    __syncthreads();
  }
  const float inv = 1.0f / sqrtf(red[0] / (float)hidden + eps);
  T* o = out + row * hidden;
  for (int i = threadIdx.x; i < hidden; i += blockDim.x)
    Elem<T>::store(o + i, Elem<T>::load(x + i) * inv * Elem<T>::load(w + i));
}

__device__ inline float block_sum(float v, float* red) {
  red[threadIdx.x] = v;
  __syncthreads();
  for (int s = blockDim.x / 2; s > 0; s >>= 1) {
    if (threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
    __syncthreads();
  }
  const float r = red[0];
  __syncthreads();
  return r;
}

// One workgroup per row: optional residual add, the row mean, the variance of
// the centred row (a second pass over the row, which is in L2 / LDS-sized), then
// (x - mean) / sqrt(var + eps) * w + b.
template <typename T>
__global__ __launch_bounds__(256) void layer_norm_kernel(T* __restrict__ out, T* __restrict__ res,
                                                         const T* __restrict__ add,
                                                         const T* __restrict__ w,
                                                         const T* __restrict__ bias, int hidden,
                                                         float eps) {
  __shared__ float red[256];
  const int64_t row = blockIdx.x;
  T* x = res + row * hidden;
  const T* a = add ? add + row * hidden : nullptr;
  float sum = 0.f;
  for (int i = threadIdx.x; i < hidden; i += blockDim.x) {
    if (a) Elem<T>::store(x + i, Elem<T>::load(x + i) + Elem<T>::load(a + i));
    sum += Elem<T>::load(x + i);
  }
  const float mean = block_sum(sum, red) / (float)hidden;
  float ss = 0.f;
  for (int i = threadIdx.x; i < hidden; i += blockDim.x) {
    const float d = Elem<T>::load(x + i) - mean;
    ss += d * d;
  }
  const float inv = 1.0f / sqrtf(block_sum(ss, red) / (float)hidden + eps);
  T* o = out + row * hidden;
  for (int i = threadIdx.x; i < hidden; i += blockDim.x) {
    float y = (Elem<T>::load(x + i) - mean) * inv * Elem<T>::load(w + i);
    if (bias) y += Elem<T>::load(bias + i);
    Elem<T>::store(o + i, y);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void silu_mul_kernel(T* __restrict__ out,
                                                       const T* __restrict__ gu, int inter,
                                                       int64_t n) {
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / inter;
    const int i = (int)(e % inter);
    const float g = Elem<T>::load(gu + r * 2 * inter + i);
    const float u = Elem<T>::load(gu + r * 2 * inter + inter + i);
    Elem<T>::store(out + e, g / (1.0f + expf(-g)) * u);
  }
}

}  // namespace
}  // namespace pa

using namespace pa;

extern "C" int32_t pa_rms_norm(void* out, void* residual, const void* add, const void* weight,
                               int32_t rows, int32_t hidden, float eps, int32_t dtype,
                               pa_stream_t stream) {
  clear_error();
  PA_REQUIRE(dtype_ok(dtype), PA_ERR_INVALID_ARG, "pa_rms_norm: unknown dtype %d", dtype);
  PA_REQUIRE(rows >= 0 && hidden > 0, PA_ERR_INVALID_ARG, "pa_rms_norm: bad sizes");
  if (rows == 0) return PA_OK;
  PA_REQUIRE(out && residual && weight, PA_ERR_INVALID_ARG, "pa_rms_norm: null pointer");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == PA_DTYPE_BF16)
    rms_norm_kernel<uint16_t><<<rows, 256, 0, s>>>((uint16_t*)out, (uint16_t*)residual,
                                                   (const uint16_t*)add, (const uint16_t*)weight,
                                                   hidden, eps);
  else
    rms_norm_kernel<float><<<rows, 256, 0, s>>>((float*)out, (float*)residual,
                                                (const float*)add, (const float*)weight, hidden,
                                                eps);
  return check_launch("pa_rms_norm");
}

extern "C" int32_t pa_layer_norm(void* out, void* residual, const void* add, const void* weight,
                                 const void* bias, int32_t rows, int32_t hidden, float eps,
                                 int32_t dtype, pa_stream_t stream) {
  clear_error();
  PA_REQUIRE(dtype_ok(dtype), PA_ERR_INVALID_ARG, "pa_layer_norm: unknown dtype %d", dtype);
  PA_REQUIRE(rows >= 0 && hidden > 0, PA_ERR_INVALID_ARG, "pa_layer_norm: bad sizes");
  if (rows == 0) return PA_OK;
  PA_REQUIRE(out && residual && weight, PA_ERR_INVALID_ARG, "pa_layer_norm: null pointer");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == PA_DTYPE_BF16)
    layer_norm_kernel<uint16_t><<<rows, 256, 0, s>>>(
        (uint16_t*)out, (uint16_t*)residual, (const uint16_t*)add, (const uint16_t*)weight,
        (const uint16_t*)bias, hidden, eps);
  else
    layer_norm_kernel<float><<<rows, 256, 0, s>>>((float*)out, (float*)residual,
                                                  (const float*)add, (const float*)weight,
                                                  (const float*)bias, hidden, eps);
  return check_launch("pa_layer_norm");
}

extern "C" int32_t pa_silu_mul(void* out, const void* gate_up, int32_t rows, int32_t inter,
                               int32_t dtype, pa_stream_t stream) {
  clear_error();
  PA_REQUIRE(dtype_ok(dtype), PA_ERR_INVALID_ARG, "pa_silu_mul: unknown dtype %d", dtype);
  PA_REQUIRE(rows >= 0 && inter > 0, PA_ERR_INVALID_ARG, "pa_silu_mul: bad sizes");
  if (rows == 0) return PA_OK;
  PA_REQUIRE(out && gate_up, PA_ERR_INVALID_ARG, "pa_silu_mul: null pointer");
  const int64_t n = (int64_t)rows * inter;
  const int blocks = (int)((n + 255) / 256 < 8192 ? (n + 255) / 256 : 8192);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == PA_DTYPE_BF16)
    silu_mul_kernel<uint16_t><<<blocks, 256, 0, s>>>((uint16_t*)out, (const uint16_t*)gate_up,
                                                     inter, n);
  else
    silu_mul_kernel<float><<<blocks, 256, 0, s>>>((float*)out, (const float*)gate_up, inter, n);
  return check_launch("pa_silu_mul");
}
