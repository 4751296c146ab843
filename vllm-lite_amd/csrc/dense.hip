// Dense-side kernels of an end-to-end decoder step (pa_dense.h): residual
// add + RMSNorm or LayerNorm, and the SwiGLU activation.  All are HBM-bound
// row passes.
#include <algorithm>

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


// Skinny-M linear layer (decode-step projections): Y[M, N] = X[M, K] · W[N, K]ᵀ
// in bf16 with f32 accumulation, for M of a few tens of rows, where the
// weights dominate the bytes (HBM-bound, ~M flops per weight byte).
// v_mfma_f32_16x16x32_bf16 on Yᵀ tiles: A = 16 weight rows (lane: row c,
// k 8j .. 8j+7, streamed from HBM; from the packed layout of
// linear_pack_kernel every fragment is one contiguous KB), B = 16 batch rows
// of X (same k slice, from L2), D = Yᵀ[weight row 4j + r][batch row c].
// A wavefront computes NT x 16 weight rows x 32 batch rows over its share of
// the K steps (32 each), loading the operands of the next stage of U steps
// while it multiplies the current one; NT > 1 reuses each X fragment for NT
// weight tiles.
// The kw wavefronts of a workgroup (up to 16 for NT = 1 with U = 4, else 8)
// split K and sum their partial tiles in LDS; wavefront 0 applies the
// epilogue:
//   EPI 0: none, EPI 1: + bias[n],
//   EPI 2 (NT = 2): SwiGLU on a fused gate|up weight [2 I, K]: the two weight
//          tiles are gate rows a0 + c and up rows I + a0 + c, and
//          out[m][a] = silu(bf16(g)) * bf16(u) (the rounding of the unfused
//          path, whose projection output is bf16).
// Weight tiles of the last column block that lie past N (N a multiple of 16)
// read row n0 and are not stored.
template <int EPI, int NT, bool PK, int U>
__global__ __launch_bounds__(NT == 1 && U == 4 ? 1024 : 512) void linear_skinny_kernel(
    uint16_t* __restrict__ out, const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ bias, int M, int N, int K, int kw, int flags, float eps) {
  static_assert(EPI != 2 || NT == 2, "SwiGLU pairs one gate and one up tile");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, j = lane >> 4;
  const int nsteps = K / 32;
  const int s0 = wave * nsteps / kw, s1 = (wave + 1) * nsteps / kw;
  const int m0 = blockIdx.y * 32;
  const int n0 = blockIdx.x * (EPI == 2 ? 16 : 16 * NT);
  // Weight fragment of tile t (16 rows from row r0) at step s:
  //   row-major:  w + (r0 + c) * K + 32 s + 8 j
  //   packed:     w + ((r0 / 16 * nsteps + s) * 64 + lane) * 8  (one contiguous KB)
  const uint16_t* wp[NT];
  bool tv[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    tv[t] = EPI == 2 || n0 + 16 * t < N;
    const int64_t r0 = EPI == 2 ? (t == 0 ? n0 : (int64_t)N + n0) : (tv[t] ? n0 + 16 * t : n0);
    wp[t] = PK ? w + (r0 / 16 * nsteps * 64 + lane) * 8 : w + (r0 + c) * K + 8 * j;
  }
  const uint16_t* xp0 = x + (int64_t)(m0 + c < M ? m0 + c : 0) * K + 8 * j;
  const uint16_t* xp1 = x + (int64_t)(m0 + 16 + c < M ? m0 + 16 + c : 0) * K + 8 * j;
  f32x4 acc[NT][2];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[t][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  // PA_LINEAR_RMS_IN: per-lane sums of squares of the X fragments (batch rows
  // c and 16 + c, this lane's 8 columns of each step)
  const bool rms = (flags & PA_LINEAR_RMS_IN) != 0;
  float ss[2] = {0.f, 0.f};

  bf16x8 a[2][U][NT], b[2][U][2];
  // Loads are unconditional (a step past the wavefront's share reloads its
  // last step, whose product is then skipped; a batch row past M reads row 0,
  // whose output column is never stored), so the compiler can count them.
  auto load = [&](int st, bf16x8 (&aa)[U][NT], bf16x8 (&bb)[U][2]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int step = min(st + u, s1 - 1);
      const int k = step * 32;
#pragma unroll
      for (int t = 0; t < NT; ++t)
        aa[u][t] = *reinterpret_cast<const bf16x8*>(wp[t] + (PK ? step * 512 : k));
      bb[u][0] = *reinterpret_cast<const bf16x8*>(xp0 + k);
      bb[u][1] = *reinterpret_cast<const bf16x8*>(xp1 + k);
    }
  };
  auto mma = [&](int st, const bf16x8 (&aa)[U][NT], const bf16x8 (&bb)[U][2]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (st + u < s1) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int q = 0; q < 2; ++q)
            acc[t][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aa[u][t], bb[u][q], acc[t][q], 0, 0, 0);
        if (rms) {
#pragma unroll
          for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const float v = (float)bb[u][q][i];
              ss[q] += v * v;
            }
        }
      }
    }
  };
  if (s0 < s1) load(s0, a[0], b[0]);
  for (int s = s0; s < s1; s += 2 * U) {
    if (s + U < s1) load(s + U, a[1], b[1]);
    mma(s, a[0], b[0]);
    if (s + U >= s1) break;
    if (s + 2 * U < s1) load(s + 2 * U, a[0], b[0]);
    mma(s + U, a[1], b[1]);
  }

  constexpr int MAXW = NT == 1 && U == 4 ? 16 : 8;
  __shared__ f32x4 red[MAXW - 1][2 * NT][64];
  __shared__ float rss[MAXW][2][16];
  if (rms) {
    // a batch row's columns are spread over the 4 lanes j of its c
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      ss[q] += __shfl_xor(ss[q], 16, 64);
      ss[q] += __shfl_xor(ss[q], 32, 64);
    }
    if (j == 0) {
      rss[wave][0][c] = ss[0];
      rss[wave][1][c] = ss[1];
    }
  }
  if (kw > 1) {
    if (wave > 0) {
#pragma unroll
      for (int q = 0; q < 2 * NT; ++q) red[wave - 1][q][lane] = acc[q >> 1][q & 1];
    }
    __syncthreads();
    if (wave != 0) return;
    for (int v = 0; v < kw - 1; ++v)
#pragma unroll
      for (int q = 0; q < 2 * NT; ++q) acc[q >> 1][q & 1] += red[v][q][lane];
  } else if (rms) {
    __syncthreads();
  }
  // 1 / rms of the batch rows (1 without PA_LINEAR_RMS_IN); the norm weight
  // is folded into the packed weight's columns
  float inv[2] = {1.f, 1.f};
  if (rms) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      float t = 0.f;
      for (int v = 0; v < kw; ++v) t += rss[v][q][c];
      inv[q] = 1.0f / sqrtf(t / (float)K + eps);
    }
  }
  const bool add_out = (flags & PA_LINEAR_ADD_OUT) != 0;
#pragma unroll
  for (int bb = 0; bb < 2; ++bb) {
    const int m = m0 + 16 * bb + c;
    if (m >= M) continue;
    if constexpr (EPI == 2) {
      uint16_t o4[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float g = bf16_bits_to_f32(f32_to_bf16_bits(acc[0][bb][r] * inv[bb]));
        const float u = bf16_bits_to_f32(f32_to_bf16_bits(acc[1][bb][r] * inv[bb]));
        o4[r] = f32_to_bf16_bits(g / (1.0f + expf(-g)) * u);
      }
      *reinterpret_cast<uint64_t*>(out + (int64_t)m * N + n0 + 4 * j) =
          *reinterpret_cast<const uint64_t*>(o4);
    } else {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if (!tv[t]) continue;
        const int n = n0 + 16 * t + 4 * j;
        uint64_t* dst = reinterpret_cast<uint64_t*>(out + (int64_t)m * N + n);
        uint16_t prev[4];
        if (add_out) *reinterpret_cast<uint64_t*>(prev) = *dst;
        uint16_t o4[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float y = acc[t][bb][r] * inv[bb];
          if constexpr (EPI == 1) y += bf16_bits_to_f32(bias[n + r]);
          // residual add: the projection output rounded to bf16 first, as
          // when it is materialised and added by the norm kernel
          if (add_out) y = bf16_bits_to_f32(prev[r]) + bf16_bits_to_f32(f32_to_bf16_bits(y));
          o4[r] = f32_to_bf16_bits(y);
        }
        *dst = *reinterpret_cast<const uint64_t*>(o4);
      }
    }
  }
}

// Packs a row-major bf16 weight [N, K] (N a multiple of 16, K of 32) into the
// MFMA-fragment order linear_skinny_kernel<., ., true> reads: fragment
// (tile, step) = rows 16 tile .. +15, columns 32 step .. +31 is 1 KB at
// ((tile * K / 32 + step) * 64) * 8 elements, lane l = 16 j + c holding row
// 16 tile + c, columns 32 step + 8 j .. +7, optionally times col_scale[col]
// (rounded to bf16).  One thread per 16-byte piece.
__global__ __launch_bounds__(256) void linear_pack_kernel(uint16_t* __restrict__ dst,
                                                          const uint16_t* __restrict__ src,
                                                          const uint16_t* __restrict__ col_scale,
                                                          int N, int K) {
  const int64_t total = (int64_t)N * K / 8;
  const int nsteps = K / 32;
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < total;
       q += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(q & 63);
    const int64_t frag = q >> 6;
    const int64_t tile = frag / nsteps;
    const int step = (int)(frag % nsteps);
    const int64_t row = tile * 16 + (lane & 15);
    const int col = step * 32 + 8 * (lane >> 4);
    uint4 v = *reinterpret_cast<const uint4*>(src + row * K + col);
    if (col_scale) {
      uint16_t* e = reinterpret_cast<uint16_t*>(&v);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        e[i] = f32_to_bf16_bits(bf16_bits_to_f32(e[i]) * bf16_bits_to_f32(col_scale[col + i]));
    }
    *reinterpret_cast<uint4*>(dst + q * 8) = v;
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

extern "C" int32_t pa_linear(void* out, const void* x, const void* weight, const void* bias,
                             int32_t rows, int32_t out_features, int32_t in_features, int32_t act,
                             int32_t packed, int32_t flags, float eps, int32_t dtype,
                             pa_stream_t stream) {
  clear_error();
  PA_REQUIRE(dtype == PA_DTYPE_BF16, PA_ERR_UNSUPPORTED, "pa_linear: dtype %d (bf16 only)", dtype);
  PA_REQUIRE(act == PA_ACT_NONE || act == PA_ACT_SILU_MUL, PA_ERR_INVALID_ARG,
             "pa_linear: unknown activation %d", act);
  PA_REQUIRE(rows >= 0 && out_features > 0 && in_features > 0, PA_ERR_INVALID_ARG,
             "pa_linear: bad sizes");
  PA_REQUIRE(in_features % 32 == 0, PA_ERR_UNSUPPORTED,
             "pa_linear: in_features %d not a multiple of 32", in_features);
  PA_REQUIRE(out_features % 16 == 0, PA_ERR_UNSUPPORTED,
             "pa_linear: out_features %d not a multiple of 16", out_features);
  PA_REQUIRE(act == PA_ACT_NONE || !bias, PA_ERR_INVALID_ARG,
             "pa_linear: bias with the SwiGLU epilogue");
  PA_REQUIRE((flags & ~(PA_LINEAR_RMS_IN | PA_LINEAR_ADD_OUT)) == 0, PA_ERR_INVALID_ARG,
             "pa_linear: unknown flags %d", flags);
  PA_REQUIRE(!(flags & PA_LINEAR_ADD_OUT) || act == PA_ACT_NONE, PA_ERR_INVALID_ARG,
             "pa_linear: residual add with the SwiGLU epilogue");
  PA_REQUIRE(!(flags & PA_LINEAR_RMS_IN) || eps > 0.f, PA_ERR_INVALID_ARG,
             "pa_linear: eps must be positive");
  if (rows == 0) return PA_OK;
  PA_REQUIRE(out && x && weight, PA_ERR_INVALID_ARG, "pa_linear: null pointer");
  PA_REQUIRE(((uintptr_t)x | (uintptr_t)weight | (uintptr_t)out) % 16 == 0, PA_ERR_INVALID_ARG,
             "pa_linear: x, weight and out must be 16-byte aligned");
  PA_REQUIRE((rows + 31) / 32 <= 65535, PA_ERR_UNSUPPORTED, "pa_linear: %d rows", rows);
  // Weight tiles per wavefront: 4 for wide outputs (each X fragment then
  // feeds 4 tiles), 1 where 2 would leave fewer than ~512 wavefronts, else 2.
  // K split: NT = 1 runs up to 16 wavefronts per workgroup, with one stage of
  // 8 steps when K is short and stages of 4 otherwise; NT > 1 up to 8
  // wavefronts of about 8 steps (two stages of 4).
  const int nsteps = in_features / 32;
  int kw = std::max(1, std::min(8, (nsteps + 7) / 8));
  int nt = 2;
  if (act != PA_ACT_SILU_MUL) {
    if ((out_features + 63) / 64 >= 1024) nt = 4;
    else if ((long long)((out_features + 31) / 32) * kw < 512) nt = 1;
  }
  int stage = 4;
  if (nt == 1) {
    if (nsteps <= 64) {
      stage = 8;
    } else {
      kw = std::min(16, (nsteps + 7) / 8);
    }
  }
  const int cols = act == PA_ACT_SILU_MUL ? 16 : 16 * nt;
  const dim3 grid((out_features + cols - 1) / cols, (rows + 31) / 32);
  hipStream_t s = (hipStream_t)stream;
  auto* o = (uint16_t*)out;
  auto* xx = (const uint16_t*)x;
  auto* ww = (const uint16_t*)weight;
  auto* bb = (const uint16_t*)bias;
#define PA_LAUNCH_LINEAR_U(EPI, NT, UU)                                                       \
  (packed ? linear_skinny_kernel<EPI, NT, true, UU><<<grid, 64 * kw, 0, s>>>(                  \
                o, xx, ww, bb, rows, out_features, in_features, kw, flags, eps)               \
          : linear_skinny_kernel<EPI, NT, false, UU><<<grid, 64 * kw, 0, s>>>(                 \
                o, xx, ww, bb, rows, out_features, in_features, kw, flags, eps))
#define PA_LAUNCH_LINEAR(EPI, NT)                                                             \
  (NT == 1 && stage == 8 ? PA_LAUNCH_LINEAR_U(EPI, 1, 8) : PA_LAUNCH_LINEAR_U(EPI, NT, 4))
  if (act == PA_ACT_SILU_MUL)
    PA_LAUNCH_LINEAR_U(2, 2, 4);
  else if (bias)
    nt == 4 ? PA_LAUNCH_LINEAR_U(1, 4, 4) : nt == 2 ? PA_LAUNCH_LINEAR_U(1, 2, 4) : PA_LAUNCH_LINEAR(1, 1);
  else
    nt == 4 ? PA_LAUNCH_LINEAR_U(0, 4, 4) : nt == 2 ? PA_LAUNCH_LINEAR_U(0, 2, 4) : PA_LAUNCH_LINEAR(0, 1);
#undef PA_LAUNCH_LINEAR
#undef PA_LAUNCH_LINEAR_U
  return check_launch("pa_linear");
}

extern "C" int32_t pa_linear_pack(void* packed, const void* weight, const void* col_scale,
                                  int32_t rows, int32_t cols, int32_t dtype, pa_stream_t stream) {
  clear_error();
  PA_REQUIRE(dtype == PA_DTYPE_BF16, PA_ERR_UNSUPPORTED, "pa_linear_pack: dtype %d (bf16 only)",
             dtype);
  PA_REQUIRE(rows > 0 && cols > 0 && rows % 16 == 0 && cols % 32 == 0, PA_ERR_UNSUPPORTED,
             "pa_linear_pack: %d x %d (rows a multiple of 16, cols of 32)", rows, cols);
  PA_REQUIRE(packed && weight && packed != weight, PA_ERR_INVALID_ARG,
             "pa_linear_pack: null or aliased pointers");
  PA_REQUIRE(((uintptr_t)packed | (uintptr_t)weight) % 16 == 0, PA_ERR_INVALID_ARG,
             "pa_linear_pack: pointers must be 16-byte aligned");
  const int64_t pieces = (int64_t)rows * cols / 8;
  const int blocks = (int)std::min<int64_t>((pieces + 255) / 256, 65536);
  linear_pack_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>(
      (uint16_t*)packed, (const uint16_t*)weight, (const uint16_t*)col_scale, rows, cols);
  return check_launch("pa_linear_pack");
}
