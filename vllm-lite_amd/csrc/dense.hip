// Dense-side kernels of an end-to-end decoder step (pa_dense.h): residual
// add + RMSNorm or LayerNorm, the SwiGLU activation, skinny-M projections and
// the greedy argmax over logit rows.  All are HBM-bound.
#include <algorithm>
#include <climits>
#include <type_traits>

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

// bf16 rows of hidden % 8 == 0, hidden <= 64 * 8 * kNormChunks: one wavefront
// per row (4 rows per workgroup), the row held in registers as 16-byte
// chunks (chunk i of lane l is chunk l + 64 i of the row), so x is read once
// and written at most once; the sum of squares reduced by lane shuffles.
// Same results as rms_norm_kernel up to the order of the f32 sum.
constexpr int kNormChunks = 4;
__global__ __launch_bounds__(256) void rms_norm_rows_kernel(uint16_t* __restrict__ out,
                                                           uint16_t* __restrict__ res,
                                                           const uint16_t* __restrict__ add,
                                                           const uint16_t* __restrict__ w,
                                                           int rows, int hidden, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nch = hidden / 8;
  uint16_t* x = res + row * hidden;
  const uint16_t* a = add ? add + row * hidden : nullptr;
  bf16x8 v[kNormChunks], av[kNormChunks];
#pragma unroll
  for (int i = 0; i < kNormChunks; ++i) {
    const int ch = lane + 64 * i;
    if (ch < nch) {
      v[i] = *reinterpret_cast<const bf16x8*>(x + 8 * ch);
      if (a) av[i] = *reinterpret_cast<const bf16x8*>(a + 8 * ch);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kNormChunks; ++i) {
    const int ch = lane + 64 * i;
    if (ch < nch) {
      if (a) {
        // the residual is kept in the storage dtype, as the sum tensor would be
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = (__bf16)((float)v[i][e] + (float)av[i][e]);
        *reinterpret_cast<bf16x8*>(x + 8 * ch) = v[i];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += (float)v[i][e] * (float)v[i][e];
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
  const float inv = 1.0f / sqrtf(ss / (float)hidden + eps);
  uint16_t* orow = out + row * hidden;
#pragma unroll
  for (int i = 0; i < kNormChunks; ++i) {
    const int ch = lane + 64 * i;
    if (ch < nch) {
      const bf16x8 wv = *reinterpret_cast<const bf16x8*>(w + 8 * ch);
      bf16x8 r;
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] = (__bf16)((float)v[i][e] * inv * (float)wv[e]);
      *reinterpret_cast<bf16x8*>(orow + 8 * ch) = r;
    }
  }
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
// Epilogue 3 (NT = 1; the decode step's QKV projection with RoPE and the
// KV-cache write fused in): per token row m its position and cache slot, the
// inverse-frequency table, the layer's caches ([NB, Hkv, 16, D] keys,
// token-minor [NB, Hkv, D, 16] values) and the head layout of the output
// columns (Hq query heads, then Hkv key heads, then Hkv value heads of D).
struct RopeCacheArgs {
  const int64_t* positions;
  const int64_t* slots;
  const float* inv_freq;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t num_slots;
  int Hq, Hkv, D;
};

template <int EPI, int NT, bool PK, int U>
__global__ __launch_bounds__(NT == 1 && U == 4 ? 1024 : 512) void linear_skinny_kernel(
    uint16_t* __restrict__ out, const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ bias, int M, int N, int K, int kw, int flags, float eps,
    float* __restrict__ ws, int* __restrict__ counters, const RopeCacheArgs ra) {
  static_assert(EPI != 2 || NT == 2, "SwiGLU pairs one gate and one up tile");
  static_assert(EPI != 3 || NT == 1, "RoPE pairs sit in one tile, partners 32 lanes apart");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, j = lane >> 4;
  const int nsteps = K / 32;
  // K split: workgroup z of gridDim.z takes steps [k0, k1), its wavefronts
  // an equal share each
  const int splits = gridDim.z;
  const int k0 = blockIdx.z * nsteps / splits, k1 = (blockIdx.z + 1) * nsteps / splits;
  const int s0 = k0 + wave * (k1 - k0) / kw, s1 = k0 + (wave + 1) * (k1 - k0) / kw;
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
  // Epilogue 3: with rope pairs, tile u of a query or key head holds head
  // rows 8 u .. 8 u + 7 (tile rows 0-7: first members) and D / 2 + 8 u ..
  // D / 2 + 8 u + 7 (tile rows 8-15: second members), as linear_pack_kernel
  // packs them.  Lane (c, j) holds tile rows 4 j .. 4 j + 3 (head rows
  // f .. f + 3), so its row 4 j + r belongs to pair 8 u + 4 (j & 1) + r and
  // the partner member is in lane ^ 32; value heads keep their row order.
  // Wavefront 0 loads the epilogue's other operands (bias, cache slots,
  // positions); the one-stage instance (U = 8) ahead of the weight stream,
  // so their round trips do not queue behind it, the 1024-thread instance,
  // whose registers are fewer, after its K loop.
  uint16_t bias3[4] = {0, 0, 0, 0};
  int64_t slot3[2] = {-1, -1};
  int64_t pos3 = 0;
  auto epi_operands = [&]() {
    if (EPI == 3 && wave == 0) {
      const int D = ra.D;
      const int head = n0 / D, u = (n0 % D) / 16;
      const bool rot = head < ra.Hq + ra.Hkv;
      const int f = rot ? (j >> 1) * (D / 2) + 8 * u + 4 * (j & 1) : 16 * u + 4 * j;
      if (bias) {
#pragma unroll
        for (int r = 0; r < 4; ++r) bias3[r] = bias[head * D + f + r];
      }
#pragma unroll
      for (int bb = 0; bb < 2; ++bb) slot3[bb] = ra.slots[min(m0 + 16 * bb + c, M - 1)];
      if (rot) pos3 = ra.positions[min(m0 + (j >= 2 ? 16 : 0) + c, M - 1)];
    }
  };
  if constexpr (U == 8) epi_operands();
  if (s0 < s1) load(s0, a[0], b[0]);
  // The rotation angles of batch rows c (bb 0) and 16 + c (bb 1), computed
  // by wavefront 0 (with the operands above: U = 8 while its loads are in
  // flight): lanes j < 2 take batch row c, lanes j >= 2 batch row 16 + c
  // (the same pairs), and the partners swap results.
  float rsn[2][4], rcs[2][4];
  auto angles = [&]() {
    if constexpr (EPI == 3) {
      const int head = n0 / ra.D;
      if (wave == 0 && head < ra.Hq + ra.Hkv) {
        const int pi0 = 8 * ((n0 % ra.D) / 16) + 4 * (j & 1);
        const bool hi = j >= 2;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float sn, cs;
          sincosf((float)pos3 * ra.inv_freq[pi0 + r], &sn, &cs);
          const float osn = __shfl_xor(sn, 32, 64), ocs = __shfl_xor(cs, 32, 64);
          rsn[0][r] = hi ? osn : sn;
          rcs[0][r] = hi ? ocs : cs;
          rsn[1][r] = hi ? sn : osn;
          rcs[1][r] = hi ? cs : ocs;
        }
      }
    }
  };
  if constexpr (U == 8) angles();
  for (int s = s0; s < s1; s += 2 * U) {
    if (s + U < s1) load(s + U, a[1], b[1]);
    mma(s, a[0], b[0]);
    if (s + U >= s1) break;
    if (s + 2 * U < s1) load(s + 2 * U, a[0], b[0]);
    mma(s + U, a[1], b[1]);
  }

  if constexpr (U != 8) {
    epi_operands();
    angles();
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
  float ssum[2] = {0.f, 0.f};  // sums of squares of batch rows c, 16 + c
  if (rms) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
      for (int v = 0; v < kw; ++v) ssum[q] += rss[v][q][c];
  }
  if (splits > 1) {
    // Split K: the workgroup's partial tile (and sums of squares) goes to
    // its record in the workspace; the last of the tile's `splits`
    // workgroups to arrive (counted by a device-scope atomic) sums the
    // records in split order, so the result does not depend on the arrival
    // order, applies the epilogue and sets the counter back to zero for the
    // next call.
    // The records cross workgroups on other XCDs, whose L2s are not
    // coherent with this one.  Publication follows the HIP memory model:
    // the records are written as agent-scope relaxed atomics (stores
    // written through past the non-coherent levels), the arrival is an
    // agent-scope release RMW on the tile's counter, and the workgroup that
    // observes the final count issues an agent-scope acquire fence before
    // it reads the records.  The release orders this wavefront's record
    // stores (program order within the wavefront, then the release at
    // agent scope) before the increment; every earlier arrival's increment
    // heads a release sequence the last RMW reads from, so the acquire
    // fence makes all `splits` records visible.
    constexpr int RECF = 2 * NT * 256 + 32;  // floats per record
    const int64_t tile = (int64_t)blockIdx.y * gridDim.x + blockIdx.x;
    float* mine = ws + (tile * splits + blockIdx.z) * RECF;
    auto put = [](float* p, float v) {
      __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    auto get = [](const float* p) {
      return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
#pragma unroll
    for (int q = 0; q < 2 * NT; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r) put(mine + (q * 64 + lane) * 4 + r, acc[q >> 1][q & 1][r]);
    if (j == 0) {
      put(mine + 2 * NT * 256 + c, ssum[0]);
      put(mine + 2 * NT * 256 + 16 + c, ssum[1]);
    }
    int arrived = 0;
    if (lane == 0)
      arrived = __hip_atomic_fetch_add(counters + tile, 1, __ATOMIC_RELEASE,
                                       __HIP_MEMORY_SCOPE_AGENT);
    if (__builtin_amdgcn_readfirstlane(arrived) != splits - 1) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
#pragma unroll
    for (int q = 0; q < 2 * NT; ++q) acc[q >> 1][q & 1] = f32x4{0.f, 0.f, 0.f, 0.f};
    ssum[0] = ssum[1] = 0.f;
    for (int z = 0; z < splits; ++z) {
      const float* rec = ws + (tile * splits + z) * RECF;
#pragma unroll
      for (int q = 0; q < 2 * NT; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[q >> 1][q & 1][r] += get(rec + (q * 64 + lane) * 4 + r);
      ssum[0] += get(rec + 2 * NT * 256 + c);
      ssum[1] += get(rec + 2 * NT * 256 + 16 + c);
    }
    if (lane == 0)
      __hip_atomic_store(counters + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // 1 / rms of the batch rows (1 without PA_LINEAR_RMS_IN); the norm weight
  // is folded into the packed weight's columns
  float inv[2] = {1.f, 1.f};
  if (rms) {
#pragma unroll
    for (int q = 0; q < 2; ++q) inv[q] = 1.0f / sqrtf(ssum[q] / (float)K + eps);
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
    } else if constexpr (EPI == 3) {
      // Rounded to bf16 as the unfused projection output, then rotated as
      // rope_cache_kernel does (the partner member from lane ^ 32; lanes c
      // and c ^ 32 share the batch row, so both take this branch or neither).
      // Value heads keep their row order.
      const int D = ra.D;
      const int head = n0 / D, u = (n0 % D) / 16;
      const bool rot = head < ra.Hq + ra.Hkv;
      const int f = rot ? (j >> 1) * (D / 2) + 8 * u + 4 * (j & 1) : 16 * u + 4 * j;  // head row
      float y[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float a0 = acc[0][bb][r] * inv[bb];
        if (bias) a0 += bf16_bits_to_f32(bias3[r]);
        y[r] = bf16_bits_to_f32(f32_to_bf16_bits(a0));
      }
      if (rot) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = __shfl_xor(y[r], 32, 64);
          const float sn = rsn[bb][r], cs = rcs[bb][r];
          y[r] = j < 2 ? y[r] * cs - p * sn : y[r] * cs + p * sn;
        }
      }
      uint16_t o4[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) o4[r] = f32_to_bf16_bits(y[r]);
      *reinterpret_cast<uint64_t*>(out + (int64_t)m * N + head * D + f) =
          *reinterpret_cast<const uint64_t*>(o4);
      const int64_t slot = slot3[bb];
      if (head >= ra.Hq && slot >= 0 && slot < ra.num_slots) {
        const int64_t blk = slot / kBlock;
        const int off = (int)(slot % kBlock);
        if (rot) {
          uint16_t* kd = ra.k_cache + ((blk * ra.Hkv + (head - ra.Hq)) * kBlock + off) * D + f;
          *reinterpret_cast<uint64_t*>(kd) = *reinterpret_cast<const uint64_t*>(o4);
        } else {
          uint16_t* vd =
              ra.v_cache + ((blk * ra.Hkv + (head - ra.Hq - ra.Hkv)) * D + f) * kBlock + off;
#pragma unroll
          for (int r = 0; r < 4; ++r) vd[r * kBlock] = o4[r];
        }
      }
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

// Wide projections of one batch tile (M <= 32 rows, N / 16 >= kWideMinTiles
// weight tiles over packed weights: the LM head) with the batch rows held in
// LDS.  A persistent grid of one WG-wavefront workgroup per CU: each
// workgroup copies X [M, K] into LDS once (rows padded by 16 bytes so the 16
// rows one operand read touches fall in distinct banks; rows past M zero),
// with PA_LINEAR_RMS_IN forms 1 / rms of each row once, and then every
// wavefront streams its own contiguous range of 16-row weight tiles from HBM
// (two tiles at a time, each step's X fragments read from LDS once for both)
// with the whole K per wavefront: no partial sums cross wavefronts.  The
// weight stream runs in units of U K steps through NB register buffers,
// across tile boundaries, so the next tile's first fragments are in flight
// during a tile pair's epilogue.  Tiles are dealt evenly over the grid's
// wavefronts, so every CU reads the same share of the weight.
constexpr int kWideMinTiles = 4096;
constexpr int kWideMaxK = 992;  // X in at most 64 KB of dynamic LDS
template <int U, int NB, int WG>
__global__ __launch_bounds__(64 * WG) void linear_wide_kernel(uint16_t* __restrict__ out,
                                                         const uint16_t* __restrict__ x,
                                                         const uint16_t* __restrict__ w, int M,
                                                         int N, int K, int flags, float eps) {
  extern __shared__ __attribute__((aligned(16))) uint8_t xs[];  // [32][2 K + 16] bytes, inv[32]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, j = lane >> 4;
  const int nsteps = K / 32;
  const int rowb = 2 * K + 16;
  float* inv_s = reinterpret_cast<float*>(xs + 32 * rowb);

  // this wavefront's tiles [t0, t1), in pairs (the last pair of an odd
  // range repeats its tile and stores it once)
  const int T = N / 16;
  const int64_t gw = (int64_t)blockIdx.x * WG + wave, GW = (int64_t)gridDim.x * WG;
  const int t0 = (int)(gw * T / GW), t1 = (int)((gw + 1) * T / GW);
  const int npairs = (t1 - t0 + 1) / 2;
  const int nu = nsteps / U;  // units per tile pair
  const int total = npairs * nu;
  const uint8_t* xr0 = xs + c * rowb + 16 * j;
  const uint8_t* xr1 = xs + (16 + c) * rowb + 16 * j;

  bf16x8 a0[U][2], a1[U][2];
  f32x4 acc[2][2];
#pragma unroll
  for (int t = 0; t < 2; ++t) acc[t][0] = acc[t][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  // U divides the K steps, so a unit's fragments of a tile are U
  // consecutive KB of the packed weight.  Raw buffer loads over the tile
  // (non-temporal: with the default policy the same launch after a write
  // of 512 MB took 113 instead of 64 us, the weight's lines evicting dirty
  // ones; only back-to-back launches whose weight stays partly in the MALL
  // read faster with it): the lane's offset is one fixed register and the unit's
  // a scalar, so no address registers are rewritten per unit (rewriting
  // them made the compiler wait for loads in flight that had been given
  // the same registers).
  // X into LDS and 1 / rms of its rows, by the whole workgroup; called
  // after the first weight units are in flight, so their latencies overlap
  float inv[2];
  auto stage_x = [&]() {
    for (int e = threadIdx.x; e < 32 * (K / 8); e += 64 * WG) {
      const int m = e / (K / 8), ch = e % (K / 8);
      bf16x8 v = bf16x8{};
      if (m < M) v = *reinterpret_cast<const bf16x8*>(x + (int64_t)m * K + 8 * ch);
      *reinterpret_cast<bf16x8*>(xs + m * rowb + 16 * ch) = v;
    }
    __syncthreads();
    if (threadIdx.x < 32 * 8) {
      // eight lanes per row: sum of squares of the row's bf16 values
      const int m = threadIdx.x >> 3, part = threadIdx.x & 7;
      float ss = 0.f;
      for (int ch = part; ch < K / 8; ch += 8) {
        const bf16x8 v = *reinterpret_cast<const bf16x8*>(xs + m * rowb + 16 * ch);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += (float)v[e] * (float)v[e];
      }
      ss += __shfl_xor(ss, 1, 64);
      ss += __shfl_xor(ss, 2, 64);
      ss += __shfl_xor(ss, 4, 64);
      if (part == 0)
        inv_s[m] = (flags & PA_LINEAR_RMS_IN) ? 1.0f / sqrtf(ss / (float)K + eps) : 1.0f;
    }
    __syncthreads();
    inv[0] = inv_s[c];
    inv[1] = inv_s[16 + c];
  };
  const int voff = lane * 16;
  const int tile_bytes = nsteps * 1024;
  auto load = [&](int u, bf16x8 (&a)[U][2]) __attribute__((always_inline)) {
    const int p = u / nu, st = u % nu;
    const int ta = t0 + 2 * p, tb = min(ta + 1, t1 - 1);
    const auto ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(w + (int64_t)ta * nsteps * 512), 0, tile_bytes, 0x00020000);
    const auto rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(w + (int64_t)tb * nsteps * 512), 0, tile_bytes, 0x00020000);
#pragma unroll
    for (int uu = 0; uu < U; ++uu) {
      const int so = (st * U + uu) * 1024;
      a[uu][0] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(ra, voff, so, 2));
      a[uu][1] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rb, voff, so, 2));
    }
  };
  auto mma = [&](int u, const bf16x8 (&a)[U][2]) __attribute__((always_inline)) {
    const int p = u / nu, st = u % nu;
    // the unit's X fragments first
    bf16x8 b[U][2];
#pragma unroll
    for (int uu = 0; uu < U; ++uu) {
      b[uu][0] = *reinterpret_cast<const bf16x8*>(xr0 + 64 * (st * U + uu));
      b[uu][1] = *reinterpret_cast<const bf16x8*>(xr1 + 64 * (st * U + uu));
    }
#pragma unroll
    for (int uu = 0; uu < U; ++uu)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        acc[t][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[uu][t], b[uu][0], acc[t][0], 0, 0, 0);
        acc[t][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[uu][t], b[uu][1], acc[t][1], 0, 0, 0);
      }
    if (st == nu - 1) {
      // the pair's epilogue: lane (c, j) holds weight rows 4 j .. 4 j + 3 of
      // each tile for batch rows c and 16 + c
      const int ta = t0 + 2 * p;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (ta + t < t1) {
#pragma unroll
          for (int bb = 0; bb < 2; ++bb) {
            const int m = 16 * bb + c;
            if (m < M) {
              uint16_t o4[4];
#pragma unroll
              for (int r = 0; r < 4; ++r) o4[r] = f32_to_bf16_bits(acc[t][bb][r] * inv[bb]);
              *reinterpret_cast<uint64_t*>(out + (int64_t)m * N + (int64_t)(ta + t) * 16 + 4 * j) =
                  *reinterpret_cast<const uint64_t*>(o4);
            }
          }
        }
        acc[t][0] = acc[t][1] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
  };
  // Loads are unconditional (past the last unit they repeat it and are not
  // used), so the compiler's wait counts see one straight sequence: a load
  // under a branch makes every later wait count for it as well.
  // The scheduling barriers keep each unit's loads ahead of the previous
  // unit's products (the scheduler would otherwise sink them between the
  // products, after the waits for the previous unit's data).
  if constexpr (NB == 2) {
    if (total > 0) load(0, a0);
    stage_x();
    for (int u = 0; u < total; u += 2) {
      load(min(u + 1, total - 1), a1);
      __builtin_amdgcn_sched_barrier(0);
      mma(u, a0);
      if (u + 1 >= total) break;
      load(min(u + 2, total - 1), a0);
      __builtin_amdgcn_sched_barrier(0);
      mma(u + 1, a1);
    }
  } else {
    bf16x8 a2[U][2];
    if (total > 0) {
      load(0, a0);
      load(min(1, total - 1), a1);
    }
    stage_x();
    for (int u = 0; u < total; u += 3) {
      load(min(u + 2, total - 1), a2);
      __builtin_amdgcn_sched_barrier(0);
      mma(u, a0);
      if (u + 1 >= total) break;
      load(min(u + 3, total - 1), a0);
      __builtin_amdgcn_sched_barrier(0);
      mma(u + 1, a1);
      if (u + 2 >= total) break;
      load(min(u + 4, total - 1), a1);
      __builtin_amdgcn_sched_barrier(0);
      mma(u + 2, a2);
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
                                                          int N, int K, int rope_d,
                                                          int rope_rows) {
  const int64_t total = (int64_t)N * K / 8;
  const int nsteps = K / 32;
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < total;
       q += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(q & 63);
    const int64_t frag = q >> 6;
    const int64_t tile = frag / nsteps;
    const int step = (int)(frag % nsteps);
    const int64_t row = tile * 16 + (lane & 15);
    // With rope pairs (rope_d = head_dim, the first rope_rows rows being
    // query and key heads): row c of packed tile u of a head is the head's
    // row 8 u + c for c < 8 and D / 2 + 8 u + c - 8 for c >= 8, so a tile
    // holds both members of the rotation pairs 8 u .. 8 u + 7.
    int64_t src_row = row;
    if (row < rope_rows) {
      const int64_t hd = row / rope_d;
      const int u = (int)(row % rope_d) / 16, c = lane & 15;
      src_row = hd * rope_d + (c >> 3) * (rope_d / 2) + 8 * u + (c & 7);
    }
    const int col = step * 32 + 8 * (lane >> 4);
    uint4 v = *reinterpret_cast<const uint4*>(src + src_row * K + col);
    if (col_scale) {
      uint16_t* e = reinterpret_cast<uint16_t*>(&v);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        e[i] = f32_to_bf16_bits(bf16_bits_to_f32(e[i]) * bf16_bits_to_f32(col_scale[col + i]));
    }
    *reinterpret_cast<uint4*>(dst + q * 8) = v;
  }
}


// Greedy token choice over logit rows, argmax_logits's rule
// (crates/traits/src/sampling.rs:439-453): the first index holding the
// largest value; NaN never wins; a row with no value above -inf (or no
// columns) gives 0.  One workgroup of 1024 threads per row.  A thread scans
// its elements in increasing index order keeping the first strict maximum,
// then (value, index) pairs are combined by larger value, ties to the
// smaller index, across the wavefront by lane shuffles and across the
// wavefronts in LDS.  VEC: elements per load (8 bf16 or 4 f32 = 16 bytes,
// when the rows are 16-byte aligned; else 1).
constexpr int kArgmaxThreads = 1024;
template <typename T, int VEC>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(int64_t* __restrict__ out,
                                                                const T* __restrict__ x,
                                                                int cols, int64_t row_stride) {
  const T* row = x + (int64_t)blockIdx.x * row_stride;
  float best = -INFINITY;
  int bi = INT_MAX;
  const int nv = cols / VEC;
  constexpr int UN = 4;  // loads in flight per thread
  for (int v0 = threadIdx.x; v0 < nv; v0 += UN * kArgmaxThreads) {
    float e[UN][VEC];
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const int v = v0 + u * kArgmaxThreads;
      if (v < nv) {
        if constexpr (VEC == 1) {
          e[u][0] = Elem<T>::load(row + v);
        } else {
          typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
          const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row) + v);
          const uint32_t wd[4] = {w[0], w[1], w[2], w[3]};
#pragma unroll
          for (int i = 0; i < VEC; ++i) {
            if constexpr (sizeof(T) == 2)
              e[u][i] = bf16_bits_to_f32((uint16_t)(wd[i / 2] >> (16 * (i & 1))));
            else
              e[u][i] = __uint_as_float(wd[i]);
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) e[u][i] = -INFINITY;
      }
    }
#pragma unroll
    for (int u = 0; u < UN; ++u)
#pragma unroll
      for (int i = 0; i < VEC; ++i)
        if (e[u][i] > best) {
          best = e[u][i];
          bi = (v0 + u * kArgmaxThreads) * VEC + i;
        }
  }
  // columns past the last whole vector (VEC > 1 and cols % VEC != 0 never
  // happens: the host takes VEC = 1 then)
  auto better = [](float v, int i, float bv, int bj) {
    return v > bv || (v == bv && i < bj);
  };
#pragma unroll
  for (int w = 32; w > 0; w >>= 1) {
    const float ov = __shfl_xor(best, w, 64);
    const int oi = __shfl_xor(bi, w, 64);
    if (better(ov, oi, best, bi)) {
      best = ov;
      bi = oi;
    }
  }
  __shared__ float sv[kArgmaxThreads / 64];
  __shared__ int si[kArgmaxThreads / 64];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wave] = best;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kArgmaxThreads / 64; ++w)
      if (better(sv[w], si[w], best, bi)) {
        best = sv[w];
        bi = si[w];
      }
    out[blockIdx.x] = bi == INT_MAX ? 0 : bi;
  }
}


// ---------------------------------------------------------------------------
// Prefill-sized linear layer: Y[M, N] = X[M, K] · W[N, K]ᵀ (bf16, f32
// accumulation) for batches of many rows (prompt chunks), where the
// arithmetic, not the weight stream, bounds the work.
//
// Workgroup = WM x WN wavefronts; wavefront (wm, wn) computes TM x TN tiles
// of 32 x 32 (v_mfma_f32_32x32x16_bf16), so the workgroup tile is
// BM = 32 WM TM rows x BN = 32 WN TN weight rows, K in steps of BK.  Each
// step's X and W tiles are copied HBM -> LDS with global_load_lds (no
// register staging) into one of two buffers, one step ahead of use; the
// grid is persistent (the LDS-resident workgroups of the GPU), and a
// workgroup's steps run as one sequence over its tiles, so the next tile's
// first copy is in flight during a tile's epilogue.
// Operand reads: lane l = 32 g + n takes row n of a 32-row tile, k 8 g ..
// 8 g + 7 of the MFMA's 16 (one 16-byte LDS read, which feeds TN or TM
// MFMAs); the tiles' rows (2 BK bytes) hold their 16-byte k chunks
// XOR-swizzled by the row's position above the rows that share 256 bytes
// (chunk position ch ^ ((r / (256 / 2 BK)) % (BK / 8))), so the 16 rows a
// read serves at once hit 16 distinct bank slots.
// The MFMAs compute the transposed tile (W rows x X rows: A = W, B = X), so
// lane (n, g) holds X row n and, in register r, output column
// 8 (r / 4) + 4 g + r % 4: four consecutive columns per 8-byte store.
// Epilogues (EPI): 0 none; 1 + bias[n]; 2 SwiGLU over a fused gate|up
// weight [2 N, K]: the workgroup's BN weight rows are gate rows a0 ..
// a0 + BN/2 - 1 then the up rows N + a0 .. (a0 = BN/2 x the column tile),
// wavefront wn takes its TN/2 gate tiles and the matching up tiles, and
// out[m][a] = silu(bf16(g)) * bf16(u) (the exponential
// __expf, the reciprocal v_rcp_f32); with add_out the result is added into
// out (out = bf16(out + bf16(y))).  Rows past M read row M - 1, weight rows
// past N (EPI 0 / 1: N need not fill the last tile) read row N - 1, and
// neither is stored.
#ifndef PA_GEMM_BIG_BK
#define PA_GEMM_BIG_BK 64
#define PA_GEMM_BIG_S 2
#define PA_GEMM_SMALL_BK 64
#define PA_GEMM_SMALL_S 2
#endif
constexpr int kSkinnyMaxRows = 64;
// HBM -> LDS copy of 16 bytes per lane (lane l's bytes land at lds + 16 l),
// written out in assembly: with the builtin, the compiler cannot tell that
// the operand reads which follow use the other LDS buffer, and makes them
// wait for the copy (vmcnt(0) right after every copy, so no copy overlapped
// any compute).  The kernel orders copies and reads itself (vmcnt(0) and a
// barrier at the top of every step).
__device__ inline void lds_copy16(const void* src, void* lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(m0)
               : "memory", "m0");
}
// Compute units of the current device (cached per device).
int gemm_compute_units() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}  // pa_linear's skinny kernel up to here
constexpr int kGemmKMultiple = 64;  // K the tiled kernel takes: a multiple of this
constexpr int kGemmGroupM = 4;  // row tiles per group of the tile order
template <int EPI, int WM, int WN, int TM, int TN, int BK, int S>
__global__ __launch_bounds__(64 * WM * WN) void gemm_tiled_kernel(
    uint16_t* __restrict__ out, const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ bias, int M, int N, int K, int add_out, int ntm, int ntn) {
  constexpr int NW = WM * WN;
  constexpr int BM = 32 * WM * TM, BN = 32 * WN * TN;
  static_assert(kGemmKMultiple % BK == 0, "K steps");
  constexpr int RB = BK * 2;           // bytes per tile row
  constexpr int RPC = 1024 / RB;       // rows per 1 KB copy chunk
  constexpr int LPR = RB / 16;         // lanes (16-byte chunks) per row
  constexpr int CA = BM / RPC / NW, CB = BN / RPC / NW;  // copy chunks per wavefront
  static_assert(CA * NW * RPC == BM && CB * NW * RPC == BN && (EPI != 2 || TN % 2 == 0),
                "tiles");
  __shared__ __attribute__((aligned(1024))) uint8_t lds_a[S][BM * RB];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_b[S][BN * RB];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int n = lane & 31, g = lane >> 5;
  // Persistent grid, tile order: workgroups are dealt round-robin to the 8
  // XCDs; XCD x takes the contiguous range [x per_xcd, (x + 1) per_xcd) of
  // the logical order, its workgroups (slots) taking every nslot-th tile of
  // it, so the tiles in flight on an XCD are neighbours in the order.  The
  // order goes through groups of kGemmGroupM row tiles, column tiles outer
  // within a group, so those workgroups share X rows and W rows in the
  // XCD's L2.
  const int total = ntm * ntn, per_xcd = (total + 7) / 8;
  const int xcd = (int)(blockIdx.x % 8), slot = (int)(blockIdx.x / 8);
  const int nslot = (int)(gridDim.x / 8);
  const int lo = xcd * per_xcd, hi = min(total, lo + per_xcd);
  if (lo + slot >= hi) return;
  const int my_tiles = (hi - 1 - lo - slot) / nslot + 1;
  auto tile_origin = [&](int i, int& m0, int& c0) __attribute__((always_inline)) {
    const int L = lo + slot + i * nslot;
    const int grp = L / (kGemmGroupM * ntn), first_m = grp * kGemmGroupM;
    const int gsz = min(kGemmGroupM, ntm - first_m);
    const int r = L % (kGemmGroupM * ntn);
    m0 = (first_m + r % gsz) * BM;
    c0 = (r / gsz) * (EPI == 2 ? BN / 2 : BN);  // first output column
  };
  auto swz = [](int r) -> int { return (r / (256 / RB)) % LPR; };
  // this wavefront's copies: RPC rows per 1 KB chunk; lane l fills chunk
  // position l % LPR of row l / LPR, i.e. source chunk (l % LPR) ^ swz(row)
  int xr[CA], wr[CB], xch[CA], wch[CB];
#pragma unroll
  for (int i = 0; i < CA; ++i) {
    xr[i] = (CA * wave + i) * RPC + lane / LPR;
    xch[i] = ((lane % LPR) ^ swz(xr[i])) * 8;
  }
#pragma unroll
  for (int i = 0; i < CB; ++i) {
    wr[i] = (CB * wave + i) * RPC + lane / LPR;
    wch[i] = ((lane % LPR) ^ swz(wr[i])) * 8;
  }
  // copies of step kt of the tile whose source rows are xs / ws into
  // buffer BUF; the rows change only per tile (set_sources)
  const uint16_t* xs[CA];
  const uint16_t* ws[CB];
  auto set_sources = [&](int i) __attribute__((always_inline)) {
    int m0, c0;
    tile_origin(i, m0, c0);
#pragma unroll
    for (int u = 0; u < CA; ++u) xs[u] = x + (int64_t)min(m0 + xr[u], M - 1) * K + xch[u];
#pragma unroll
    for (int u = 0; u < CB; ++u) {
      const int r = wr[u];
      const int row = EPI == 2 ? (r < BN / 2 ? c0 + r : N + c0 + r - BN / 2) : min(c0 + r, N - 1);
      ws[u] = w + (int64_t)row * K + wch[u];
    }
  };
  auto issue = [&](int kt, int buf) __attribute__((always_inline)) {
    uint8_t* la = lds_a[buf];
    uint8_t* lb = lds_b[buf];
#pragma unroll
    for (int u = 0; u < CA; ++u)
      lds_copy16(xs[u] + kt * BK, &la[(CA * wave + u) * 1024]);
#pragma unroll
    for (int u = 0; u < CB; ++u)
      lds_copy16(ws[u] + kt * BK, &lb[(CB * wave + u) * 1024]);
  };
  // LDS rows of this wavefront's operand tiles (SwiGLU: gate tiles, then
  // the matching up tiles)
  int arow[TM], brow[TN];
#pragma unroll
  for (int t = 0; t < TM; ++t) arow[t] = (wm * TM + t) * 32 + n;
#pragma unroll
  for (int t = 0; t < TN; ++t)
    brow[t] = EPI == 2 ? (t < TN / 2 ? (wn * TN / 2 + t) * 32 + n
                                     : BN / 2 + (wn * TN / 2 + t - TN / 2) * 32 + n)
                       : (wn * TN + t) * 32 + n;
  f32x16 acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.f;
  // epilogue of the tile at (m0, c0)
  auto store_tile = [&](int m0, int c0) __attribute__((always_inline)) {
  // epilogue: acc[a][b] is the transposed tile (W rows x X rows), so lane
  // (n, g) holds X row n and, in registers 4 q .. 4 q + 3, the four
  // consecutive output columns 8 q + 4 g .. 8 q + 4 g + 3 (one 8-byte store)
  const bool vec = N % 4 == 0;
#pragma unroll
  for (int a = 0; a < TM; ++a) {
    const int row = m0 + (wm * TM + a) * 32 + n;
    if (row >= M) continue;
    uint16_t* orow = out + (int64_t)row * N;
    if constexpr (EPI == 2) {
#pragma unroll
      for (int b = 0; b < TN / 2; ++b)
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          const int col = c0 + (wn * TN / 2 + b) * 32 + 8 * qd + 4 * g;
          uint16_t v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float gg = (float)(__bf16)acc[a][b][4 * qd + e];
            const float uu = (float)(__bf16)acc[a][b + TN / 2][4 * qd + e];
            v[e] = __builtin_bit_cast(
                uint16_t, (__bf16)(gg * __builtin_amdgcn_rcpf(1.0f + __expf(-gg)) * uu));
          }
          *reinterpret_cast<uint64_t*>(orow + col) = *reinterpret_cast<const uint64_t*>(v);
        }
    } else {
      // every load of the epilogue is issued before any of its values is
      // used (bias once for the tile, the residual row's values per row),
      // so the round trips overlap instead of following one another
      float bv[TN][4][4];
#pragma unroll
      for (int b = 0; b < TN; ++b)
#pragma unroll
        for (int qd = 0; qd < 4; ++qd)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int col = c0 + (wn * TN + b) * 32 + 8 * qd + 4 * g + e;
            bv[b][qd][e] = EPI == 1 ? bf16_bits_to_f32(bias[min(col, N - 1)]) : 0.f;
          }
      uint64_t ow[TN][4];
      if (add_out && vec) {
#pragma unroll
        for (int b = 0; b < TN; ++b)
#pragma unroll
          for (int qd = 0; qd < 4; ++qd) {
            const int col = c0 + (wn * TN + b) * 32 + 8 * qd + 4 * g;
            ow[b][qd] = col < N ? *reinterpret_cast<const uint64_t*>(orow + col) : 0;
          }
      }
#pragma unroll
      for (int b = 0; b < TN; ++b)
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          const int col = c0 + (wn * TN + b) * 32 + 8 * qd + 4 * g;
          if (col >= N) continue;
          float y[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) y[e] = acc[a][b][4 * qd + e] + bv[b][qd][e];
          if (vec) {
            uint16_t v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float t = y[e];
              if (add_out)
                t = bf16_bits_to_f32((uint16_t)(ow[b][qd] >> (16 * e))) +
                    bf16_bits_to_f32(f32_to_bf16_bits(t));
              v[e] = f32_to_bf16_bits(t);
            }
            *reinterpret_cast<uint64_t*>(orow + col) = *reinterpret_cast<const uint64_t*>(v);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if (col + e >= N) continue;
              float t = y[e];
              if (add_out) t = bf16_bits_to_f32(orow[col + e]) + bf16_bits_to_f32(f32_to_bf16_bits(t));
              orow[col + e] = f32_to_bf16_bits(t);
            }
          }
        }
    }
  }
  };
  // The workgroup's steps run as one sequence over its tiles (step gs =
  // step gs % nk of tile gs / nk, in buffer gs % 2), the copy of step gs + 1
  // issued before step gs is computed -- across tile boundaries too, so the
  // next tile's first copy is in flight during the epilogue.
  const int nk = K / BK, nsteps = my_tiles * nk;
  // Copies run S - 1 steps ahead: before step gs computes, the copies of
  // steps gs + 1 .. gs + S - 2 may still be in flight (CA + CB loads each).
  constexpr int PER = CA + CB;
  static_assert(PER * (S - 2) <= 63 && S >= 2 && S <= 4, "vmcnt range");
  int cur = 0;      // tile of the step being computed
  int iss = 0;      // next step to copy, and its tile / step within the tile
  int iss_tile = 0, iss_kt = 0;
  set_sources(0);
  auto issue_next = [&]() __attribute__((always_inline)) {
    if (iss_kt == nk) {  // the step starts the next tile
      ++iss_tile;
      iss_kt = 0;
      set_sources(iss_tile);
    }
    issue(iss_kt, iss % S);
    ++iss;
    ++iss_kt;
  };
  for (int t = 0; t < S - 1 && t < nsteps; ++t) issue_next();
  for (int gs = 0; gs < nsteps; ++gs) {
    const int kt = gs - cur * nk;
    const int ahead = iss - 1 - gs;  // copies of later steps in flight
    if (ahead >= 2)
      __builtin_amdgcn_s_waitcnt(0x0F70 | ((2 * PER) & 0xF) | (((2 * PER) >> 4) << 14));
    else if (ahead == 1)
      __builtin_amdgcn_s_waitcnt(0x0F70 | (PER & 0xF) | ((PER >> 4) << 14));
    else
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    // step gs has landed for every wavefront, and every wavefront is done
    // with step gs - 1's buffer, which the next copy reuses
    __syncthreads();
    if (iss < nsteps) issue_next();
    const uint8_t* at = lds_a[gs % S];
    const uint8_t* bt = lds_b[gs % S];
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      bf16x8 af[TM], bfr[TN];
#pragma unroll
      for (int t = 0; t < TM; ++t)
        af[t] = *reinterpret_cast<const bf16x8*>(at + arow[t] * RB +
                                                 (((2 * s + g) ^ swz(arow[t])) * 16));
#pragma unroll
      for (int t = 0; t < TN; ++t)
        bfr[t] = *reinterpret_cast<const bf16x8*>(bt + brow[t] * RB +
                                                  (((2 * s + g) ^ swz(brow[t])) * 16));
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[b], af[a], acc[a][b], 0, 0, 0);
    }
    if (kt == nk - 1) {
      int m0, c0;
      tile_origin(cur, m0, c0);
      store_tile(m0, c0);
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
#pragma unroll
          for (int q = 0; q < 16; ++q) acc[a][b][q] = 0.f;
      ++cur;
    }
  }
}

}  // namespace
}  // namespace pa

using namespace pa;

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

extern "C" int32_t pa_rms_norm(void* out, void* residual, const void* add, const void* weight,
                               int32_t rows, int32_t hidden, float eps, int32_t dtype,
                               pa_stream_t stream) {
  clear_error();
  PA_REQUIRE(dtype_ok(dtype), PA_ERR_INVALID_ARG, "pa_rms_norm: unknown dtype %d", dtype);
  PA_REQUIRE(rows >= 0 && hidden > 0, PA_ERR_INVALID_ARG, "pa_rms_norm: bad sizes");
  if (rows == 0) return PA_OK;
  PA_REQUIRE(out && residual && weight, PA_ERR_INVALID_ARG, "pa_rms_norm: null pointer");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == PA_DTYPE_BF16 && hidden % 8 == 0 && hidden <= 64 * 8 * kNormChunks &&
      aligned16(out) && aligned16(residual) && (!add || aligned16(add)) && aligned16(weight))
    rms_norm_rows_kernel<<<(rows + 3) / 4, 256, 0, s>>>((uint16_t*)out, (uint16_t*)residual,
                                                        (const uint16_t*)add,
                                                        (const uint16_t*)weight, rows, hidden, eps);
  else if (dtype == PA_DTYPE_BF16)
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

namespace {
// Launch shape of pa_linear.
//   nt: weight tiles per wavefront: 4 for wide outputs (each X fragment then
//       feeds 4 tiles), 1 where 2 would leave fewer than ~512 wavefronts,
//       else 2.
//   splits: workgroups sharing a tile's K range (needs the workspace): for
//       long K (>= 2048) and fewer than 128 tiles, enough to give ~256
//       workgroups, at most 8 and at least 16 steps each.
//   kw: wavefronts per workgroup splitting its K range: NT = 1 runs up to 16,
//       with one stage of 8 steps when the range is short and stages of 4
//       otherwise; NT > 1 up to 8 wavefronts of about 8 steps (two stages of 4).
// Plans split K only for at most kMaxSplitTiles output tiles; their counters
// fill the workspace's first kSplitCounterBytes.
constexpr int kMaxSplitTiles = 127;
constexpr size_t kSplitCounterBytes = 512;
static_assert(kMaxSplitTiles * sizeof(int) <= kSplitCounterBytes, "counter region");
struct LinearPlan {
  int nt, kw, stage, splits;
  dim3 grid;
};
LinearPlan linear_plan(int rows, int n, int k, int act, bool can_split) {
  LinearPlan p{2, 1, 4, 1, dim3(1)};
  const int nsteps = k / 32;
  const int kw0 = std::max(1, std::min(8, (nsteps + 7) / 8));
  if (act != PA_ACT_SILU_MUL) {
    if ((n + 63) / 64 >= 1024) p.nt = 4;
    else if ((long long)((n + 31) / 32) * kw0 < 512) p.nt = 1;
  }
  const int cols = act == PA_ACT_SILU_MUL ? 16 : 16 * p.nt;
  const long long tiles = (long long)((n + cols - 1) / cols) * ((rows + 31) / 32);
  if (can_split && nsteps >= 64 && tiles <= kMaxSplitTiles)
    p.splits = (int)std::max(1LL, std::min({8LL, 256 / tiles, (long long)nsteps / 16}));
  const int steps = (nsteps + p.splits - 1) / p.splits;  // per workgroup
  p.kw = std::max(1, std::min(8, (steps + 7) / 8));
  if (p.nt == 1) {
    if (steps <= 64)
      p.stage = 8;
    else
      p.kw = std::min(16, (steps + 7) / 8);
  }
  p.grid = dim3((n + cols - 1) / cols, (rows + 31) / 32, p.splits);
  return p;
}
// Workspace of a split plan: a counter region of fixed size (one int per
// tile for the largest tile count that splits), then one record per (tile,
// split) of 2 NT x 64 partial f32x4 plus 32 sums of squares.  The counter
// region does not depend on the plan, so one workspace serves calls of
// different shapes in any order: every counter is back at zero after a call.
size_t linear_ws_bytes(const LinearPlan& p) {
  if (p.splits <= 1) return 0;
  const size_t tiles = (size_t)p.grid.x * p.grid.y;
  return kSplitCounterBytes + tiles * p.splits * (2 * p.nt * 256 + 32) * sizeof(float);
}
}  // namespace

extern "C" size_t pa_linear_workspace_size(int32_t rows, int32_t out_features,
                                           int32_t in_features, int32_t act) {
  if (rows <= 0 || out_features <= 0 || in_features < 32) return 0;
  return linear_ws_bytes(linear_plan(rows, out_features, in_features, act, true));
}

extern "C" int32_t pa_linear(void* out, const void* x, const void* weight, const void* bias,
                             int32_t rows, int32_t out_features, int32_t in_features, int32_t act,
                             int32_t packed, int32_t flags, float eps, void* workspace,
                             size_t workspace_bytes, int32_t dtype, pa_stream_t stream) {
  clear_error();
  PA_REQUIRE(dtype == PA_DTYPE_BF16, PA_ERR_UNSUPPORTED, "pa_linear: dtype %d (bf16 only)", dtype);
  PA_REQUIRE(act == PA_ACT_NONE || act == PA_ACT_SILU_MUL, PA_ERR_INVALID_ARG,
             "pa_linear: unknown activation %d", act);
  PA_REQUIRE(rows >= 0 && out_features > 0 && in_features > 0, PA_ERR_INVALID_ARG,
             "pa_linear: bad sizes");
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
  // Batches of many rows (prompt chunks), and output widths the skinny
  // kernel's 16-row tiles do not divide: the tiled GEMM over row-major
  // weights, when K fits its steps (and the SwiGLU width its 64 columns).
  const bool tiled = !packed && !(flags & PA_LINEAR_RMS_IN) && in_features % kGemmKMultiple == 0 &&
                     (act != PA_ACT_SILU_MUL || out_features % 64 == 0) &&
                     (rows > kSkinnyMaxRows || out_features % 16 != 0);
  PA_REQUIRE(tiled || in_features % 32 == 0, PA_ERR_UNSUPPORTED,
             "pa_linear: in_features %d not a multiple of 32", in_features);
  PA_REQUIRE(tiled || out_features % 16 == 0, PA_ERR_UNSUPPORTED,
             "pa_linear: out_features %d not a multiple of 16", out_features);
  if (tiled) {
    // Large outputs: 256 x 256 workgroup tiles (8 wavefronts of 64 x 128:
    // each operand read feeds 4 or 2 MFMAs); otherwise 128 x 128 (4
    // wavefronts of 64 x 64), which keeps small projections spread over
    // more workgroups.
    hipStream_t s = (hipStream_t)stream;
    const int add = (flags & PA_LINEAR_ADD_OUT) ? 1 : 0;
    auto* o = (uint16_t*)out;
    auto* xx = (const uint16_t*)x;
    auto* ww = (const uint16_t*)weight;
    auto* bb = (const uint16_t*)bias;
    const int wcols = act == PA_ACT_SILU_MUL ? 2 * out_features : out_features;
    const bool big = (long long)((rows + 255) / 256) * ((wcols + 255) / 256) >= 256 &&
                     (act != PA_ACT_SILU_MUL || out_features % 128 == 0);
    auto launch = [&](auto wmc, auto wnc, auto tmc, auto tnc) -> int32_t {
      constexpr int WM_ = decltype(wmc)::value, WN_ = decltype(wnc)::value;
      constexpr int TM_ = decltype(tmc)::value, TN_ = decltype(tnc)::value;
      // K steps of 64 through two LDS buffers (measured at the config-5
      // shapes against steps of 32 through 2, 3 or 4 buffers: equal for the
      // 256 x 256 tiles, 28.6 vs 33.6-36.4 us for the 128 x 128 ones)
      constexpr int BK_ = WM_ * WN_ == 8 ? PA_GEMM_BIG_BK : PA_GEMM_SMALL_BK;
      constexpr int S_ = WM_ * WN_ == 8 ? PA_GEMM_BIG_S : PA_GEMM_SMALL_S;
      constexpr int WPC = WM_ * WN_ == 8 ? 1 : 2;  // workgroups per CU (LDS)
      static_assert(WPC == 1 || WPC == 2, "");
      constexpr int BM_ = 32 * WM_ * TM_, BN_ = 32 * WN_ * TN_;
      const int ntn = act == PA_ACT_SILU_MUL ? out_features / (BN_ / 2)
                                             : (out_features + BN_ - 1) / BN_;
      const int ntm = (rows + BM_ - 1) / BM_;
      PA_REQUIRE((long long)ntm * ntn < (1ll << 30), PA_ERR_UNSUPPORTED, "pa_linear: %d rows",
                 rows);
      const int per_xcd = (ntm * ntn + 7) / 8;
      // persistent for the large tiles (one workgroup per CU: its next
      // tile's first copy overlaps the epilogue); a workgroup per tile for
      // the small ones (two per CU: one's epilogue overlaps the other's loop)
      const dim3 grid(8 * (WPC == 1 ? std::max(1, std::min(per_xcd, gemm_compute_units() / 8))
                                    : per_xcd));
      if (act == PA_ACT_SILU_MUL)
        gemm_tiled_kernel<2, WM_, WN_, TM_, TN_, BK_, S_><<<grid, 64 * WM_ * WN_, 0, s>>>(
            o, xx, ww, nullptr, rows, out_features, in_features, 0, ntm, ntn);
      else if (bias)
        gemm_tiled_kernel<1, WM_, WN_, TM_, TN_, BK_, S_><<<grid, 64 * WM_ * WN_, 0, s>>>(
            o, xx, ww, bb, rows, out_features, in_features, add, ntm, ntn);
      else
        gemm_tiled_kernel<0, WM_, WN_, TM_, TN_, BK_, S_><<<grid, 64 * WM_ * WN_, 0, s>>>(
            o, xx, ww, nullptr, rows, out_features, in_features, add, ntm, ntn);
      return PA_OK;
    };
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I4 = std::integral_constant<int, 4>;
    const int32_t rc = big ? launch(I4{}, I2{}, I2{}, I4{}) : launch(I2{}, I2{}, I2{}, I2{});
    if (rc != PA_OK) return rc;
    return check_launch("pa_linear");
  }
  PA_REQUIRE((rows + 31) / 32 <= 65535, PA_ERR_UNSUPPORTED, "pa_linear: %d rows", rows);
  // A wide projection of one batch tile over packed weights (the LM head):
  // the batch rows in LDS, a persistent grid of two workgroups per CU.
  if (packed && rows <= 32 && act == PA_ACT_NONE && !bias && !(flags & PA_LINEAR_ADD_OUT) &&
      out_features / 16 >= kWideMinTiles && in_features <= kWideMaxK) {
    const size_t lds = 32 * (2 * (size_t)in_features + 16) + 32 * sizeof(float);
    const int nsteps = in_features / 32;
    // one 8-wavefront workgroup per CU (X staged once per CU); units of 7
    // K steps (U divides the steps) through two register buffers, or of 4,
    // 2 or 1 through three (the LM head back to back: 55-56 us; two
    // 4-wavefront workgroups per CU 57-58 us; three buffers of 7 steps 58)
    auto launch_wide = [&](auto uc, auto nbc) {
      const int grid = std::min(gemm_compute_units(), (out_features / 16 + 7) / 8);
      linear_wide_kernel<decltype(uc)::value, decltype(nbc)::value, 8>
          <<<grid, 512, lds, (hipStream_t)stream>>>(
          (uint16_t*)out, (const uint16_t*)x, (const uint16_t*)weight, rows, out_features,
          in_features, flags, eps);
    };
    using std::integral_constant;
    if (nsteps % 7 == 0)
      launch_wide(integral_constant<int, 7>{}, integral_constant<int, 2>{});
    else if (nsteps % 4 == 0)
      launch_wide(integral_constant<int, 4>{}, integral_constant<int, 3>{});
    else if (nsteps % 2 == 0)
      launch_wide(integral_constant<int, 2>{}, integral_constant<int, 3>{});
    else
      launch_wide(integral_constant<int, 1>{}, integral_constant<int, 3>{});
    return check_launch("pa_linear");
  }
  // The split plan when the workspace holds it, else one workgroup per tile.
  LinearPlan plan = linear_plan(rows, out_features, in_features, act, true);
  const size_t ws_need = linear_ws_bytes(plan);
  if (ws_need == 0 || !workspace || workspace_bytes < ws_need)
    plan = linear_plan(rows, out_features, in_features, act, false);
  else
    PA_REQUIRE((uintptr_t)workspace % 256 == 0, PA_ERR_INVALID_ARG,
               "pa_linear: workspace must be 256-byte aligned");
  const int nt = plan.nt, kw = plan.kw, stage = plan.stage;
  const dim3 grid = plan.grid;
  int* counters = (int*)workspace;
  float* ws = plan.splits > 1 ? (float*)((char*)workspace + kSplitCounterBytes) : nullptr;
  hipStream_t s = (hipStream_t)stream;
  auto* o = (uint16_t*)out;
  auto* xx = (const uint16_t*)x;
  auto* ww = (const uint16_t*)weight;
  auto* bb = (const uint16_t*)bias;
#define PA_LAUNCH_LINEAR_U(EPI, NT, UU)                                                       \
  (packed ? linear_skinny_kernel<EPI, NT, true, UU><<<grid, 64 * kw, 0, s>>>(                  \
                o, xx, ww, bb, rows, out_features, in_features, kw, flags, eps, ws, counters,  \
                RopeCacheArgs{})                                                              \
          : linear_skinny_kernel<EPI, NT, false, UU><<<grid, 64 * kw, 0, s>>>(                 \
                o, xx, ww, bb, rows, out_features, in_features, kw, flags, eps, ws, counters,  \
                RopeCacheArgs{}))
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
      (uint16_t*)packed, (const uint16_t*)weight, (const uint16_t*)col_scale, rows, cols, 1, 0);
  return check_launch("pa_linear_pack");
}

extern "C" int32_t pa_linear_pack_qkv(void* packed, const void* weight, const void* col_scale,
                                      int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                      int32_t cols, int32_t dtype, pa_stream_t stream) {
  clear_error();
  PA_REQUIRE(dtype == PA_DTYPE_BF16, PA_ERR_UNSUPPORTED,
             "pa_linear_pack_qkv: dtype %d (bf16 only)", dtype);
  PA_REQUIRE(num_heads > 0 && num_kv_heads > 0 && head_dim > 0 && cols > 0, PA_ERR_INVALID_ARG,
             "pa_linear_pack_qkv: bad sizes");
  PA_REQUIRE(head_dim % 32 == 0 && cols % 32 == 0, PA_ERR_UNSUPPORTED,
             "pa_linear_pack_qkv: head_dim %d and cols %d must be multiples of 32", head_dim,
             cols);
  PA_REQUIRE(packed && weight && packed != weight, PA_ERR_INVALID_ARG,
             "pa_linear_pack_qkv: null or aliased pointers");
  PA_REQUIRE(((uintptr_t)packed | (uintptr_t)weight) % 16 == 0, PA_ERR_INVALID_ARG,
             "pa_linear_pack_qkv: pointers must be 16-byte aligned");
  const int rows = (num_heads + 2 * num_kv_heads) * head_dim;
  const int64_t pieces = (int64_t)rows * cols / 8;
  const int blocks = (int)std::min<int64_t>((pieces + 255) / 256, 65536);
  linear_pack_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>(
      (uint16_t*)packed, (const uint16_t*)weight, (const uint16_t*)col_scale, rows, cols,
      head_dim, (num_heads + num_kv_heads) * head_dim);
  return check_launch("pa_linear_pack_qkv");
}

extern "C" int32_t pa_argmax(int64_t* out, const void* logits, int32_t rows, int32_t cols,
                             int64_t row_stride, int32_t dtype, pa_stream_t stream) {
  clear_error();
  PA_REQUIRE(dtype_ok(dtype), PA_ERR_INVALID_ARG, "pa_argmax: unknown dtype %d", dtype);
  PA_REQUIRE(rows >= 0 && cols >= 0, PA_ERR_INVALID_ARG, "pa_argmax: bad sizes");
  if (row_stride == 0) row_stride = cols;
  PA_REQUIRE(row_stride >= cols, PA_ERR_INVALID_ARG,
             "pa_argmax: row stride %lld below cols %d", (long long)row_stride, cols);
  if (rows == 0) return PA_OK;
  PA_REQUIRE(out && (logits || cols == 0), PA_ERR_INVALID_ARG, "pa_argmax: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const int esz = dtype == PA_DTYPE_BF16 ? 2 : 4;
  const bool vec = (uintptr_t)logits % 16 == 0 && (row_stride * esz) % 16 == 0 &&
                   (cols * esz) % 16 == 0;
  if (dtype == PA_DTYPE_BF16) {
    if (vec)
      argmax_kernel<uint16_t, 8><<<rows, kArgmaxThreads, 0, s>>>(out, (const uint16_t*)logits,
                                                                 cols, row_stride);
    else
      argmax_kernel<uint16_t, 1><<<rows, kArgmaxThreads, 0, s>>>(out, (const uint16_t*)logits,
                                                                 cols, row_stride);
  } else {
    if (vec)
      argmax_kernel<float, 4><<<rows, kArgmaxThreads, 0, s>>>(out, (const float*)logits, cols,
                                                              row_stride);
    else
      argmax_kernel<float, 1><<<rows, kArgmaxThreads, 0, s>>>(out, (const float*)logits, cols,
                                                              row_stride);
  }
  return check_launch("pa_argmax");
}

extern "C" int32_t pa_linear_rope_cache(void* out, const void* x, const void* weight,
                                        const void* bias, int32_t rows, int32_t num_heads,
                                        int32_t num_kv_heads, int32_t head_dim,
                                        int32_t in_features, int32_t flags, float eps,
                                        const int64_t* positions, const int64_t* slot_mapping,
                                        const float* inv_freq, void* k_cache, void* v_cache,
                                        int32_t num_blocks, int32_t dtype, pa_stream_t stream) {
  clear_error();
  PA_REQUIRE(dtype == PA_DTYPE_BF16, PA_ERR_UNSUPPORTED,
             "pa_linear_rope_cache: dtype %d (bf16 only)", dtype);
  PA_REQUIRE(rows >= 0 && num_heads > 0 && num_kv_heads > 0 && head_dim > 0 &&
                 in_features > 0 && num_blocks > 0,
             PA_ERR_INVALID_ARG, "pa_linear_rope_cache: bad sizes");
  PA_REQUIRE(head_dim % 32 == 0 && in_features % 32 == 0, PA_ERR_UNSUPPORTED,
             "pa_linear_rope_cache: head_dim %d and in_features %d must be multiples of 32",
             head_dim, in_features);
  PA_REQUIRE((flags & ~PA_LINEAR_RMS_IN) == 0, PA_ERR_INVALID_ARG,
             "pa_linear_rope_cache: flags %d (only PA_LINEAR_RMS_IN)", flags);
  PA_REQUIRE(!(flags & PA_LINEAR_RMS_IN) || eps > 0.f, PA_ERR_INVALID_ARG,
             "pa_linear_rope_cache: eps must be positive");
  if (rows == 0) return PA_OK;
  PA_REQUIRE(out && x && weight && positions && slot_mapping && inv_freq && k_cache && v_cache,
             PA_ERR_INVALID_ARG, "pa_linear_rope_cache: null pointer");
  PA_REQUIRE(((uintptr_t)x | (uintptr_t)weight | (uintptr_t)out | (uintptr_t)k_cache) % 16 == 0,
             PA_ERR_INVALID_ARG, "pa_linear_rope_cache: x, weight, out and k_cache must be "
             "16-byte aligned");
  PA_REQUIRE((rows + 31) / 32 <= 65535, PA_ERR_UNSUPPORTED, "pa_linear_rope_cache: %d rows",
             rows);
  const int n = (num_heads + 2 * num_kv_heads) * head_dim;
  // K split over the wavefronts as pa_linear splits it for this shape (up
  // to the 8 wavefronts this instance launches with), so the f32 sums, and
  // so the bf16 outputs, are those of pa_linear
  // K split over the wavefronts as pa_linear splits it for this shape (the
  // same instance size), so the f32 sums, and so the bf16 outputs, are
  // those of pa_linear
  const LinearPlan lp = linear_plan(rows, n, in_features, PA_ACT_NONE, false);
  const int kw = lp.kw;
  const RopeCacheArgs ra{positions, slot_mapping, inv_freq, (uint16_t*)k_cache,
                         (uint16_t*)v_cache, (int64_t)num_blocks * kBlock, num_heads,
                         num_kv_heads, head_dim};
  const dim3 grid(n / 16, (rows + 31) / 32);
  if (lp.stage == 8)
    linear_skinny_kernel<3, 1, true, 8><<<grid, 64 * kw, 0, (hipStream_t)stream>>>(
        (uint16_t*)out, (const uint16_t*)x, (const uint16_t*)weight, (const uint16_t*)bias, rows,
        n, in_features, kw, flags, eps, nullptr, nullptr, ra);
  else
    linear_skinny_kernel<3, 1, true, 4><<<grid, 64 * kw, 0, (hipStream_t)stream>>>(
        (uint16_t*)out, (const uint16_t*)x, (const uint16_t*)weight, (const uint16_t*)bias, rows,
        n, in_features, kw, flags, eps, nullptr, nullptr, ra);
  return check_launch("pa_linear_rope_cache");
}
