// int8-in-f32 per-block quantised caches: the reference's PagedKvCache with
// quantized = true (crates/model/src/paged_tensor/tensor_store/buffer.rs:
// 170-231 for the write, :320-331 for the read, mod.rs:69 for the initial
// scale 1.0).  The caches stay f32 (one integer value per element) with one
// scale per block; a write re-quantises the whole block, so tokens that
// land in the same block are applied in order by one workgroup.
#include "pa_common.hpp"
#include "pa_internal.hpp"

namespace pa {
namespace {

// One workgroup per block task: block task_block[w] receives tokens
// tok[i] at offsets off[i] for i in [task_beg[w], task_beg[w + 1]), in order.
// hashes (optional): hashes[tok[i]] = the block hash after token tok[i].
// Per token, as write_kv: every element of the block is dequantised with the
// block's current scale (x * s), the token's K / V rows are stored raw, the
// new scale is max(max|K|, max|V|) / 127 (1 for an all-zero block) and every
// element becomes round(x / scale) (half away from zero).
__global__ __launch_bounds__(256) void quant_write_kernel(
    float* __restrict__ kc, float* __restrict__ vc, float* __restrict__ scales,
    const float* __restrict__ k, const float* __restrict__ v, int H, int D,
    const int32_t* __restrict__ task_block, const int32_t* __restrict__ task_beg,
    const int32_t* __restrict__ tok, const int32_t* __restrict__ off,
    uint64_t* __restrict__ hashes) {
  __shared__ float red[256];
  __shared__ uint64_t hred[256];
  const int w = blockIdx.x, tid = threadIdx.x;
  const int64_t blk = task_block[w];
  const int n = H * kBlock * D;
  float* kb = kc + blk * n;
  float* vb = vc + blk * n;  // token-minor: element (h, d, slot)
  float s = scales[blk];
  for (int i = task_beg[w]; i < task_beg[w + 1]; ++i) {
    const int t = tok[i], o = off[i];
    float mx = 0.f;
    for (int e = tid; e < n; e += blockDim.x) {
      const int h = e / (kBlock * D), r = e % (kBlock * D);
      const float kx = (r / D == o) ? k[((int64_t)t * H + h) * D + r % D] : kb[e] * s;
      const int vd = (e / kBlock) % D;
      const float vx = (e % kBlock == o) ? v[((int64_t)t * H + h) * D + vd] : vb[e] * s;
      kb[e] = kx;
      vb[e] = vx;
      mx = fmaxf(mx, fmaxf(fabsf(kx), fabsf(vx)));
    }
    red[tid] = mx;
    __syncthreads();
    for (int st = blockDim.x / 2; st > 0; st >>= 1) {
      if (tid < st) red[tid] = fmaxf(red[tid], red[tid + st]);
      __syncthreads();
    }
    const float m = red[0];
    const float sc = m > 0.f ? m / 127.0f : 1.0f;
    for (int e = tid; e < n; e += blockDim.x) {
      kb[e] = roundf(kb[e] / sc);
      vb[e] = roundf(vb[e] / sc);
    }
    s = sc;
    __syncthreads();  // red[] is reused by the next token
    // the block hash of the stored (quantised) K after this token
    // (buffer.rs:263-264), when asked for
    if (hashes) {
      const uint64_t h = workgroup_block_hash(n, [&](int e) { return kb[e]; }, hred);
      if (tid == 0) hashes[t] = h;
    }
  }
  if (tid == 0) scales[blk] = s;
}

// Dequantising gather: x * scale + 0.0 (candle's affine), f32.
__global__ __launch_bounds__(256) void quant_read_kernel(const float* __restrict__ kc,
                                                         const float* __restrict__ vc,
                                                         const float* __restrict__ scales,
                                                         const int32_t* __restrict__ block_ids,
                                                         int H, int D, float* __restrict__ out_k,
                                                         float* __restrict__ out_v) {
  const int t = blockIdx.x;
  const int32_t blk = block_ids[t / kBlock];
  const int slot = t % kBlock;
  const float s = scales[blk];
  for (int i = threadIdx.x; i < H * D; i += blockDim.x) {
    const int h = i / D, d = i % D;
    const float kx = kc[(((int64_t)blk * H + h) * kBlock + slot) * D + d];
    const float vx = vc[(((int64_t)blk * H + h) * D + d) * kBlock + slot];
    out_k[(int64_t)t * H * D + i] = kx * s + 0.0f;
    out_v[(int64_t)t * H * D + i] = vx * s + 0.0f;
  }
}

}  // namespace

int32_t launch_quant_write(float* k_cache, float* v_cache, float* scales, const float* k,
                           const float* v, int H, int D, int num_tasks, const int32_t* task_block,
                           const int32_t* task_beg, const int32_t* tok, const int32_t* off,
                           uint64_t* hashes, hipStream_t stream) {
  if (num_tasks == 0) return PA_OK;
  quant_write_kernel<<<num_tasks, 256, 0, stream>>>(k_cache, v_cache, scales, k, v, H, D,
                                                    task_block, task_beg, tok, off, hashes);
  return check_launch("quantised write_kv");
}

int32_t launch_quant_read(const float* k_cache, const float* v_cache, const float* scales,
                          const int32_t* block_ids, int seq_len, int H, int D, float* out_k,
                          float* out_v, hipStream_t stream) {
  if (seq_len == 0) return PA_OK;
  quant_read_kernel<<<seq_len, 256, 0, stream>>>(k_cache, v_cache, scales, block_ids, H, D, out_k,
                                                 out_v);
  return check_launch("quantised read_kv");
}

}  // namespace pa
