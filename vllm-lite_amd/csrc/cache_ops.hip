// KV-cache write / read kernels and their C entry points:
// pa_reshape_and_cache, pa_slot_mapping, pa_read_kv, pa_block_hash.
//
// These are HBM-bound copies.  A token's K row for one head is D contiguous
// elements in both source and cache; its V row is scattered into the
// token-minor V block ([D, 16] per head), one element per 32 B (bf16) or
// 64 B (f32) row of the block.
#include <type_traits>

#include "pa_common.hpp"
#include "pa_internal.hpp"

namespace pa {

namespace {
thread_local std::string g_err;
}

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
}
void clear_error() { g_err.clear(); }

namespace {

// ---------------------------------------------------------------------------
// Scatter.  One workgroup per token; each thread moves VEC consecutive
// elements of one head (VEC = 8 when D % 8 == 0, else 1).
template <typename T, int VEC>
__global__ __launch_bounds__(256) void reshape_and_cache_kernel(
    const T* __restrict__ key, const T* __restrict__ value, T* __restrict__ k_cache,
    T* __restrict__ v_cache, const int64_t* __restrict__ slots, int H, int D, int64_t num_slots,
    int64_t key_stride, int64_t value_stride) {
  const int t = blockIdx.x;
  const int64_t slot = slots[t];
  if (slot < 0 || slot >= num_slots) return;
  const int64_t blk = slot / kBlock;
  const int off = (int)(slot % kBlock);
  const int per_head = D / VEC;
  for (int i = threadIdx.x; i < H * per_head; i += blockDim.x) {
    const int h = i / per_head;
    const int d0 = (i % per_head) * VEC;
    const T* ks = key + t * key_stride + (int64_t)h * D + d0;
    const T* vs = value + t * value_stride + (int64_t)h * D + d0;
    T* kd = k_cache + ((blk * H + h) * kBlock + off) * (int64_t)D + d0;
    T* vd = v_cache + ((blk * H + h) * (int64_t)D + d0) * kBlock + off;
    if constexpr (VEC * sizeof(T) == 16) {
      *reinterpret_cast<uint4*>(kd) = *reinterpret_cast<const uint4*>(ks);
      uint4 vv = *reinterpret_cast<const uint4*>(vs);
      const T* ve = reinterpret_cast<const T*>(&vv);
#pragma unroll
      for (int e = 0; e < VEC; ++e) vd[e * kBlock] = ve[e];
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        kd[e] = ks[e];
        vd[e * kBlock] = vs[e];
      }
    }
  }
}

// Quantising scatter into FP8 caches: as reshape_and_cache_kernel, each
// thread encodes VEC consecutive elements of one head (VEC = 8: one 8-byte
// K store; the V bytes go to VEC rows of the token-minor block).
template <typename T, int VEC>
__global__ __launch_bounds__(256) void reshape_and_cache_fp8_kernel(
    const T* __restrict__ key, const T* __restrict__ value, uint8_t* __restrict__ k_cache,
    uint8_t* __restrict__ v_cache, const int64_t* __restrict__ slots, int H, int D,
    int64_t num_slots, int64_t key_stride, int64_t value_stride, uint8_t* __restrict__ flags) {
  const int t = blockIdx.x;
  const int64_t slot = slots[t];
  if (slot < 0 || slot >= num_slots) return;
  const int64_t blk = slot / kBlock;
  const int off = (int)(slot % kBlock);
  const int per_head = D / VEC;
  for (int i = threadIdx.x; i < H * per_head; i += blockDim.x) {
    const int h = i / per_head;
    const int d0 = (i % per_head) * VEC;
    const T* ks = key + t * key_stride + (int64_t)h * D + d0;
    const T* vs = value + t * value_stride + (int64_t)h * D + d0;
    uint8_t* kd = k_cache + ((blk * H + h) * kBlock + off) * (int64_t)D + d0;
    uint8_t* vd = v_cache + ((blk * H + h) * (int64_t)D + d0) * kBlock + off;
    uint8_t kb[VEC];
    uint32_t ex = 0;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      kb[e] = fp8_encode(Elem<T>::load(ks + e));
      const uint8_t vb = fp8_encode(Elem<T>::load(vs + e));
      vd[e * kBlock] = vb;
      ex |= fp8_exotic_bits((uint32_t)kb[e] | ((uint32_t)vb << 8));
    }
    if (flags && (ex & 0x8080u)) flags[blk] = 1;
    if constexpr (VEC == 8) {
      *reinterpret_cast<uint2*>(kd) = *reinterpret_cast<const uint2*>(kb);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) kd[e] = kb[e];
    }
  }
}

// ---------------------------------------------------------------------------
// Block-coalesced scatter (the write path for D % 8 == 0 and 16-byte aligned
// operands).  Workgroup g owns input tokens [16 g, 16 g + 16).  When the
// token 16 g goes to offset o of its block and the 16 tokens from 16 g - o
// go to offsets 0 .. 15 of that one block in order (a prefill chunk's run of
// consecutive slots), the workgroup writes that whole block: each head's K
// block [16, D] and its token-minor V block [D, 16] are contiguous, so every
// store is a full 16-byte piece (the V block is transposed through LDS).
// Tokens of the workgroup's range that no such full-block range covers
// (its own, or the one workgroup g + 1 writes) go one by one as in
// reshape_and_cache_kernel: a decode step's scattered tokens, the partial
// blocks at the ends of a chunk.  Each token is written once; with
// duplicate slots in slot_mapping the surviving value is unspecified.
// TC = TS copies bits; TC = uint8_t encodes with the reference's FP8
// encoder (fp8_encode).

template <typename TS, typename TC>
struct Unit8 {
  TC v[8];
};
template <typename TS, typename TC>
__device__ inline Unit8<TS, TC> load_unit(const TS* __restrict__ p) {
  Unit8<TS, TC> u;
  if constexpr (sizeof(TC) == 1) {
    TS raw[8];
    if constexpr (sizeof(TS) == 2) {
      *reinterpret_cast<uint4*>(raw) = *reinterpret_cast<const uint4*>(p);
    } else {
      reinterpret_cast<uint4*>(raw)[0] = reinterpret_cast<const uint4*>(p)[0];
      reinterpret_cast<uint4*>(raw)[1] = reinterpret_cast<const uint4*>(p)[1];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) u.v[e] = fp8_encode(Elem<TS>::load(raw + e));
  } else {
    static_assert(sizeof(TS) == sizeof(TC), "copy");
#pragma unroll
    for (int q = 0; q < (int)sizeof(TC) / 2; ++q)
      reinterpret_cast<uint4*>(u.v)[q] = reinterpret_cast<const uint4*>(p)[q];
  }
  return u;
}
template <typename TS, typename TC>
__device__ inline void store_unit(TC* __restrict__ p, const Unit8<TS, TC>& u) {
  if constexpr (sizeof(TC) == 1) {
    *reinterpret_cast<uint2*>(p) = *reinterpret_cast<const uint2*>(u.v);
  } else {
#pragma unroll
    for (int q = 0; q < (int)sizeof(TC) / 2; ++q)
      reinterpret_cast<uint4*>(p)[q] = reinterpret_cast<const uint4*>(u.v)[q];
  }
}

// FP8 units: whether the K or V unit holds a code the hardware conversion
// reads differently from the reference (encoded from NaN / inf input); the
// flagged write records its block for pa_decode_fp8_flagged.
template <typename TS, typename TC>
__device__ inline bool unit_exotic(const Unit8<TS, TC>& k, const Unit8<TS, TC>& v) {
  if constexpr (sizeof(TC) == 1) {
    uint32_t w[4];
    __builtin_memcpy(w, k.v, 8);
    __builtin_memcpy(w + 2, v.v, 8);
    return ((fp8_exotic_bits(w[0]) | fp8_exotic_bits(w[1]) | fp8_exotic_bits(w[2]) |
             fp8_exotic_bits(w[3])) & 0x80808080u) != 0;
  } else {
    return false;
  }
}

template <typename TS, typename TC>
__global__ __launch_bounds__(256) void cache_write_kernel(
    const TS* __restrict__ key, const TS* __restrict__ value, TC* __restrict__ k_cache,
    TC* __restrict__ v_cache, const int64_t* __restrict__ slots, int T, int H, int D,
    int64_t num_slots, int64_t key_stride, int64_t value_stride, uint8_t* __restrict__ flags) {
  __shared__ int range_start[2];  // full-block range of this workgroup / of g + 1, or -1
  __shared__ __align__(16) TC vt[kBlock * 512];
  const int tid = threadIdx.x;
  const int t0 = blockIdx.x * kBlock;
  const int h = blockIdx.y;  // one kv head per workgroup
  if (tid < 64) {
    // lanes 0-15 test this workgroup's range, 16-31 the next one's
    const int half = (tid >> 4) & 1, j = tid & 15;
    const int tb = t0 + kBlock * half;
    int start = -1;
    bool ok = false;
    if (tid < 32 && tb < T) {
      const int64_t s0 = slots[tb];
      if (s0 >= 0 && s0 < num_slots) {
        start = tb - (int)(s0 % kBlock);
        if (start >= 0 && start + kBlock <= T)
          ok = slots[start + j] == s0 - s0 % kBlock + j;
      }
    }
    const uint64_t bal = __builtin_amdgcn_ballot_w64(ok);
    if (tid == 0) range_start[0] = (bal & 0xFFFFull) == 0xFFFFull ? start : -1;
    if (tid == 16) range_start[1] = ((bal >> 16) & 0xFFFFull) == 0xFFFFull ? start : -1;
  }
  __syncthreads();
  const int r0 = range_start[0], r1 = range_start[1];
  const int units = D / 8;  // 8-element units per head row
  if (r0 >= 0) {
    const int64_t blk = slots[r0] / kBlock;
    // K: the head's block [16, D] in order; V: staged as [16 tokens][D] in
    // LDS, then each thread writes one dim row of 16 tokens
    TC* kd = k_cache + (blk * H + h) * kBlock * (int64_t)D;
    for (int i = tid; i < kBlock * units; i += blockDim.x) {
      const int u = i % units, j = i / units;
      const int64_t src = (int64_t)(r0 + j) * key_stride + (int64_t)h * D + 8 * u;
      const Unit8<TS, TC> ku = load_unit<TS, TC>(key + src);
      store_unit<TS, TC>(kd + j * D + 8 * u, ku);
      const int64_t vsrc = (int64_t)(r0 + j) * value_stride + (int64_t)h * D + 8 * u;
      const Unit8<TS, TC> vu = load_unit<TS, TC>(value + vsrc);
      store_unit<TS, TC>(vt + j * D + 8 * u, vu);
      if (flags && unit_exotic(ku, vu)) flags[blk] = 1;
    }
    __syncthreads();
    TC* vd = v_cache + (blk * H + h) * (int64_t)D * kBlock;
    for (int d = tid; d < D; d += blockDim.x) {
      TC row[kBlock];
#pragma unroll
      for (int j = 0; j < kBlock; ++j) row[j] = vt[j * D + d];
#pragma unroll
      for (int q = 0; q < (int)(kBlock * sizeof(TC)) / 16; ++q)
        reinterpret_cast<uint4*>(vd + d * kBlock)[q] = reinterpret_cast<const uint4*>(row)[q];
    }
  }
  // tokens of [t0, t0 + 16) outside both full-block ranges, one unit per
  // thread: K unit stores, V element by element into the block rows
  for (int i = tid; i < kBlock * units; i += blockDim.x) {
    const int j = i / units, u = i % units;
    const int t = t0 + j;
    if (t >= T) break;
    if ((r0 >= 0 && t >= r0 && t < r0 + kBlock) || (r1 >= 0 && t >= r1 && t < r1 + kBlock))
      continue;
    const int64_t slot = slots[t];
    if (slot < 0 || slot >= num_slots) continue;
    const int64_t blk = slot / kBlock;
    const int off = (int)(slot % kBlock);
    const Unit8<TS, TC> ku =
        load_unit<TS, TC>(key + (int64_t)t * key_stride + (int64_t)h * D + 8 * u);
    store_unit<TS, TC>(k_cache + ((blk * H + h) * kBlock + off) * (int64_t)D + 8 * u, ku);
    const Unit8<TS, TC> vv =
        load_unit<TS, TC>(value + (int64_t)t * value_stride + (int64_t)h * D + 8 * u);
    if (flags && unit_exotic(ku, vv)) flags[blk] = 1;
    TC* vd = v_cache + ((blk * H + h) * (int64_t)D + 8 * u) * kBlock + off;
#pragma unroll
    for (int e = 0; e < 8; ++e) vd[e * kBlock] = vv.v[e];
  }
}

// Dequantising gather from FP8 caches (f32 out).
__global__ __launch_bounds__(256) void read_kv_fp8_kernel(const uint8_t* __restrict__ k_cache,
                                                          const uint8_t* __restrict__ v_cache,
                                                          const int32_t* __restrict__ block_ids,
                                                          int H, int D, int num_blocks,
                                                          float* __restrict__ out_k,
                                                          float* __restrict__ out_v) {
  const int t = blockIdx.x;
  const int32_t blk = block_ids[t / kBlock];
  const bool ok = blk >= 0 && blk < num_blocks;
  const int off = t % kBlock;
  for (int i = threadIdx.x; i < H * D; i += blockDim.x) {
    const int h = i / D, d = i % D;
    float kx = 0.f, vx = 0.f;
    if (ok) {
      kx = fp8_decode(k_cache[(((int64_t)blk * H + h) * kBlock + off) * D + d]);
      vx = fp8_decode(v_cache[(((int64_t)blk * H + h) * D + d) * kBlock + off]);
    }
    out_k[(int64_t)t * H * D + i] = kx;
    out_v[(int64_t)t * H * D + i] = vx;
  }
}

// slot_mapping[t] = block_tables[s][pos / 16] * 16 + pos % 16.
// The offsets cu are device data: clamped to the call's T tokens, so
// inconsistent offsets (a caller error) never index outside positions /
// slots.
__global__ void slot_mapping_kernel(const int32_t* __restrict__ block_tables, int mbs,
                                    const int64_t* __restrict__ positions,
                                    const int32_t* __restrict__ cu, int T,
                                    int64_t* __restrict__ slots) {
  const int s = blockIdx.x;
  const int begin = min(max(cu[s], 0), T), end = min(max(cu[s + 1], begin), T);
  for (int t = begin + threadIdx.x; t < end; t += blockDim.x) {
    const int64_t pos = positions[t];
    const int64_t bi = pos / kBlock;
    if (pos < 0 || bi >= mbs) {
      slots[t] = -1;
    } else {
      const int32_t blk = block_tables[(int64_t)s * mbs + bi];
      slots[t] = blk < 0 ? -1 : (int64_t)blk * kBlock + pos % kBlock;
    }
  }
}

// Gather: one workgroup per token.  Ids: a device array, or (SmallIds, by
// value in the kernel arguments) the few block ids of a short read, which
// then needs no upload.
struct SmallIds {
  int32_t id[kSmallIds];
};
template <typename T, typename Ids>
__global__ __launch_bounds__(256) void read_kv_kernel(const T* __restrict__ k_cache,
                                                      const T* __restrict__ v_cache, Ids block_ids,
                                                      int H, int D, int num_blocks,
                                                      T* __restrict__ out_k,
                                                      T* __restrict__ out_v) {
  const int t = blockIdx.x;
  int32_t blk;
  if constexpr (std::is_pointer_v<Ids>)
    blk = block_ids[t / kBlock];
  else
    blk = block_ids.id[t / kBlock];
  const bool ok = blk >= 0 && blk < num_blocks;
  const int off = t % kBlock;
  for (int i = threadIdx.x; i < H * D; i += blockDim.x) {
    const int h = i / D, d = i % D;
    T kx = T(0), vx = T(0);
    if (ok) {
      kx = k_cache[(((int64_t)blk * H + h) * kBlock + off) * D + d];
      vx = v_cache[(((int64_t)blk * H + h) * D + d) * kBlock + off];
    }
    out_k[(int64_t)t * H * D + i] = kx;
    out_v[(int64_t)t * H * D + i] = vx;
  }
}

// write_kv of one token (buffer.rs:103-267) in one launch: the hash of the K
// block as it stands after the token (buffer.rs:263-264; the token's rows
// from the input, the others from the cache), then the token's K row and V
// entries stored; the hash goes to *hash_out (host-mapped memory, read after
// the caller's synchronisation).
template <typename T>
__global__ __launch_bounds__(256) void write_token_kernel(T* __restrict__ k_cache,
                                                          T* __restrict__ v_cache,
                                                          const T* __restrict__ key,
                                                          const T* __restrict__ value, int H,
                                                          int D, int64_t blk, int off,
                                                          uint64_t* __restrict__ hash_out) {
  __shared__ uint64_t red[256];
  const int n = H * kBlock * D;
  const T* base = k_cache + blk * n;
  const uint64_t h = workgroup_block_hash(
      n,
      [&](int e) -> float {
        const int hd = e / (kBlock * D), r = e % (kBlock * D);
        return r / D == off ? Elem<T>::load(key + (int64_t)hd * D + r % D)
                            : Elem<T>::load(base + e);
      },
      red);  // ends with a barrier: every read of the block precedes the stores
  if (threadIdx.x == 0) *hash_out = h;
  for (int i = threadIdx.x; i < H * D; i += blockDim.x) {
    const int hd = i / D, d = i % D;
    k_cache[((blk * H + hd) * kBlock + off) * D + d] = key[i];
    v_cache[((blk * H + hd) * D + d) * kBlock + off] = value[i];
  }
}

// The reference's block-hash bookkeeping of a write (buffer.rs:263-264):
// after every token written, the hash of the K block it landed in.  Runs
// before the scatter of the same tokens, on the cache as it was before the
// call: one workgroup per block task walks the task's tokens in order; per
// token, slot o's rows come from the token that last wrote slot o in this
// call (last[o]), the other slots from the cache; hashes[tok[i]] is the
// hash after token tok[i] (tokens in call order).
template <typename T>
__global__ __launch_bounds__(256) void block_hash_replay_kernel(
    const T* __restrict__ k_cache, const T* __restrict__ key, int H, int D,
    const int32_t* __restrict__ task_block, const int32_t* __restrict__ task_beg,
    const int32_t* __restrict__ tok, const int32_t* __restrict__ off,
    uint64_t* __restrict__ hashes) {
  __shared__ uint64_t red[256];
  __shared__ int last[kBlock];
  const int w = blockIdx.x;
  const int n = H * kBlock * D;
  const T* base = k_cache + (int64_t)task_block[w] * n;
  if (threadIdx.x < kBlock) last[threadIdx.x] = -1;
  __syncthreads();
  for (int i = task_beg[w]; i < task_beg[w + 1]; ++i) {
    if (threadIdx.x == 0) last[off[i]] = tok[i];
    __syncthreads();
    const uint64_t h = workgroup_block_hash(
        n,
        [&](int e) -> float {
          const int hd = e / (kBlock * D), r = e % (kBlock * D);
          const int j = last[r / D];
          return j >= 0 ? Elem<T>::load(key + ((int64_t)j * H + hd) * D + r % D)
                        : Elem<T>::load(base + e);
        },
        red);
    if (threadIdx.x == 0) hashes[tok[i]] = h;
  }
}

// Polynomial hash sum_i x_i * 31^(n-1-i) (mod 2^64), split into per-thread
// contiguous chunks that are hashed sequentially and then combined.
__global__ __launch_bounds__(256) void block_hash_kernel(const float* __restrict__ k_cache,
                                                         const int32_t* __restrict__ block_ids,
                                                         int64_t n, int num_blocks,
                                                         uint64_t* __restrict__ out) {
  __shared__ uint64_t part[256];
  const int32_t blk = block_ids[blockIdx.x];
  if (blk < 0 || blk >= num_blocks) {
    if (threadIdx.x == 0) out[blockIdx.x] = 0;
    return;
  }
  const float* p = k_cache + (int64_t)blk * n;
  const int64_t chunk = (n + blockDim.x - 1) / blockDim.x;
  const int64_t b = threadIdx.x * chunk;
  const int64_t e = b + chunk < n ? b + chunk : n;
  uint64_t h = 0;
  for (int64_t i = b; i < e; ++i) h = h * 31u + hash_term(p[i]);
  part[threadIdx.x] = h;
  __syncthreads();
  if (threadIdx.x == 0) {
    // Every chunk except possibly the tail ones has `chunk` terms.
    uint64_t acc = 0;
    for (int c = 0; c < (int)blockDim.x; ++c) {
      const int64_t cb = c * chunk;
      const int64_t ce = cb + chunk < n ? cb + chunk : n;
      const int64_t len = ce > cb ? ce - cb : 0;
      acc = acc * pow_u64(31u, (uint64_t)len) + part[c];
    }
    out[blockIdx.x] = acc;
  }
}

}  // namespace

int32_t launch_write_token(void* k_cache, void* v_cache, const void* key, const void* value,
                           int32_t dtype, int H, int D, int64_t blk, int off,
                           uint64_t* hash_out, hipStream_t stream) {
  if (dtype == PA_DTYPE_BF16)
    write_token_kernel<uint16_t><<<1, 256, 0, stream>>>(
        (uint16_t*)k_cache, (uint16_t*)v_cache, (const uint16_t*)key, (const uint16_t*)value, H,
        D, blk, off, hash_out);
  else
    write_token_kernel<float><<<1, 256, 0, stream>>>((float*)k_cache, (float*)v_cache,
                                                     (const float*)key, (const float*)value, H,
                                                     D, blk, off, hash_out);
  return check_launch("write_kv");
}

int32_t launch_read_kv_small(const void* k_cache, const void* v_cache, int32_t dtype,
                             const int32_t* ids, int n_ids, int seq_len, int H, int D,
                             int num_blocks, void* out_k, void* out_v, hipStream_t stream) {
  SmallIds v{};
  for (int i = 0; i < n_ids && i < kSmallIds; ++i) v.id[i] = ids[i];
  if (dtype == PA_DTYPE_BF16)
    read_kv_kernel<uint16_t, SmallIds><<<seq_len, 256, 0, stream>>>(
        (const uint16_t*)k_cache, (const uint16_t*)v_cache, v, H, D, num_blocks,
        (uint16_t*)out_k, (uint16_t*)out_v);
  else
    read_kv_kernel<float, SmallIds><<<seq_len, 256, 0, stream>>>(
        (const float*)k_cache, (const float*)v_cache, v, H, D, num_blocks, (float*)out_k,
        (float*)out_v);
  return check_launch("read_kv");
}

int32_t launch_block_hash_replay(const void* k_cache, const void* key, int32_t dtype, int H,
                                 int D, int num_tasks, const int32_t* task_block,
                                 const int32_t* task_beg, const int32_t* tok,
                                 const int32_t* off, uint64_t* hashes, hipStream_t stream) {
  if (num_tasks == 0) return PA_OK;
  if (dtype == PA_DTYPE_BF16)
    block_hash_replay_kernel<uint16_t><<<num_tasks, 256, 0, stream>>>(
        (const uint16_t*)k_cache, (const uint16_t*)key, H, D, task_block, task_beg, tok, off,
        hashes);
  else
    block_hash_replay_kernel<float><<<num_tasks, 256, 0, stream>>>(
        (const float*)k_cache, (const float*)key, H, D, task_block, task_beg, tok, off, hashes);
  return check_launch("write_kv block hashes");
}

}  // namespace pa

using namespace pa;

extern "C" const char* pa_last_error(void) { return g_err.c_str(); }

extern "C" const char* pa_version(void) { return "vllm-lite-amd paged attention 0.1 (gfx950)"; }

extern "C" int32_t pa_reshape_and_cache(const void* key, const void* value, void* k_cache,
                                        void* v_cache, const int64_t* slot_mapping,
                                        int32_t num_tokens, int32_t num_kv_heads,
                                        int32_t head_dim, int32_t num_blocks, int64_t key_stride,
                                        int64_t value_stride, int32_t dtype, pa_stream_t stream) {
  clear_error();
  PA_REQUIRE(dtype_ok(dtype), PA_ERR_INVALID_ARG, "pa_reshape_and_cache: unknown dtype %d", dtype);
  PA_REQUIRE(num_tokens >= 0 && num_kv_heads > 0 && head_dim > 0 && num_blocks > 0,
             PA_ERR_INVALID_ARG, "pa_reshape_and_cache: bad sizes T=%d H=%d D=%d NB=%d",
             num_tokens, num_kv_heads, head_dim, num_blocks);
  if (num_tokens == 0) return PA_OK;
  PA_REQUIRE(key && value && k_cache && v_cache && slot_mapping, PA_ERR_INVALID_ARG,
             "pa_reshape_and_cache: null pointer");
  const int64_t row = (int64_t)num_kv_heads * head_dim;
  if (key_stride == 0) key_stride = row;
  if (value_stride == 0) value_stride = row;
  PA_REQUIRE(key_stride >= row && value_stride >= row, PA_ERR_INVALID_ARG,
             "pa_reshape_and_cache: token stride smaller than Hkv*D");
  const int64_t num_slots = (int64_t)num_blocks * kBlock;
  const size_t es = dtype_size(dtype);
  const bool vec = head_dim % 8 == 0 && (key_stride * es) % 16 == 0 &&
                   (value_stride * es) % 16 == 0 && ((uintptr_t)key % 16) == 0 &&
                   ((uintptr_t)value % 16) == 0 && ((uintptr_t)k_cache % 16) == 0;
  const dim3 grid(num_tokens), block(256);
  hipStream_t s = (hipStream_t)stream;
  const dim3 wgrid((num_tokens + kBlock - 1) / kBlock, num_kv_heads);
  if (vec && head_dim <= 512 && ((uintptr_t)v_cache % 16) == 0) {
    if (dtype == PA_DTYPE_BF16)
      cache_write_kernel<uint16_t, uint16_t><<<wgrid, block, 0, s>>>(
          (const uint16_t*)key, (const uint16_t*)value, (uint16_t*)k_cache, (uint16_t*)v_cache,
          slot_mapping, num_tokens, num_kv_heads, head_dim, num_slots, key_stride, value_stride,
          nullptr);
    else
      cache_write_kernel<float, float><<<wgrid, block, 0, s>>>(
          (const float*)key, (const float*)value, (float*)k_cache, (float*)v_cache, slot_mapping,
          num_tokens, num_kv_heads, head_dim, num_slots, key_stride, value_stride, nullptr);
    return check_launch("pa_reshape_and_cache");
  }
  if (dtype == PA_DTYPE_BF16) {
    auto* kc = (uint16_t*)k_cache;
    auto* vc = (uint16_t*)v_cache;
    if (vec)
      reshape_and_cache_kernel<uint16_t, 8><<<grid, block, 0, s>>>(
          (const uint16_t*)key, (const uint16_t*)value, kc, vc, slot_mapping, num_kv_heads,
          head_dim, num_slots, key_stride, value_stride);
    else
      reshape_and_cache_kernel<uint16_t, 1><<<grid, block, 0, s>>>(
          (const uint16_t*)key, (const uint16_t*)value, kc, vc, slot_mapping, num_kv_heads,
          head_dim, num_slots, key_stride, value_stride);
  } else {
    auto* kc = (float*)k_cache;
    auto* vc = (float*)v_cache;
    if (head_dim % 4 == 0 && vec)
      reshape_and_cache_kernel<float, 4><<<grid, block, 0, s>>>(
          (const float*)key, (const float*)value, kc, vc, slot_mapping, num_kv_heads, head_dim,
          num_slots, key_stride, value_stride);
    else
      reshape_and_cache_kernel<float, 1><<<grid, block, 0, s>>>(
          (const float*)key, (const float*)value, kc, vc, slot_mapping, num_kv_heads, head_dim,
          num_slots, key_stride, value_stride);
  }
  return check_launch("pa_reshape_and_cache");
}

namespace {
int32_t reshape_and_cache_fp8_impl(const void* key, const void* value, uint8_t* k_cache,
                                   uint8_t* v_cache, const int64_t* slot_mapping,
                                   int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
                                   int32_t num_blocks, int64_t key_stride, int64_t value_stride,
                                   int32_t src_dtype, uint8_t* flags, pa_stream_t stream) {
  clear_error();
  PA_REQUIRE(dtype_ok(src_dtype), PA_ERR_INVALID_ARG,
             "pa_reshape_and_cache_fp8: source dtype %d is not f32 or bf16", src_dtype);
  PA_REQUIRE(num_tokens >= 0 && num_kv_heads > 0 && head_dim > 0 && num_blocks > 0,
             PA_ERR_INVALID_ARG, "pa_reshape_and_cache_fp8: bad sizes T=%d H=%d D=%d NB=%d",
             num_tokens, num_kv_heads, head_dim, num_blocks);
  if (num_tokens == 0) return PA_OK;
  PA_REQUIRE(key && value && k_cache && v_cache && slot_mapping, PA_ERR_INVALID_ARG,
             "pa_reshape_and_cache_fp8: null pointer");
  const int64_t row = (int64_t)num_kv_heads * head_dim;
  if (key_stride == 0) key_stride = row;
  if (value_stride == 0) value_stride = row;
  PA_REQUIRE(key_stride >= row && value_stride >= row, PA_ERR_INVALID_ARG,
             "pa_reshape_and_cache_fp8: token stride smaller than Hkv*D");
  const int64_t num_slots = (int64_t)num_blocks * kBlock;
  const bool vec = head_dim % 8 == 0 && ((uintptr_t)k_cache % 8) == 0;
  const dim3 grid(num_tokens), block(256);
  hipStream_t s = (hipStream_t)stream;
  const size_t es = dtype_size(src_dtype);
  if (vec && head_dim <= 512 && ((uintptr_t)v_cache % 16) == 0 && ((uintptr_t)key % 16) == 0 &&
      ((uintptr_t)value % 16) == 0 && (key_stride * es) % 16 == 0 &&
      (value_stride * es) % 16 == 0) {
    const dim3 wgrid((num_tokens + kBlock - 1) / kBlock, num_kv_heads);
    if (src_dtype == PA_DTYPE_BF16)
      cache_write_kernel<uint16_t, uint8_t><<<wgrid, block, 0, s>>>(
          (const uint16_t*)key, (const uint16_t*)value, k_cache, v_cache, slot_mapping,
          num_tokens, num_kv_heads, head_dim, num_slots, key_stride, value_stride, flags);
    else
      cache_write_kernel<float, uint8_t><<<wgrid, block, 0, s>>>(
          (const float*)key, (const float*)value, k_cache, v_cache, slot_mapping, num_tokens,
          num_kv_heads, head_dim, num_slots, key_stride, value_stride, flags);
    return check_launch("pa_reshape_and_cache_fp8");
  }
#define PA_LAUNCH_Q(T, V)                                                                    \
  reshape_and_cache_fp8_kernel<T, V><<<grid, block, 0, s>>>(                                 \
      (const T*)key, (const T*)value, k_cache, v_cache, slot_mapping, num_kv_heads, head_dim, \
      num_slots, key_stride, value_stride, flags)
  if (src_dtype == PA_DTYPE_BF16) {
    if (vec)
      PA_LAUNCH_Q(uint16_t, 8);
    else
      PA_LAUNCH_Q(uint16_t, 1);
  } else {
    if (vec)
      PA_LAUNCH_Q(float, 8);
    else
      PA_LAUNCH_Q(float, 1);
  }
#undef PA_LAUNCH_Q
  return check_launch("pa_reshape_and_cache_fp8");
}
}  // namespace

extern "C" int32_t pa_reshape_and_cache_fp8(const void* key, const void* value, uint8_t* k_cache,
                                            uint8_t* v_cache, const int64_t* slot_mapping,
                                            int32_t num_tokens, int32_t num_kv_heads,
                                            int32_t head_dim, int32_t num_blocks,
                                            int64_t key_stride, int64_t value_stride,
                                            int32_t src_dtype, pa_stream_t stream) {
  return reshape_and_cache_fp8_impl(key, value, k_cache, v_cache, slot_mapping, num_tokens,
                                    num_kv_heads, head_dim, num_blocks, key_stride, value_stride,
                                    src_dtype, nullptr, stream);
}

extern "C" int32_t pa_reshape_and_cache_fp8_flagged(
    const void* key, const void* value, uint8_t* k_cache, uint8_t* v_cache,
    const int64_t* slot_mapping, int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
    int32_t num_blocks, int64_t key_stride, int64_t value_stride, int32_t src_dtype,
    uint8_t* block_flags, pa_stream_t stream) {
  if (!block_flags) {
    clear_error();
    set_error("pa_reshape_and_cache_fp8_flagged: null block_flags");
    return PA_ERR_INVALID_ARG;
  }
  return reshape_and_cache_fp8_impl(key, value, k_cache, v_cache, slot_mapping, num_tokens,
                                    num_kv_heads, head_dim, num_blocks, key_stride, value_stride,
                                    src_dtype, block_flags, stream);
}

extern "C" int32_t pa_slot_mapping(const int32_t* block_tables, int32_t max_blocks_per_seq,
                                   const int64_t* positions, const int32_t* cu_seq_tokens,
                                   int32_t num_seqs, int32_t num_tokens, int64_t* slot_mapping,
                                   pa_stream_t stream) {
  clear_error();
  PA_REQUIRE(num_seqs >= 0 && num_tokens >= 0 && max_blocks_per_seq >= 0, PA_ERR_INVALID_ARG,
             "pa_slot_mapping: negative size");
  if (num_seqs == 0 || num_tokens == 0) return PA_OK;
  PA_REQUIRE(block_tables && positions && cu_seq_tokens && slot_mapping, PA_ERR_INVALID_ARG,
             "pa_slot_mapping: null pointer");
  slot_mapping_kernel<<<num_seqs, 256, 0, (hipStream_t)stream>>>(
      block_tables, max_blocks_per_seq, positions, cu_seq_tokens, num_tokens, slot_mapping);
  return check_launch("pa_slot_mapping");
}

extern "C" int32_t pa_read_kv(const void* k_cache, const void* v_cache, const int32_t* block_ids,
                              int32_t n_ids, int32_t seq_len, int32_t num_kv_heads,
                              int32_t head_dim, int32_t num_blocks, void* out_k, void* out_v,
                              int32_t dtype, pa_stream_t stream) {
  clear_error();
  PA_REQUIRE(dtype_ok(dtype) || dtype == PA_DTYPE_FP8_E4M3, PA_ERR_INVALID_ARG,
             "pa_read_kv: unknown dtype %d", dtype);
  PA_REQUIRE(seq_len >= 0 && n_ids >= 0 && num_kv_heads > 0 && head_dim > 0 && num_blocks > 0,
             PA_ERR_INVALID_ARG, "pa_read_kv: bad sizes");
  if (seq_len == 0 || n_ids == 0) return PA_OK;
  PA_REQUIRE((int64_t)n_ids * kBlock >= seq_len, PA_ERR_OUT_OF_BOUNDS,
             "pa_read_kv: %d blocks cannot hold %d tokens", n_ids, seq_len);
  PA_REQUIRE(k_cache && v_cache && block_ids && out_k && out_v, PA_ERR_INVALID_ARG,
             "pa_read_kv: null pointer");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == PA_DTYPE_FP8_E4M3)
    read_kv_fp8_kernel<<<seq_len, 256, 0, s>>>(
        (const uint8_t*)k_cache, (const uint8_t*)v_cache, block_ids, num_kv_heads, head_dim,
        num_blocks, (float*)out_k, (float*)out_v);
  else if (dtype == PA_DTYPE_BF16)
    read_kv_kernel<uint16_t, const int32_t*><<<seq_len, 256, 0, s>>>(
        (const uint16_t*)k_cache, (const uint16_t*)v_cache, block_ids, num_kv_heads, head_dim,
        num_blocks, (uint16_t*)out_k, (uint16_t*)out_v);
  else
    read_kv_kernel<float, const int32_t*><<<seq_len, 256, 0, s>>>(
        (const float*)k_cache, (const float*)v_cache, block_ids, num_kv_heads, head_dim,
        num_blocks, (float*)out_k, (float*)out_v);
  return check_launch("pa_read_kv");
}

extern "C" int32_t pa_block_hash(const float* k_cache, const int32_t* block_ids, int32_t n,
                                 int32_t num_kv_heads, int32_t head_dim, int32_t num_blocks,
                                 uint64_t* hashes, pa_stream_t stream) {
  clear_error();
  PA_REQUIRE(n >= 0 && num_kv_heads > 0 && head_dim > 0 && num_blocks > 0, PA_ERR_INVALID_ARG,
             "pa_block_hash: bad sizes");
  if (n == 0) return PA_OK;
  PA_REQUIRE(k_cache && block_ids && hashes, PA_ERR_INVALID_ARG, "pa_block_hash: null pointer");
  const int64_t per_block = (int64_t)num_kv_heads * kBlock * head_dim;
  block_hash_kernel<<<n, 256, 0, (hipStream_t)stream>>>(k_cache, block_ids, per_block, num_blocks,
                                                        hashes);
  return check_launch("pa_block_hash");
}
