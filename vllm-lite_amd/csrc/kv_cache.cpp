// Host-side PagedKvCache mirror (pa_kv_cache_* in pa_kv_cache.h).
//
// Owns one K and one V device buffer per layer and implements the
// reference's write_kv / write_kv_batch / write_prefill_kv / read_kv on top
// of the stateless kernels: index arithmetic and bounds checks run on the
// host exactly where the reference checks them, the data movement is one
// kernel launch per call.  A quantised cache (the reference's
// quantized = true) keeps int8 values in f32 with one scale per block; its
// writes re-quantise whole blocks (quant.hip).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "../../include/pa_kv_cache.h"
#include "pa_common.hpp"
#include "pa_internal.hpp"

struct pa_kv_cache {
  int num_layers = 0, num_heads = 0, head_dim = 0, num_blocks = 0, dtype = 0;
  bool quantized = false;
  std::vector<void*> key, value;
  std::vector<float*> scales;  // quantised caches: [num_blocks] per layer
  // The reference's per-layer block-hash map (tensor_store/mod.rs:42):
  // hash of a K block after a token was written -> the block's id.
  std::vector<std::unordered_map<uint64_t, int64_t>> block_hashes;
  // Staging for host index arrays: pinned host copy -> device copy.
  void* host_stage = nullptr;
  void* dev_stage = nullptr;
  size_t stage_bytes = 0;
  // One token's block hash, written by the device into host-mapped memory
  // (write_kv of a single token: no index upload, no copy back).
  uint64_t* hash_host = nullptr;
  uint64_t* hash_dev = nullptr;

  int32_t ensure_hash_slot() {
    if (hash_host) return PA_OK;
    void* h = nullptr;
    void* d = nullptr;
    if (hipHostMalloc(&h, 256, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess ||
        hipHostGetDevicePointer(&d, h, 0) != hipSuccess) {
      if (h) (void)hipHostFree(h);
      pa::set_error("pa_kv_cache: allocating the mapped hash slot failed");
      return PA_ERR_HIP;
    }
    hash_host = (uint64_t*)h;
    hash_dev = (uint64_t*)d;
    return PA_OK;
  }

  size_t layer_bytes() const {
    return (size_t)num_blocks * num_heads * pa::kBlock * head_dim * pa::dtype_size(dtype);
  }

  int32_t ensure_stage(size_t bytes) {
    if (bytes <= stage_bytes) return PA_OK;
    if (host_stage) (void)hipHostFree(host_stage);
    if (dev_stage) (void)hipFree(dev_stage);
    host_stage = dev_stage = nullptr;
    stage_bytes = 0;
    size_t cap = bytes < 4096 ? 4096 : bytes;
    if (hipHostMalloc(&host_stage, cap, hipHostMallocDefault) != hipSuccess ||
        hipMalloc(&dev_stage, cap) != hipSuccess) {
      pa::set_error("pa_kv_cache: staging allocation of %zu bytes failed", cap);
      return PA_ERR_HIP;
    }
    stage_bytes = cap;
    return PA_OK;
  }

  // Copies `bytes` of host data to the device stage on `stream` and returns
  // the device pointer.  The caller synchronises the stream before the
  // stage is reused.
  void* upload(const void* src, size_t bytes, hipStream_t stream, int32_t* rc) {
    *rc = ensure_stage(bytes);
    if (*rc != PA_OK) return nullptr;
    std::memcpy(host_stage, src, bytes);
    if (hipMemcpyAsync(dev_stage, host_stage, bytes, hipMemcpyHostToDevice, stream) !=
        hipSuccess) {
      pa::set_error("pa_kv_cache: index upload failed");
      *rc = PA_ERR_HIP;
      return nullptr;
    }
    return dev_stage;
  }
};

namespace {

// Waits for the call's upload and launch.  Also after a failed launch: the
// upload from the pinned stage may still be in flight, and the next call
// refills the stage.  The first error is the one reported.
int32_t finish(hipStream_t stream, int32_t rc) {
  const bool synced = hipStreamSynchronize(stream) == hipSuccess;
  if (rc != PA_OK) return rc;
  if (!synced) {
    pa::set_error("pa_kv_cache: stream synchronisation failed");
    return PA_ERR_HIP;
  }
  return PA_OK;
}

// Writes T tokens at host-computed slots as the reference's per-token
// write_kv does, block-hash bookkeeping included (buffer.rs:263-264): the
// tokens are grouped by block (keeping their order) into tasks; every
// token's K block is hashed as it stands after that token, and the map of
// the layer receives hash -> block in token order.  Non-quantised caches:
// the hashes are replayed from the cache before the scatter (one kernel),
// then the tokens are scattered; quantised caches: each block is
// re-quantised once per token (quant_write_kernel), which also hashes it.
int32_t scatter(pa_kv_cache* c, int layer, const std::vector<int64_t>& slots, const void* k,
                const void* v, hipStream_t stream) {
  std::map<int64_t, std::vector<int32_t>> by_block;  // block -> token indices, in order
  for (size_t t = 0; t < slots.size(); ++t) by_block[slots[t] / pa::kBlock].push_back((int32_t)t);
  const int tasks = (int)by_block.size();
  const int T = (int)slots.size();
  // one upload: slots (int64 [T]), hashes (uint64 [T], written on the
  // device), then the int32 task arrays
  const size_t n32 = (size_t)tasks + (tasks + 1) + 2 * (size_t)T;
  std::vector<int64_t> host(2 * (size_t)T + (n32 + 1) / 2);
  // The scatter writes every slot once, from the last token that names it
  // (the reference writes token by token, so the last one wins; a slot
  // named twice in one scatter would be unspecified): earlier ones are -1.
  {
    std::unordered_set<int64_t> seen;
    seen.reserve(2 * (size_t)T);
    for (int t = T - 1; t >= 0; --t) host[t] = seen.insert(slots[t]).second ? slots[t] : -1;
  }
  auto* i32 = reinterpret_cast<int32_t*>(host.data() + 2 * T);
  int32_t* blk = i32;
  int32_t* beg = blk + tasks;
  int32_t* tok = beg + tasks + 1;
  int32_t* off = tok + T;
  int w = 0, i = 0;
  for (const auto& kv : by_block) {
    blk[w] = (int32_t)kv.first;
    beg[w] = i;
    for (int32_t t : kv.second) {
      tok[i] = t;
      off[i] = (int32_t)(slots[t] % pa::kBlock);
      ++i;
    }
    ++w;
  }
  beg[tasks] = i;
  int32_t rc = PA_OK;
  auto* d = (char*)c->upload(host.data(), host.size() * sizeof(int64_t), stream, &rc);
  if (rc != PA_OK) return rc;
  const auto* d_slots = (const int64_t*)d;
  auto* d_hash = (uint64_t*)(d + (size_t)T * sizeof(int64_t));
  const auto* d32 = (const int32_t*)(d + 2 * (size_t)T * sizeof(int64_t));
  const int32_t *d_blk = d32, *d_beg = d32 + tasks, *d_tok = d_beg + tasks + 1, *d_off = d_tok + T;
  if (c->quantized) {
    rc = pa::launch_quant_write((float*)c->key[layer], (float*)c->value[layer], c->scales[layer],
                                (const float*)k, (const float*)v, c->num_heads, c->head_dim,
                                tasks, d_blk, d_beg, d_tok, d_off, d_hash, stream);
  } else {
    rc = pa::launch_block_hash_replay(c->key[layer], k, c->dtype, c->num_heads, c->head_dim,
                                      tasks, d_blk, d_beg, d_tok, d_off, d_hash, stream);
    if (rc == PA_OK)
      rc = pa_reshape_and_cache(k, v, c->key[layer], c->value[layer], d_slots, T, c->num_heads,
                                c->head_dim, c->num_blocks, 0, 0, c->dtype, (pa_stream_t)stream);
  }
  rc = finish(stream, rc);
  if (rc != PA_OK) return rc;
  std::vector<uint64_t> hashes(T);
  if (hipMemcpy(hashes.data(), d_hash, (size_t)T * sizeof(uint64_t), hipMemcpyDeviceToHost) !=
      hipSuccess) {
    pa::set_error("pa_kv_cache: reading the block hashes back failed");
    return PA_ERR_HIP;
  }
  auto& map = c->block_hashes[layer];
  for (int t = 0; t < T; ++t) map[hashes[t]] = slots[t] / pa::kBlock;
  return PA_OK;
}

}  // namespace

extern "C" int32_t pa_kv_cache_create(int32_t num_layers, int32_t num_kv_heads, int32_t head_dim,
                                      int32_t num_blocks, int32_t dtype, pa_kv_cache** out) {
  pa::clear_error();
  PA_REQUIRE(out, PA_ERR_INVALID_ARG, "pa_kv_cache_create: null out");
  *out = nullptr;
  PA_REQUIRE(pa::dtype_ok(dtype), PA_ERR_INVALID_ARG, "pa_kv_cache_create: unknown dtype %d",
             dtype);
  PA_REQUIRE(num_layers > 0 && num_kv_heads > 0 && head_dim > 0 && num_blocks > 0,
             PA_ERR_INVALID_ARG, "pa_kv_cache_create: sizes must be positive");
  auto* c = new pa_kv_cache();
  c->num_layers = num_layers;
  c->num_heads = num_kv_heads;
  c->head_dim = head_dim;
  c->num_blocks = num_blocks;
  c->dtype = dtype;
  c->block_hashes.resize(num_layers);
  const size_t bytes = c->layer_bytes();
  for (int l = 0; l < num_layers; ++l) {
    void *k = nullptr, *v = nullptr;
    if (hipMalloc(&k, bytes) != hipSuccess || hipMalloc(&v, bytes) != hipSuccess ||
        hipMemset(k, 0, bytes) != hipSuccess || hipMemset(v, 0, bytes) != hipSuccess) {
      if (k) (void)hipFree(k);
      if (v) (void)hipFree(v);
      pa_kv_cache_destroy(c);
      pa::set_error("pa_kv_cache_create: allocating %zu bytes per layer failed", bytes);
      return PA_ERR_HIP;
    }
    c->key.push_back(k);
    c->value.push_back(v);
  }
  *out = c;
  return PA_OK;
}

extern "C" int32_t pa_kv_cache_create_quantized(int32_t num_layers, int32_t num_kv_heads,
                                                int32_t head_dim, int32_t num_blocks,
                                                pa_kv_cache** out) {
  int32_t rc = pa_kv_cache_create(num_layers, num_kv_heads, head_dim, num_blocks, PA_DTYPE_F32,
                                  out);
  if (rc != PA_OK) return rc;
  pa_kv_cache* c = *out;
  c->quantized = true;
  const std::vector<float> ones(num_blocks, 1.0f);  // mod.rs:69
  for (int l = 0; l < num_layers; ++l) {
    float* sp = nullptr;
    if (hipMalloc(&sp, num_blocks * sizeof(float)) != hipSuccess ||
        hipMemcpy(sp, ones.data(), num_blocks * sizeof(float), hipMemcpyHostToDevice) !=
            hipSuccess) {
      if (sp) (void)hipFree(sp);
      pa_kv_cache_destroy(c);
      *out = nullptr;
      pa::set_error("pa_kv_cache_create_quantized: allocating the block scales failed");
      return PA_ERR_HIP;
    }
    c->scales.push_back(sp);
  }
  return PA_OK;
}

extern "C" void pa_kv_cache_destroy(pa_kv_cache* c) {
  if (!c) return;
  for (void* p : c->key) (void)hipFree(p);
  for (void* p : c->value) (void)hipFree(p);
  for (float* p : c->scales) (void)hipFree(p);
  if (c->host_stage) (void)hipHostFree(c->host_stage);
  if (c->hash_host) (void)hipHostFree(c->hash_host);
  if (c->dev_stage) (void)hipFree(c->dev_stage);
  delete c;
}

extern "C" int32_t pa_kv_cache_num_layers(const pa_kv_cache* c) { return c ? c->num_layers : 0; }
extern "C" int32_t pa_kv_cache_num_blocks(const pa_kv_cache* c) { return c ? c->num_blocks : 0; }
extern "C" int32_t pa_kv_cache_block_size(const pa_kv_cache*) { return pa::kBlock; }
extern "C" int32_t pa_kv_cache_num_heads(const pa_kv_cache* c) { return c ? c->num_heads : 0; }
extern "C" int32_t pa_kv_cache_head_dim(const pa_kv_cache* c) { return c ? c->head_dim : 0; }
extern "C" int32_t pa_kv_cache_dtype(const pa_kv_cache* c) { return c ? c->dtype : -1; }

extern "C" int32_t pa_kv_cache_is_quantized(const pa_kv_cache* c) {
  return c && c->quantized ? 1 : 0;
}
extern "C" float* pa_kv_cache_scales_ptr(pa_kv_cache* c, int32_t layer) {
  return (c && c->quantized && layer >= 0 && layer < c->num_layers) ? c->scales[layer] : nullptr;
}

extern "C" void* pa_kv_cache_key_ptr(pa_kv_cache* c, int32_t layer) {
  return (c && layer >= 0 && layer < c->num_layers) ? c->key[layer] : nullptr;
}
extern "C" void* pa_kv_cache_value_ptr(pa_kv_cache* c, int32_t layer) {
  return (c && layer >= 0 && layer < c->num_layers) ? c->value[layer] : nullptr;
}

extern "C" int32_t pa_kv_cache_write_kv(pa_kv_cache* c, int32_t layer, int64_t block_id,
                                        int64_t token_offset, const void* k, const void* v,
                                        pa_stream_t stream) {
  pa::clear_error();
  PA_REQUIRE(c && k && v, PA_ERR_INVALID_ARG, "write_kv: null argument");
  PA_REQUIRE(layer >= 0 && layer < c->num_layers, PA_ERR_OUT_OF_BOUNDS,
             "layer_idx %d out of bounds for %d layers", layer, c->num_layers);
  PA_REQUIRE(block_id >= 0 && block_id < c->num_blocks, PA_ERR_OUT_OF_BOUNDS,
             "block_id %lld out of bounds for %d blocks", (long long)block_id, c->num_blocks);
  PA_REQUIRE(token_offset >= 0 && token_offset < pa::kBlock, PA_ERR_OUT_OF_BOUNDS,
             "token_offset %lld out of bounds for block size %d", (long long)token_offset,
             pa::kBlock);
  hipStream_t s = (hipStream_t)stream;
  if (!c->quantized) {
    // one launch: the block's hash after the token, then the token's rows
    int32_t rc = c->ensure_hash_slot();
    if (rc != PA_OK) return rc;
    rc = pa::launch_write_token(c->key[layer], c->value[layer], k, v, c->dtype, c->num_heads,
                                c->head_dim, block_id, (int)token_offset, c->hash_dev, s);
    rc = finish(s, rc);
    if (rc != PA_OK) return rc;
    const uint64_t h = *(volatile uint64_t*)c->hash_host;
    c->block_hashes[layer][h] = block_id;
    return PA_OK;
  }
  return scatter(c, layer, {block_id * pa::kBlock + token_offset}, k, v, s);
}

extern "C" int32_t pa_kv_cache_write_kv_batch(pa_kv_cache* c, int32_t layer, int64_t block_id,
                                              int64_t token_offset, const void* k, const void* v,
                                              int32_t num_tokens, pa_stream_t stream) {
  pa::clear_error();
  PA_REQUIRE(c && k && v, PA_ERR_INVALID_ARG, "write_kv_batch: null argument");
  PA_REQUIRE(layer >= 0 && layer < c->num_layers, PA_ERR_OUT_OF_BOUNDS,
             "layer_idx %d out of bounds for %d layers", layer, c->num_layers);
  PA_REQUIRE(num_tokens >= 0 && block_id >= 0 && block_id < c->num_blocks && token_offset >= 0,
             PA_ERR_OUT_OF_BOUNDS, "write_kv_batch: block_id %lld / offset %lld out of range",
             (long long)block_id, (long long)token_offset);
  const int64_t space = ((int64_t)c->num_blocks - block_id) * pa::kBlock;
  PA_REQUIRE(token_offset + num_tokens <= space, PA_ERR_OUT_OF_BOUNDS,
             "Token offset %lld + num_tokens %d exceeds available space %lld",
             (long long)token_offset, num_tokens, (long long)space);
  if (num_tokens == 0) return PA_OK;
  std::vector<int64_t> slots(num_tokens);
  int64_t blk = block_id, off = token_offset;
  for (int t = 0; t < num_tokens; ++t) {
    // Offsets >= 16 in the first block are walked the same way the
    // reference's per-token loop walks them: write_kv would reject them.
    PA_REQUIRE(off < pa::kBlock, PA_ERR_OUT_OF_BOUNDS,
               "token_offset %lld out of bounds for block size %d", (long long)off, pa::kBlock);
    slots[t] = blk * pa::kBlock + off;
    if (++off >= pa::kBlock) {
      ++blk;
      off = 0;
    }
  }
  return scatter(c, layer, slots, k, v, (hipStream_t)stream);
}

extern "C" int32_t pa_kv_cache_write_prefill_kv(pa_kv_cache* c, int32_t layer,
                                                const int64_t* block_ids, int32_t n_ids,
                                                const int64_t* positions, int32_t n_pos,
                                                int32_t num_tokens, const void* k, const void* v,
                                                pa_stream_t stream) {
  pa::clear_error();
  PA_REQUIRE(c && k && v && (block_ids || n_ids == 0), PA_ERR_INVALID_ARG,
             "write_prefill_kv: null argument");
  PA_REQUIRE(layer >= 0 && layer < c->num_layers, PA_ERR_OUT_OF_BOUNDS,
             "layer_idx %d out of bounds for %d layers", layer, c->num_layers);
  PA_REQUIRE(num_tokens >= 0, PA_ERR_INVALID_ARG, "write_prefill_kv: negative token count");
  if (num_tokens == 0) return PA_OK;
  std::vector<int64_t> slots(num_tokens);
  for (int t = 0; t < num_tokens; ++t) {
    const int64_t pos = (positions && t < n_pos) ? positions[t] : t;
    PA_REQUIRE(pos >= 0, PA_ERR_OUT_OF_BOUNDS, "write_prefill_kv: negative position");
    const int64_t bi = pos / pa::kBlock;
    PA_REQUIRE(bi < n_ids, PA_ERR_OUT_OF_BOUNDS,
               "write_prefill_kv: position %lld needs block index %lld, table has %d",
               (long long)pos, (long long)bi, n_ids);
    const int64_t blk = block_ids[bi];
    PA_REQUIRE(blk >= 0 && blk < c->num_blocks, PA_ERR_OUT_OF_BOUNDS,
               "block_id %lld out of bounds for %d blocks", (long long)blk, c->num_blocks);
    slots[t] = blk * pa::kBlock + pos % pa::kBlock;
  }
  return scatter(c, layer, slots, k, v, (hipStream_t)stream);
}

extern "C" int32_t pa_kv_cache_read_kv(pa_kv_cache* c, int32_t layer, const int64_t* block_ids,
                                       int32_t n_ids, int32_t seq_len, void* out_k, void* out_v,
                                       int32_t* n_read, pa_stream_t stream) {
  pa::clear_error();
  PA_REQUIRE(c && n_read, PA_ERR_INVALID_ARG, "read_kv: null argument");
  *n_read = 0;
  PA_REQUIRE(layer >= 0 && layer < c->num_layers, PA_ERR_OUT_OF_BOUNDS,
             "layer_idx %d out of bounds for %d layers", layer, c->num_layers);
  if (n_ids <= 0 || seq_len <= 0) return PA_OK;
  PA_REQUIRE(block_ids && out_k && out_v, PA_ERR_INVALID_ARG, "read_kv: null argument");
  const int64_t cover = (int64_t)n_ids * pa::kBlock;
  const int32_t n = (int32_t)(seq_len < cover ? seq_len : cover);
  const int32_t used = (n + pa::kBlock - 1) / pa::kBlock;
  std::vector<int32_t> ids(used);
  for (int b = 0; b < used; ++b) {
    PA_REQUIRE(block_ids[b] >= 0 && block_ids[b] < c->num_blocks, PA_ERR_OUT_OF_BOUNDS,
               "block_id %lld out of bounds for %d blocks", (long long)block_ids[b],
               c->num_blocks);
    ids[b] = (int32_t)block_ids[b];
  }
  hipStream_t s = (hipStream_t)stream;
  int32_t rc = PA_OK;
  if (!c->quantized && used <= pa::kSmallIds) {
    // the ids go in the kernel arguments: no upload, so nothing to wait for
    rc = pa::launch_read_kv_small(c->key[layer], c->value[layer], c->dtype, ids.data(), used, n,
                                  c->num_heads, c->head_dim, c->num_blocks, out_k, out_v, s);
    if (rc == PA_OK) *n_read = n;
    return rc;
  }
  void* d_ids = c->upload(ids.data(), ids.size() * sizeof(int32_t), s, &rc);
  if (rc != PA_OK) return rc;
  if (c->quantized)
    rc = pa::launch_quant_read((const float*)c->key[layer], (const float*)c->value[layer],
                               c->scales[layer], (const int32_t*)d_ids, n, c->num_heads,
                               c->head_dim, (float*)out_k, (float*)out_v, s);
  else
    rc = pa_read_kv(c->key[layer], c->value[layer], (const int32_t*)d_ids, used, n, c->num_heads,
                    c->head_dim, c->num_blocks, out_k, out_v, c->dtype, stream);
  rc = finish(s, rc);
  if (rc == PA_OK) *n_read = n;
  return rc;
}

extern "C" int32_t pa_kv_cache_block_hash_count(const pa_kv_cache* c, int32_t layer,
                                                int64_t* count) {
  pa::clear_error();
  PA_REQUIRE(c && count, PA_ERR_INVALID_ARG, "block_hash_count: null argument");
  PA_REQUIRE(layer >= 0 && layer < c->num_layers, PA_ERR_OUT_OF_BOUNDS,
             "layer_idx %d out of bounds for %d layers", layer, c->num_layers);
  *count = (int64_t)c->block_hashes[layer].size();
  return PA_OK;
}

extern "C" int32_t pa_kv_cache_block_hashes(const pa_kv_cache* c, int32_t layer,
                                            uint64_t* hashes, int64_t* block_ids,
                                            int64_t capacity, int64_t* written) {
  pa::clear_error();
  PA_REQUIRE(c && written && capacity >= 0 && (capacity == 0 || (hashes && block_ids)),
             PA_ERR_INVALID_ARG, "block_hashes: bad arguments");
  PA_REQUIRE(layer >= 0 && layer < c->num_layers, PA_ERR_OUT_OF_BOUNDS,
             "layer_idx %d out of bounds for %d layers", layer, c->num_layers);
  std::vector<std::pair<uint64_t, int64_t>> e(c->block_hashes[layer].begin(),
                                              c->block_hashes[layer].end());
  std::sort(e.begin(), e.end());
  const int64_t n = std::min<int64_t>(capacity, (int64_t)e.size());
  for (int64_t i = 0; i < n; ++i) {
    hashes[i] = e[i].first;
    block_ids[i] = e[i].second;
  }
  *written = n;
  return PA_OK;
}

extern "C" int32_t pa_kv_cache_lookup_block_hash(const pa_kv_cache* c, int32_t layer,
                                                 uint64_t hash, int64_t* block_id) {
  pa::clear_error();
  PA_REQUIRE(c && block_id, PA_ERR_INVALID_ARG, "lookup_block_hash: null argument");
  PA_REQUIRE(layer >= 0 && layer < c->num_layers, PA_ERR_OUT_OF_BOUNDS,
             "layer_idx %d out of bounds for %d layers", layer, c->num_layers);
  const auto it = c->block_hashes[layer].find(hash);
  *block_id = it == c->block_hashes[layer].end() ? -1 : it->second;
  return PA_OK;
}
