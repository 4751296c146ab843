// Batched step orchestration (pa_batch_* in pa_kv_cache.h).
//
// The reference's CausalLm::forward_logits loops over sequences and, per
// layer, over RopeGqaAttention::forward_{prefill, prefill_continue, decode}
// (crates/model/src/causal_lm/model/mod.rs:143-164,
//  crates/model/src/components/attention/rope_gqa.rs:261-429), which write
// each token with write_kv and attend with dense candle matmuls.  Here the
// step's index arrays (positions, slots, block tables, query offsets) are
// built once on the host, uploaded once, and every layer runs one write
// launch and one attention launch for the whole batch.
#include <hip/hip_runtime.h>

#include "pa_internal.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "../../include/pa_dense.h"
#include "../../include/pa_kv_cache.h"
#include "pa_common.hpp"

struct pa_kv_cache;  // layout shared with kv_cache.cpp through the accessors

namespace {

// Device buffer that only grows.
struct DevBuf {
  void* ptr = nullptr;
  size_t bytes = 0;
  int32_t ensure(size_t need) {
    if (need <= bytes) return PA_OK;
    // queued work may still read the old array (uploads and launches are
    // stream-ordered, the host does not wait for them)
    if (ptr) {
      (void)hipDeviceSynchronize();
      (void)hipFree(ptr);
    }
    ptr = nullptr;
    bytes = 0;
    if (hipMalloc(&ptr, need) != hipSuccess) {
      pa::set_error("pa_batch: device allocation of %zu bytes failed", need);
      return PA_ERR_HIP;
    }
    bytes = need;
    return PA_OK;
  }
  ~DevBuf() {
    if (ptr) (void)hipFree(ptr);
  }
};

// A region of the batch's index buffer.
struct Region {
  void* ptr = nullptr;
  size_t bytes = 0;
};

}  // namespace

struct pa_batch {
  int num_seqs = 0, num_tokens = 0, max_blocks = 0, max_q = 0, max_ctx = 0, num_blocks = 0;
  int capacity = 0;  // fixed max context for decode launches (0 = per step)
  bool decode = false;
  // host copies for pa_batch_advance's checks: per sequence the context
  // length and the tokens its block table holds
  std::vector<int32_t> host_ctx, host_cap;
  // device arrays: the index arrays are regions of one buffer (one upload
  // per prepare), at offsets that only change when a region must grow
  DevBuf index_buf, workspace;
  Region positions, slots, tables, cu_q, past, ctx_lens;
  // pinned staging, two slots used in turn: a prepare waits (on the event
  // recorded after its uploads) only for the uploads of the prepare two
  // calls back, so the host can prepare the next step while the device
  // still runs the current one
  void* stage[2] = {nullptr, nullptr};
  size_t stage_bytes[2] = {0, 0};
  hipEvent_t uploaded[2] = {nullptr, nullptr};
  bool pending[2] = {false, false};
  int slot = 0;
  ~pa_batch() {
    for (int i = 0; i < 2; ++i) {
      if (pending[i]) (void)hipEventSynchronize(uploaded[i]);
      if (uploaded[i]) (void)hipEventDestroy(uploaded[i]);
      if (stage[i]) (void)hipHostFree(stage[i]);
    }
  }
};

extern "C" int32_t pa_batch_create(pa_batch** out) {
  pa::clear_error();
  PA_REQUIRE(out, PA_ERR_INVALID_ARG, "pa_batch_create: null out");
  *out = new pa_batch();
  return PA_OK;
}

extern "C" void pa_batch_destroy(pa_batch* b) { delete b; }

extern "C" int32_t pa_batch_num_tokens(const pa_batch* b) { return b ? b->num_tokens : 0; }

extern "C" int32_t pa_batch_set_capacity(pa_batch* b, int32_t max_context_len) {
  pa::clear_error();
  PA_REQUIRE(b && max_context_len >= 0, PA_ERR_INVALID_ARG, "pa_batch_set_capacity: bad arguments");
  b->capacity = max_context_len;
  return PA_OK;
}
extern "C" int32_t pa_batch_is_decode(const pa_batch* b) { return b && b->decode ? 1 : 0; }

extern "C" int32_t pa_batch_prepare(pa_batch* b, int32_t num_seqs, const int32_t* num_tokens,
                                    const int32_t* num_computed, const int64_t* block_ids,
                                    const int32_t* block_counts, int32_t num_blocks,
                                    pa_stream_t stream) {
  pa::clear_error();
  PA_REQUIRE(b && num_seqs >= 0 && num_blocks > 0, PA_ERR_INVALID_ARG,
             "pa_batch_prepare: bad arguments");
  PA_REQUIRE(num_seqs == 0 || (num_tokens && num_computed && block_counts), PA_ERR_INVALID_ARG,
             "pa_batch_prepare: null per-sequence array");
  int64_t total_ids = 0, total_tokens = 0;
  int max_blocks = 1, max_q = 0, max_ctx = 0;
  bool decode = num_seqs > 0;
  for (int s = 0; s < num_seqs; ++s) {
    PA_REQUIRE(num_tokens[s] >= 0 && num_computed[s] >= 0 && block_counts[s] >= 0,
               PA_ERR_INVALID_ARG, "pa_batch_prepare: negative count for sequence %d", s);
    const int64_t ctx = (int64_t)num_computed[s] + num_tokens[s];
    PA_REQUIRE(ctx <= (int64_t)block_counts[s] * pa::kBlock, PA_ERR_OUT_OF_BOUNDS,
               "pa_batch_prepare: sequence %d needs %lld tokens, its table holds %d blocks", s,
               (long long)ctx, block_counts[s]);
    total_ids += block_counts[s];
    total_tokens += num_tokens[s];
    max_blocks = std::max(max_blocks, block_counts[s]);
    max_q = std::max(max_q, num_tokens[s]);
    max_ctx = std::max<int>(max_ctx, (int)ctx);
    decode = decode && num_tokens[s] == 1 && num_computed[s] > 0;
  }
  PA_REQUIRE(total_ids == 0 || block_ids, PA_ERR_INVALID_ARG, "pa_batch_prepare: null block_ids");
  PA_REQUIRE(total_tokens < (1ll << 31), PA_ERR_INVALID_ARG, "pa_batch_prepare: too many tokens");
  for (int64_t i = 0; i < total_ids; ++i)
    PA_REQUIRE(block_ids[i] >= 0 && block_ids[i] < num_blocks, PA_ERR_OUT_OF_BOUNDS,
               "block_id %lld out of bounds for %d blocks", (long long)block_ids[i], num_blocks);

  // From here on the previous step's arrays are being replaced: until this
  // call succeeds the batch is empty (attention on it does nothing), so a
  // failure below never pairs old counts with new, partly written arrays.
  b->num_seqs = 0;
  b->num_tokens = 0;
  b->decode = false;

  // Host images of the index arrays, packed into one staging buffer.
  const int T = (int)total_tokens;
  std::vector<int64_t> pos(T), slot(T);
  std::vector<int32_t> table((size_t)num_seqs * max_blocks, 0), cu(num_seqs + 1, 0),
      past(num_seqs), ctxl(num_seqs);
  int64_t id_off = 0;
  int t = 0;
  for (int s = 0; s < num_seqs; ++s) {
    for (int i = 0; i < block_counts[s]; ++i)
      table[(size_t)s * max_blocks + i] = (int32_t)block_ids[id_off + i];
    for (int i = 0; i < num_tokens[s]; ++i, ++t) {
      const int64_t p = (int64_t)num_computed[s] + i;
      pos[t] = p;
      slot[t] = block_ids[id_off + p / pa::kBlock] * pa::kBlock + p % pa::kBlock;
    }
    id_off += block_counts[s];
    cu[s + 1] = cu[s] + num_tokens[s];
    past[s] = num_computed[s];
    ctxl[s] = num_computed[s] + num_tokens[s];
  }
  const size_t b_pos = pos.size() * 8, b_slot = slot.size() * 8, b_tab = table.size() * 4,
               b_cu = cu.size() * 4, b_past = past.size() * 4, b_ctx = ctxl.size() * 4;
  const int sl = b->slot;
  if (b->pending[sl]) {  // this slot's previous uploads have been read
    if (hipEventSynchronize(b->uploaded[sl]) != hipSuccess) {
      pa::set_error("pa_batch_prepare: waiting for an earlier upload failed");
      return PA_ERR_HIP;
    }
    b->pending[sl] = false;
  }
  if (!b->uploaded[sl] &&
      hipEventCreateWithFlags(&b->uploaded[sl], hipEventDisableTiming) != hipSuccess) {
    pa::set_error("pa_batch_prepare: event creation failed");
    return PA_ERR_HIP;
  }
  Region* regs[6] = {&b->positions, &b->slots, &b->tables, &b->cu_q, &b->past, &b->ctx_lens};
  const size_t need[6] = {std::max<size_t>(b_pos, 8),  std::max<size_t>(b_slot, 8),
                          std::max<size_t>(b_tab, 4),  std::max<size_t>(b_cu, 4),
                          std::max<size_t>(b_past, 4), std::max<size_t>(b_ctx, 4)};
  bool grow = false;
  for (int i = 0; i < 6; ++i) grow = grow || need[i] > regs[i]->bytes;
  hipStream_t s = (hipStream_t)stream;
  if (grow) {
    // New region capacities (twice the old, at least the need, 256-byte
    // aligned).  The buffer is replaced: wait for the work queued on the
    // stream (it may still read the old one) first.
    if (hipStreamSynchronize(s) != hipSuccess) {
      pa::set_error("pa_batch_prepare: stream synchronisation failed");
      return PA_ERR_HIP;
    }
    size_t cap[6], total = 0;
    for (int i = 0; i < 6; ++i) {
      cap[i] = (std::max(need[i], 2 * regs[i]->bytes) + 255) / 256 * 256;
      total += cap[i];
    }
    int32_t rc = b->index_buf.ensure(total);
    if (rc != PA_OK) {
      // the old buffer is gone: no region may point into it
      for (int i = 0; i < 6; ++i) *regs[i] = Region{};
      return rc;
    }
    size_t off = 0;
    for (int i = 0; i < 6; ++i) {
      regs[i]->ptr = (char*)b->index_buf.ptr + off;
      regs[i]->bytes = cap[i];
      off += cap[i];
    }
  }
  // the upload spans the regions up to the end of the last one used
  const size_t span = (size_t)((char*)b->ctx_lens.ptr - (char*)b->index_buf.ptr) + b_ctx;
  if (span > b->stage_bytes[sl]) {
    if (b->stage[sl]) (void)hipHostFree(b->stage[sl]);
    b->stage[sl] = nullptr;
    b->stage_bytes[sl] = 0;
    if (hipHostMalloc(&b->stage[sl], span, hipHostMallocDefault) != hipSuccess) {
      pa::set_error("pa_batch_prepare: pinned staging of %zu bytes failed", span);
      return PA_ERR_HIP;
    }
    b->stage_bytes[sl] = span;
  }
  char* st = (char*)b->stage[sl];
  const void* src[6] = {pos.data(), slot.data(), table.data(), cu.data(), past.data(), ctxl.data()};
  const size_t bytes[6] = {b_pos, b_slot, b_tab, b_cu, b_past, b_ctx};
  for (int i = 0; i < 6; ++i)
    if (bytes[i]) std::memcpy(st + ((char*)regs[i]->ptr - (char*)b->index_buf.ptr), src[i], bytes[i]);
  if (span > 0 && hipMemcpyAsync(b->index_buf.ptr, st, span, hipMemcpyHostToDevice, s) != hipSuccess) {
    pa::set_error("pa_batch_prepare: upload failed");
    return PA_ERR_HIP;
  }
  if (hipEventRecord(b->uploaded[sl], s) != hipSuccess) {
    pa::set_error("pa_batch_prepare: event record failed");
    return PA_ERR_HIP;
  }
  b->pending[sl] = true;
  b->slot = sl ^ 1;
  b->host_ctx.assign(ctxl.begin(), ctxl.end());
  b->host_cap.resize(num_seqs);
  for (int s2 = 0; s2 < num_seqs; ++s2) b->host_cap[s2] = block_counts[s2] * pa::kBlock;
  b->num_seqs = num_seqs;
  b->num_tokens = T;
  b->max_blocks = max_blocks;
  b->max_q = max_q;
  b->max_ctx = max_ctx;
  b->num_blocks = num_blocks;
  b->decode = decode;
  return PA_OK;
}

namespace {
// One decode token per sequence: the next position, its slot in the
// sequence's (already uploaded) block table, the context one longer.
__global__ __launch_bounds__(256) void batch_advance_kernel(int64_t* __restrict__ pos,
                                                            int64_t* __restrict__ slots,
                                                            const int32_t* __restrict__ tables,
                                                            int32_t* __restrict__ ctx_lens,
                                                            int max_blocks, int num_seqs) {
  const int s = blockIdx.x * blockDim.x + threadIdx.x;
  if (s >= num_seqs) return;
  const int64_t p = pos[s] + 1;
  const int64_t bi = p / pa::kBlock;
  // a table too short (a replay the caller did not size for) writes nowhere
  const int32_t blk = bi < max_blocks ? tables[(int64_t)s * max_blocks + bi] : -1;
  pos[s] = p;
  slots[s] = blk < 0 ? -1 : (int64_t)blk * pa::kBlock + p % pa::kBlock;
  ctx_lens[s] = (int32_t)(p + 1);
}
}  // namespace

extern "C" int32_t pa_batch_advance(pa_batch* b, pa_stream_t stream) {
  pa::clear_error();
  PA_REQUIRE(b, PA_ERR_INVALID_ARG, "pa_batch_advance: null batch");
  PA_REQUIRE(b->decode && b->num_seqs > 0, PA_ERR_INVALID_ARG,
             "pa_batch_advance: the batch is not a prepared decode step");
  for (int s = 0; s < b->num_seqs; ++s)
    PA_REQUIRE(b->host_ctx[s] + 1 <= b->host_cap[s], PA_ERR_OUT_OF_BOUNDS,
               "pa_batch_advance: sequence %d needs %d tokens, its table holds %d", s,
               b->host_ctx[s] + 1, b->host_cap[s]);
  // A captured advance replays without this check, and the captured decode
  // launches keep the shape of the capture: only a capacity (the shape of
  // every replay) makes them cover the contexts of later replays.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  PA_REQUIRE(hipStreamIsCapturing((hipStream_t)stream, &cap) == hipSuccess &&
                 (cap == hipStreamCaptureStatusNone || b->capacity > 0),
             PA_ERR_INVALID_ARG,
             "pa_batch_advance: capturing without a capacity (pa_batch_set_capacity)");
  for (int s = 0; s < b->num_seqs; ++s) ++b->host_ctx[s];
  ++b->max_ctx;
  batch_advance_kernel<<<(b->num_seqs + 255) / 256, 256, 0, (hipStream_t)stream>>>(
      (int64_t*)b->positions.ptr, (int64_t*)b->slots.ptr, (const int32_t*)b->tables.ptr,
      (int32_t*)b->ctx_lens.ptr, b->max_blocks, b->num_seqs);
  return pa::check_launch("pa_batch_advance");
}

extern "C" int32_t pa_batch_attention(pa_batch* b, pa_kv_cache* cache, int32_t layer,
                                      int32_t num_heads, void* q, int64_t q_stride,
                                      const void* key, int64_t key_stride, const void* value,
                                      int64_t value_stride, const float* inv_freq, float scale,
                                      void* out, pa_stream_t stream) {
  pa::clear_error();
  PA_REQUIRE(b && cache, PA_ERR_INVALID_ARG, "pa_batch_attention: null batch or cache");
  void* kc = pa_kv_cache_key_ptr(cache, layer);
  void* vc = pa_kv_cache_value_ptr(cache, layer);
  PA_REQUIRE(kc && vc, PA_ERR_OUT_OF_BOUNDS, "layer_idx %d out of bounds for %d layers", layer,
             pa_kv_cache_num_layers(cache));
  PA_REQUIRE(pa_kv_cache_num_blocks(cache) == b->num_blocks, PA_ERR_INVALID_ARG,
             "pa_batch_attention: batch prepared for %d blocks, cache has %d", b->num_blocks,
             pa_kv_cache_num_blocks(cache));
  if (b->num_tokens == 0) return PA_OK;
  const int hkv = pa_kv_cache_num_heads(cache), d = pa_kv_cache_head_dim(cache);
  const int dtype = pa_kv_cache_dtype(cache);
  PA_REQUIRE(num_heads > 0 && num_heads % hkv == 0, PA_ERR_INVALID_ARG,
             "pa_batch_attention: num_heads %d not a multiple of num_kv_heads %d", num_heads, hkv);
  PA_REQUIRE(q && out && (key != nullptr) == (value != nullptr), PA_ERR_INVALID_ARG,
             "pa_batch_attention: null tensor");
  PA_REQUIRE(key || !inv_freq, PA_ERR_INVALID_ARG,
             "pa_batch_attention: inv_freq without key / value (rotated where written)");
  const int64_t* slots = (const int64_t*)b->slots.ptr;
  int32_t rc = PA_OK;
  if (!key) {
    // the step's K / V were written by pa_batch_qkv_rope_cache
  } else if (inv_freq) {
    rc = pa_rope_reshape_and_cache(q, q_stride, key, key_stride, value, value_stride, kc, vc,
                                   slots, (const int64_t*)b->positions.ptr, inv_freq,
                                   b->num_tokens, num_heads, hkv, d, b->num_blocks, dtype,
                                   stream);
  } else {
    rc = pa_reshape_and_cache(key, value, kc, vc, slots, b->num_tokens, hkv, d, b->num_blocks,
                              key_stride, value_stride, dtype, stream);
  }
  if (rc != PA_OK) return rc;
  if (b->decode) {
    // With a capacity the launch shape depends on it alone (sequences read
    // their own lengths on the device), so the call can be replayed.
    PA_REQUIRE(b->capacity == 0 || b->max_ctx <= b->capacity, PA_ERR_INVALID_ARG,
               "pa_batch_attention: context %d exceeds the capacity %d", b->max_ctx,
               b->capacity);
    const int max_ctx = b->capacity > 0 ? b->capacity : b->max_ctx;
    const size_t need = std::max<size_t>(
        pa_decode_workspace_size(b->num_seqs, num_heads, d, max_ctx), 256);
    if (need > b->workspace.bytes) {
      // growing frees and allocates, which a stream capture cannot record
      hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
      PA_REQUIRE(hipStreamIsCapturing((hipStream_t)stream, &cap) == hipSuccess &&
                     cap == hipStreamCaptureStatusNone,
                 PA_ERR_WORKSPACE,
                 "pa_batch_attention: the decode workspace must grow to %zu bytes while the "
                 "stream is capturing; run one eager step of this shape before the capture",
                 need);
      if ((rc = b->workspace.ensure(need))) return rc;
    }
    return pa::decode_strided(out, q, q_stride, kc, vc, (const int32_t*)b->tables.ptr,
                              b->max_blocks, (const int32_t*)b->ctx_lens.ptr, max_ctx,
                              b->num_seqs, num_heads, hkv, d, b->num_blocks, scale,
                              b->workspace.ptr, b->workspace.bytes, dtype, stream);
  }
  return pa::prefill_strided(out, q, q_stride, kc, vc, (const int32_t*)b->tables.ptr,
                             b->max_blocks, (const int32_t*)b->cu_q.ptr,
                             (const int32_t*)b->past.ptr, b->num_seqs, b->num_tokens, b->max_q,
                             num_heads, hkv, d, b->num_blocks, scale, dtype, stream);
}

extern "C" int32_t pa_batch_qkv_rope_cache(pa_batch* b, pa_kv_cache* cache, int32_t layer,
                                           int32_t num_heads, void* out, const void* x,
                                           const void* weight, const void* bias,
                                           int32_t in_features, int32_t flags, float eps,
                                           const float* inv_freq, pa_stream_t stream) {
  pa::clear_error();
  PA_REQUIRE(b && cache, PA_ERR_INVALID_ARG, "pa_batch_qkv_rope_cache: null batch or cache");
  void* kc = pa_kv_cache_key_ptr(cache, layer);
  void* vc = pa_kv_cache_value_ptr(cache, layer);
  PA_REQUIRE(kc && vc, PA_ERR_OUT_OF_BOUNDS, "layer_idx %d out of bounds for %d layers", layer,
             pa_kv_cache_num_layers(cache));
  PA_REQUIRE(pa_kv_cache_num_blocks(cache) == b->num_blocks, PA_ERR_INVALID_ARG,
             "pa_batch_qkv_rope_cache: batch prepared for %d blocks, cache has %d",
             b->num_blocks, pa_kv_cache_num_blocks(cache));
  const int hkv = pa_kv_cache_num_heads(cache), d = pa_kv_cache_head_dim(cache);
  PA_REQUIRE(num_heads > 0 && num_heads % hkv == 0, PA_ERR_INVALID_ARG,
             "pa_batch_qkv_rope_cache: num_heads %d not a multiple of num_kv_heads %d",
             num_heads, hkv);
  return pa_linear_rope_cache(out, x, weight, bias, b->num_tokens, num_heads, hkv, d,
                              in_features, flags, eps, (const int64_t*)b->positions.ptr,
                              (const int64_t*)b->slots.ptr, inv_freq, kc, vc, b->num_blocks,
                              pa_kv_cache_dtype(cache), stream);
}
