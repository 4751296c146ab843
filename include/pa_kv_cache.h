/*
 * pa_kv_cache.h -- host-side mirror of vllm-lite's PagedKvCache over the
 * paged-attention kernels (libpa.so).
 *
 * The reference keeps, per layer, a K and a V tensor of shape
 * [num_blocks, H, 16, D] and exposes write_kv / write_kv_batch / read_kv
 * (crates/model/src/paged_tensor/tensor_store/mod.rs:29-84,
 *  crates/model/src/paged_tensor/tensor_store/buffer.rs:27-339)
 * plus the free functions write_prefill_kv / read_decode_kv
 * (crates/model/src/components/attention/paged_gqa.rs:29-112).  This object
 * owns the device memory of all layers and runs those operations with the
 * HIP kernels, with the reference's argument checks and error codes in
 * place of its `Err` results.  H here is the number of KV heads.
 *
 * Unlike the stateless entry points of pa.h, the cache allocates: the
 * caches themselves at creation, a small device staging buffer for block
 * ids / slots, grown on demand, and one host-mapped word for a single
 * token's block hash.  Index arguments marked "host" are read on the host
 * and validated before anything is enqueued.  Writes return after the
 * stream has run them (their block hashes come back to the host); a
 * read_kv over more than 16 blocks (or from a quantised cache) also waits
 * for its index upload, a shorter one passes the ids in the kernel
 * arguments and returns once the read is enqueued on `stream`.
 */
#ifndef VLLM_LITE_AMD_PA_KV_CACHE_H
#define VLLM_LITE_AMD_PA_KV_CACHE_H

#include "pa.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct pa_kv_cache pa_kv_cache;

/* PagedKvCache::new (tensor_store/mod.rs:50-84): zero-filled caches for
 * num_layers layers.  dtype PA_DTYPE_F32 or PA_DTYPE_BF16. */
int32_t pa_kv_cache_create(int32_t num_layers, int32_t num_kv_heads, int32_t head_dim,
                           int32_t num_blocks, int32_t dtype, pa_kv_cache** out);
void pa_kv_cache_destroy(pa_kv_cache* cache);

/* PagedKvCache::new(..., quantized = true) (tensor_store/mod.rs:50-84): an
 * f32 cache holding int8 values with one scale per block (all 1.0 at
 * creation, mod.rs:69).  Every write re-quantises the block it lands in as
 * write_kv does (buffer.rs:170-231): dequantise with the block's scale,
 * store the token, scale = max(max|K|, max|V|) / 127 (1 for an all-zero
 * block), values round(x / scale); tokens are applied in order.  read_kv
 * returns x * scale + 0.0 per block (buffer.rs:320-331). */
int32_t pa_kv_cache_create_quantized(int32_t num_layers, int32_t num_kv_heads, int32_t head_dim,
                                     int32_t num_blocks, pa_kv_cache** out);
int32_t pa_kv_cache_is_quantized(const pa_kv_cache* cache);
/* Device f32 [num_blocks] block scales of one layer (NULL unless quantised). */
float* pa_kv_cache_scales_ptr(pa_kv_cache* cache, int32_t layer);

/* Accessors (tensor_store/layout.rs:15-44). */
int32_t pa_kv_cache_num_layers(const pa_kv_cache* cache);
int32_t pa_kv_cache_num_blocks(const pa_kv_cache* cache);
int32_t pa_kv_cache_block_size(const pa_kv_cache* cache);
int32_t pa_kv_cache_num_heads(const pa_kv_cache* cache); /* kv heads */
int32_t pa_kv_cache_head_dim(const pa_kv_cache* cache);
int32_t pa_kv_cache_dtype(const pa_kv_cache* cache);
/* Device base of one layer's K cache [NB, H, 16, D] / V cache [NB, H, D, 16];
 * NULL for a bad layer. */
void* pa_kv_cache_key_ptr(pa_kv_cache* cache, int32_t layer);
void* pa_kv_cache_value_ptr(pa_kv_cache* cache, int32_t layer);

/* PagedKvCache::write_kv (buffer.rs:103-267): one token, k / v [H, D]
 * device, into (block_id, token_offset).  PA_ERR_OUT_OF_BOUNDS for a bad
 * layer, block_id >= num_blocks or token_offset >= 16 (buffer.rs:118-137). */
int32_t pa_kv_cache_write_kv(pa_kv_cache* cache, int32_t layer, int64_t block_id,
                             int64_t token_offset, const void* k, const void* v,
                             pa_stream_t stream);

/* PagedKvCache::write_kv_batch (buffer.rs:27-95): T tokens [T, H, D] from
 * (block_id, token_offset) on, continuing into block_id + 1, ... when the
 * offset wraps; fails if the run does not fit the pool (buffer.rs:69-75). */
int32_t pa_kv_cache_write_kv_batch(pa_kv_cache* cache, int32_t layer, int64_t block_id,
                                   int64_t token_offset, const void* k, const void* v,
                                   int32_t num_tokens, pa_stream_t stream);

/* write_prefill_kv (paged_gqa.rs:29-63): token t of k / v [T, H, D] goes to
 * block_ids[pos / 16] at offset pos % 16 with pos = positions[t] (t when
 * positions has fewer than T entries).  block_ids / positions are host
 * arrays.  A position whose block index is past the table is an error here
 * (the reference falls back to block 0, paged_gqa.rs:51).  As in the
 * reference's per-token loop, a slot named twice keeps the later token. */
int32_t pa_kv_cache_write_prefill_kv(pa_kv_cache* cache, int32_t layer, const int64_t* block_ids,
                                     int32_t n_ids, const int64_t* positions, int32_t n_pos,
                                     int32_t num_tokens, const void* k, const void* v,
                                     pa_stream_t stream);

/* PagedKvCache::read_kv (buffer.rs:273-339): the first seq_len tokens of the
 * sequence whose blocks are block_ids (host) into out_k / out_v
 * [seq_len, H, D].  Headroom blocks past seq_len are ignored (:302-304); a
 * table shorter than seq_len yields only the tokens it covers (the walk of
 * :296-333 simply ends); an id >= num_blocks among the walked blocks is an
 * error.  *n_read receives the number of tokens written, min(seq_len,
 * 16 * n_ids) (0 for an empty table or seq_len 0, :279-284). */
int32_t pa_kv_cache_read_kv(pa_kv_cache* cache, int32_t layer, const int64_t* block_ids,
                            int32_t n_ids, int32_t seq_len, void* out_k, void* out_v,
                            int32_t* n_read, pa_stream_t stream);

/* The per-layer block-hash map of PagedKvCache (block_hashes,
 * tensor_store/mod.rs:42): every token written by pa_kv_cache_write_kv /
 * _write_kv_batch / _write_prefill_kv inserts hash -> block_id for the K
 * block it landed in, hashed as the block stands after that token
 * (buffer.rs:263-264, in the tokens' order; an equal hash takes the later
 * block id), with compute_block_hash_from_slice (layout.rs:51-58) over the
 * block's stored K values in [head][token][dim] order (bf16 caches: their
 * bf16 values; quantised caches: the stored integer values).  Its readers
 * in the reference are the multi-node BlockDataSource::has_block and
 * verify_chain_hash (paged_kv_cache_wrapper.rs:100-140), which look at
 * layer 0.  The map lives on the host; writes through pa.h's stateless
 * entry points do not update it.
 *
 * pa_kv_cache_block_hash_count: number of entries of the layer's map.
 * pa_kv_cache_block_hashes: up to `capacity` entries, ascending by hash, into
 *   hashes / block_ids (host); *written receives the count.
 * pa_kv_cache_lookup_block_hash: *block_id = the block recorded for `hash`,
 *   or -1. */
int32_t pa_kv_cache_block_hash_count(const pa_kv_cache* cache, int32_t layer, int64_t* count);
int32_t pa_kv_cache_block_hashes(const pa_kv_cache* cache, int32_t layer, uint64_t* hashes,
                                 int64_t* block_ids, int64_t capacity, int64_t* written);
int32_t pa_kv_cache_lookup_block_hash(const pa_kv_cache* cache, int32_t layer, uint64_t hash,
                                      int64_t* block_id);

/* ---------------------------------------------------------------------- */
/* Batched step (replaces the per-sequence forward loop)                   */
/* ---------------------------------------------------------------------- */

/* One engine step's batch, built once and reused by every layer.  The
 * reference runs attention one sequence at a time
 * (crates/model/src/causal_lm/model/mod.rs:143-164 -> rope_gqa.rs:261-429);
 * a pa_batch holds the device-side index arrays of all sequences so each
 * layer is one scatter plus one attention launch. */
typedef struct pa_batch pa_batch;

int32_t pa_batch_create(pa_batch** out);
void pa_batch_destroy(pa_batch* batch);

/* Describes the step from the scheduler's per-sequence data (the Batch of
 * crates/traits/src/types.rs:84-117), all host arrays:
 *   num_tokens[s]     tokens fed this step (1 for decode)
 *   num_computed[s]   tokens already in the cache (positions start here)
 *   block_ids         all sequences' block tables concatenated (int64)
 *   block_counts[s]   table length of sequence s
 * Token rows of q / k / v / out are the sequences' tokens in order.
 * Validates every table entry against num_blocks (PA_ERR_OUT_OF_BOUNDS) and
 * that each table covers num_computed + num_tokens tokens.  Uploads the
 * index arrays on `stream` without waiting for them (the caller's host
 * arrays may be reused on return): the launches that read the batch
 * (pa_batch_attention, pa_batch_qkv_rope_cache) must be on the same stream.
 * A prepare waits only for the uploads of the prepare two calls back, so
 * the host can prepare step n + 1 while the device runs step n.
 * A call rejected by validation leaves the batch as it was; one that fails
 * later (a HIP allocation, upload or event error) leaves it empty (no
 * tokens: the batch's launches then do nothing). */
int32_t pa_batch_prepare(pa_batch* batch, int32_t num_seqs, const int32_t* num_tokens,
                         const int32_t* num_computed, const int64_t* block_ids,
                         const int32_t* block_counts, int32_t num_blocks, pa_stream_t stream);

int32_t pa_batch_num_tokens(const pa_batch* batch);
/* Fixes the maximum context the decode launches are shaped for (0 = the
 * step's own maximum).  With a capacity, successive decode steps of the same
 * batch size and table width launch identical kernels (sequence lengths are
 * read on the device), so a captured step can be replayed after each
 * pa_batch_prepare.  A step whose context exceeds the capacity is an error.
 * The decode workspace is sized for the capacity on the next call. */
int32_t pa_batch_set_capacity(pa_batch* batch, int32_t max_context_len);
/* 1 when every sequence is a single-token decode step. */
int32_t pa_batch_is_decode(const pa_batch* batch);
/* Advances a prepared decode batch by one token on the device: what
 * pa_batch_prepare with the same block tables and every num_computed one
 * higher would upload (positions, slots, context lengths), computed by one
 * small kernel from the arrays already on the device, with no host upload.
 * No counterpart in the reference (its decode step rebuilds the positions on
 * the host, crates/model/src/components/attention/rope_gqa.rs:385-429): it
 * is for callers that replay a captured decode step, which then advances
 * itself.  Checked at the call against the host's copy of the batch (every
 * sequence's table must hold the advanced context); a replay of a captured
 * call is not checked again, so the caller sizes the tables for every step
 * it replays (as the block tables of a whole generation are allocated up
 * front), and sets a capacity (pa_batch_set_capacity) that covers the
 * context of every replay: the captured decode launches keep the shape of
 * the capture.  Errors: not a decode batch, a table too short, a capture
 * without a capacity. */
int32_t pa_batch_advance(pa_batch* batch, pa_stream_t stream);

/* The prepared batch's fused QKV projection of one layer with RoPE and the
 * KV-cache write in its epilogue: pa_linear_rope_cache with the batch's
 * positions and slots and the layer's caches (bf16 cache, rows = the batch's
 * token count).  out [T, (Hq + 2 Hkv) D]: rotated q (and k), v; pass its q
 * view to pa_batch_attention with key = value = NULL.  weight from
 * pa_linear_pack_qkv; flags 0 or PA_LINEAR_RMS_IN (x's rows normalised on
 * the fly, the norm weight folded into the packed weight). */
int32_t pa_batch_qkv_rope_cache(pa_batch* batch, pa_kv_cache* cache, int32_t layer,
                                int32_t num_heads, void* out, const void* x, const void* weight,
                                const void* bias, int32_t in_features, int32_t flags, float eps,
                                const float* inv_freq, pa_stream_t stream);

/* One layer's attention for the prepared batch: writes the step's K / V
 * into the cache (rotating K, and q in place, when inv_freq is non-NULL),
 * then attends with pa_decode (all-decode batch) or pa_prefill (anything
 * else; decode rows become one-row chunks) into out [T, Hq, D].
 *   q [T, Hq, D] (rotated in place when inv_freq != NULL), key / value
 *   [T, Hkv, D], each with a token stride in elements (0 = contiguous; q, k
 *   and v may be views of one fused QKV projection output), inv_freq [D/2]
 *   device f32 or NULL, scale = attn_factor / sqrt(D).
 * key == value == NULL (and inv_freq NULL): the step's K / V are already in
 * the cache and q is final (pa_batch_qkv_rope_cache ran); attention only.
 * Allocates (once, grown on demand) the decode workspace; a call that would
 * grow it while `stream` is capturing returns PA_ERR_WORKSPACE instead (run
 * one eager step of the captured shape first). */
int32_t pa_batch_attention(pa_batch* batch, pa_kv_cache* cache, int32_t layer, int32_t num_heads,
                           void* q, int64_t q_stride, const void* key, int64_t key_stride,
                           const void* value, int64_t value_stride, const float* inv_freq,
                           float scale, void* out, pa_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* VLLM_LITE_AMD_PA_KV_CACHE_H */
