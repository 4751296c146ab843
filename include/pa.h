/*
 * pa.h -- C ABI of the MI355X paged-attention library (libpa.so).
 *
 * This is the drop-in boundary for vllm-lite's paged-attention path: the
 * KV-cache write (slot-mapping scatter into 16-token blocks) and attention
 * over the block-table-addressed cache, for single-token decode and for
 * chunked causal prefill.  Each entry point names the reference function it
 * replaces (paths relative to the vllm-lite repository root).
 *
 * Conventions
 *  - Every pointer argument is a device pointer unless the comment says
 *    "host".  The caller owns all memory; the stateless entry points
 *    allocate nothing.  Work is enqueued on `stream` (NULL = the default
 *    stream); nothing synchronises unless stated.
 *  - Return value: PA_OK (0) or a negative pa_status.  No entry point aborts,
 *    throws or unwinds; pa_last_error() gives a message for the calling
 *    thread's most recent failure.
 *  - dtype: PA_DTYPE_F32 or PA_DTYPE_BF16, shared by q, k, v, the caches and
 *    out.  Arithmetic accumulates in f32.  PA_DTYPE_FP8_E4M3 selects one-byte
 *    caches in the reference's FP8 convention
 *    (crates/model/src/components/kv_cache_fp8.rs:143-212); with it q and out
 *    are bf16, K / V are written by pa_reshape_and_cache_fp8 and pa_read_kv
 *    returns f32.
 *  - Block size is fixed at 16 tokens (crates/traits/src/types.rs:13).
 *
 * Cache layout (one layer, one of K / V; num_blocks = NB, kv heads = Hkv):
 *   K cache  [NB, Hkv, 16, D]  token-major inside a block, as the reference
 *            (crates/model/src/paged_tensor/tensor_store/mod.rs:62)
 *   V cache  [NB, Hkv, D, 16]  token-minor inside a block: one head's 16
 *            values of a dimension are contiguous, so the P·V contraction
 *            loads matrix-core operands directly.  pa_read_kv returns the
 *            reference's [seq, H, D] view, so logical contents are identical.
 *   The cache stores Hkv heads; the reference stores the expanded Hq heads
 *   (crates/model/src/components/attention/rope_gqa.rs:287-302).  Query head
 *   h reads kv head h / (Hq / Hkv) (blocked grouping, util.rs:55-87).
 */
#ifndef VLLM_LITE_AMD_PA_H
#define VLLM_LITE_AMD_PA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* pa_stream_t; /* same type as hipStream_t */

#define PA_BLOCK_SIZE 16

typedef enum pa_dtype { PA_DTYPE_F32 = 0, PA_DTYPE_BF16 = 1, PA_DTYPE_FP8_E4M3 = 2 } pa_dtype;

typedef enum pa_status {
  PA_OK = 0,
  PA_ERR_INVALID_ARG = -1,  /* bad shape, null pointer, unknown dtype */
  PA_ERR_OUT_OF_BOUNDS = -2, /* layer / block / offset outside the cache */
  PA_ERR_UNSUPPORTED = -3,  /* shape this build has no kernel for */
  PA_ERR_WORKSPACE = -4,    /* workspace missing or too small */
  PA_ERR_HIP = -5           /* a HIP runtime call failed */
} pa_status;

/* Message for the calling thread's last failed call ("" if none). */
const char* pa_last_error(void);

/* Library version string. */
const char* pa_version(void);

/* ---------------------------------------------------------------------- */
/* KV-cache write                                                         */
/* ---------------------------------------------------------------------- */

/* Scatter T tokens' K and V into the cache: token t goes to block
 * slot_mapping[t] / 16, offset slot_mapping[t] % 16.  Slots < 0 or
 * >= num_blocks * 16 are skipped.  Slots are expected to be distinct (as a
 * scheduler's slot mapping is): the reference writes tokens in order, so a
 * repeated slot keeps the last token's K / V, while here which of them
 * survives is unspecified.
 *   key, value    [T, Hkv, D] with token strides key_stride / value_stride
 *                 (elements; 0 means Hkv * D, i.e. contiguous)
 *   slot_mapping  [T] int64
 * Replaces the per-token write loop of write_prefill_kv
 * (crates/model/src/components/attention/paged_gqa.rs:29-63), the decode
 * write in read_decode_kv (paged_gqa.rs:86-107), and PagedKvCache::write_kv
 * (crates/model/src/paged_tensor/tensor_store/buffer.rs:103-267). */
int32_t pa_reshape_and_cache(const void* key, const void* value, void* k_cache, void* v_cache,
                             const int64_t* slot_mapping, int32_t num_tokens,
                             int32_t num_kv_heads, int32_t head_dim, int32_t num_blocks,
                             int64_t key_stride, int64_t value_stride, int32_t dtype,
                             pa_stream_t stream);

/* pa_reshape_and_cache into FP8 caches (PA_DTYPE_FP8_E4M3, one byte per
 * element, same block layouts): every element is quantised with the
 * reference's encoder, Fp8Quantizer::quantize / float32_to_fp8_e4m3
 * (crates/model/src/components/kv_cache_fp8.rs:59-68, :143-186), bit for
 * bit.  key / value are src_dtype (PA_DTYPE_F32 or PA_DTYPE_BF16) with
 * token strides in elements (0 = contiguous). */
int32_t pa_reshape_and_cache_fp8(const void* key, const void* value, uint8_t* k_cache,
                                 uint8_t* v_cache, const int64_t* slot_mapping, int32_t num_tokens,
                                 int32_t num_kv_heads, int32_t head_dim, int32_t num_blocks,
                                 int64_t key_stride, int64_t value_stride, int32_t src_dtype,
                                 pa_stream_t stream);

/* pa_reshape_and_cache_fp8 that also keeps per-block flags for
 * pa_decode_fp8_flagged: block_flags [num_blocks] (device, one byte per
 * block) gets 1 at every block that receives a code the hardware E4M3
 * conversion reads differently from the reference's decode (the NaN and
 * +-inf codes the encoder gives non-finite input,
 * crates/model/src/components/kv_cache_fp8.rs:143-212).  Flags are only
 * ever set; the caller zeroes them (e.g. when it hands a block to a new
 * sequence).  No reference counterpart: the reference decodes every code
 * on the host. */
int32_t pa_reshape_and_cache_fp8_flagged(const void* key, const void* value, uint8_t* k_cache,
                                         uint8_t* v_cache, const int64_t* slot_mapping,
                                         int32_t num_tokens, int32_t num_kv_heads,
                                         int32_t head_dim, int32_t num_blocks,
                                         int64_t key_stride, int64_t value_stride,
                                         int32_t src_dtype, uint8_t* block_flags,
                                         pa_stream_t stream);

/* Build slot_mapping on the device from per-sequence block tables:
 *   slot_mapping[t] = block_tables[s, positions[t] / 16] * 16 + positions[t] % 16
 * for t in [cu_seq_tokens[s], cu_seq_tokens[s+1]).  A position whose block
 * index is beyond max_blocks_per_seq maps to -1 (skipped by the scatter).
 *   block_tables [num_seqs, max_blocks_per_seq] int32, positions [T] int64,
 *   cu_seq_tokens [num_seqs + 1] int32, slot_mapping [T] int64 (out).
 * Replaces the index arithmetic of paged_gqa.rs:39-52 and :86-97.  The
 * reference silently falls back to block 0 for a missing table entry
 * (paged_gqa.rs:51, :97); here such tokens are skipped instead.  Offsets
 * outside [0, num_tokens] are clamped on the device (a caller error: the
 * tokens concerned get no slot written). */
int32_t pa_slot_mapping(const int32_t* block_tables, int32_t max_blocks_per_seq,
                        const int64_t* positions, const int32_t* cu_seq_tokens,
                        int32_t num_seqs, int32_t num_tokens, int64_t* slot_mapping,
                        pa_stream_t stream);

/* Rotary embedding fused with the cache write.  Token t (position
 * positions[t], int64) has its query heads rotated in place in q
 * [T, Hq, D] (token stride q_stride), its key heads rotated and written to
 * the K cache at slot_mapping[t], and its value heads written to the V cache
 * at the same slot (slots outside the pool write nothing; Q is still
 * rotated).  Rotation of each head: with x1 = x[0:D/2], x2 = x[D/2:D],
 * angle_i = positions[t] * inv_freq[i] (f32),
 *   x1' = x1 cos - x2 sin,   x2' = x2 cos + x1 sin.
 *   inv_freq  [D/2] f32 device array (see pa_rope_inv_freq).
 * Strides of 0 mean contiguous.
 * Replaces RoPE::apply_with_scaling on Q and K
 * (crates/model/src/components/positional/rope.rs:171-174, 507-568)
 * followed by the KV write of rope_gqa.rs:283-302 / paged_gqa.rs:29-63. */
int32_t pa_rope_reshape_and_cache(void* q, int64_t q_stride, const void* key, int64_t key_stride,
                                  const void* value, int64_t value_stride, void* k_cache,
                                  void* v_cache, const int64_t* slot_mapping,
                                  const int64_t* positions, const float* inv_freq,
                                  int32_t num_tokens, int32_t num_heads, int32_t num_kv_heads,
                                  int32_t head_dim, int32_t num_blocks, int32_t dtype,
                                  pa_stream_t stream);

typedef enum pa_rope_type {
  PA_ROPE_DEFAULT = 0,
  PA_ROPE_LINEAR = 1,
  PA_ROPE_YARN = 2,
  PA_ROPE_DYNAMIC = 3,
  PA_ROPE_SU = 4
} pa_rope_type;

/* Host function: the RoPE inverse-frequency table out[D/2] (host memory)
 * for the reference's scaling types (rope.rs:335-505): default
 * theta^(-2i/D); linear divides by `factor`; YaRN uses
 * theta * factor^(D/(D-2)); dynamic NTK recomputes the factor from
 * cur_seq_len when it exceeds original_max_position; Su divides by
 * short_factor / long_factor (host arrays of D/2, NULL = 1) on either side
 * of the dimension whose wavelength first exceeds original_max_position.
 * A factor within f32 epsilon of 1 keeps the default table. */
int32_t pa_rope_inv_freq(int32_t head_dim, float theta, int32_t rope_type, float factor,
                         int32_t original_max_position, int32_t cur_seq_len,
                         const float* short_factor, const float* long_factor, float* out);

/* ---------------------------------------------------------------------- */
/* KV-cache read                                                          */
/* ---------------------------------------------------------------------- */

/* Gather the first seq_len tokens of one sequence into dense
 * out_k / out_v [seq_len, Hkv, D] (reference layout, bit-exact copies).
 *   block_ids [n_ids] int32; block b holds tokens [16b, 16b + 16).
 * Requires n_ids * 16 >= seq_len.  Entries outside [0, num_blocks) produce
 * zero rows.  With PA_DTYPE_FP8_E4M3 caches the outputs are f32, each
 * element the reference's dequantised value (Fp8Quantizer::dequantize,
 * kv_cache_fp8.rs:70-88, :188-212: f16-exact, NaN / +-inf codes kept).
 * Replaces PagedKvCache::read_kv
 * (crates/model/src/paged_tensor/tensor_store/buffer.rs:273-339). */
int32_t pa_read_kv(const void* k_cache, const void* v_cache, const int32_t* block_ids,
                   int32_t n_ids, int32_t seq_len, int32_t num_kv_heads, int32_t head_dim,
                   int32_t num_blocks, void* out_k, void* out_v, int32_t dtype,
                   pa_stream_t stream);

/* Content hash of each listed block of an f32 K cache, computed as
 *   fold(0, acc * 31 + (|x| * 1000) as u64) over the block's H*16*D values
 * in the reference's [H, 16, D] order (wrapping u64 arithmetic; the cast
 * saturates like Rust's `as`).
 *   block_ids [n] int32, hashes [n] uint64 (out).
 * Replaces PagedKvCache::compute_block_hash_from_slice
 * (crates/model/src/paged_tensor/tensor_store/layout.rs:51-58). */
int32_t pa_block_hash(const float* k_cache, const int32_t* block_ids, int32_t n,
                      int32_t num_kv_heads, int32_t head_dim, int32_t num_blocks,
                      uint64_t* hashes, pa_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Attention                                                              */
/* ---------------------------------------------------------------------- */

/* Bytes of workspace pa_decode needs for these sizes (0 when one pass
 * suffices). */
size_t pa_decode_workspace_size(int32_t num_seqs, int32_t num_heads, int32_t head_dim,
                                int32_t max_context_len);

/* Single-token decode attention over the paged cache.
 *   out, q        [num_seqs, Hq, D]
 *   block_tables  [num_seqs, max_blocks_per_seq] int32
 *   context_lens  [num_seqs] int32: keys 0 .. context_lens[s]-1 are attended
 *                 (the new token must already be in the cache)
 *   max_context_len  host upper bound of context_lens (sizes the split and
 *                 the workspace); a sequence whose context_lens entry is
 *                 above it (a caller error) gets an unspecified result for
 *                 its rows, and nothing outside out and the workspace is
 *                 written
 *   scale         softmax scale, e.g. attn_factor / sqrt(D)
 *   workspace     pa_decode_workspace_size() bytes (may be NULL if 0)
 * out[s, h] = softmax(scale * q[s, h] · K[s, h/g]ᵀ) · V[s, h/g].
 * A table entry outside [0, num_blocks) contributes no keys (its 16
 * positions are masked); the reference would fail on such an id instead
 * (candle's narrow in read_kv), and its scheduler never produces one.
 * Replaces RopeGqaAttention::forward_decode's attention
 * (crates/model/src/components/attention/rope_gqa.rs:385-429) =
 * read_decode_kv + expand_kv + paged_attention
 * (paged_gqa.rs:71-112, util.rs:55-87, util.rs:150-176). */
int32_t pa_decode(void* out, const void* q, const void* k_cache, const void* v_cache,
                  const int32_t* block_tables, int32_t max_blocks_per_seq,
                  const int32_t* context_lens, int32_t max_context_len, int32_t num_seqs,
                  int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t num_blocks,
                  float scale, void* workspace, size_t workspace_bytes, int32_t dtype,
                  pa_stream_t stream);

/* pa_decode on FP8-E4M3 caches (dtype implied) whose blocks carry the flags
 * of pa_reshape_and_cache_fp8_flagged: blocks whose flag is 0 are converted
 * by the hardware (exact for every code but the flagged ones) without the
 * per-code test pa_decode makes on every byte it streams; a partition that
 * reads a flagged block is attended again with the reference's exact
 * decode.  Same results as pa_decode as long as every code the flags
 * describe was written through the flagged writer (a block written any
 * other way with a NaN / inf code and flag 0 would read as the hardware
 * conversion does).  block_flags [num_blocks], device.  Replaces the same
 * reference functions as pa_decode. */
int32_t pa_decode_fp8_flagged(void* out, const void* q, const void* k_cache, const void* v_cache,
                              const int32_t* block_tables, int32_t max_blocks_per_seq,
                              const int32_t* context_lens, int32_t max_context_len,
                              int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                              int32_t head_dim, int32_t num_blocks, float scale, void* workspace,
                              size_t workspace_bytes, const uint8_t* block_flags,
                              pa_stream_t stream);

/* pa_decode without a workspace argument and without any allocation.  No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops or harnesses
 * that forbid hipMalloc).  Arguments and results are those of pa_decode;
 * the split-K partial results go to a fixed device array inside the library
 * (pa_decode_noalloc_scratch_bytes() bytes, 64 MiB, one per GPU, held until
 * the process ends; its address is looked up once per device on the first
 * call).  Sizes whose split needs more (pa_decode_workspace_size() bounds
 * it) return PA_ERR_WORKSPACE without launching.  The stream must belong to
 * the calling thread's current device (PA_ERR_INVALID_ARG otherwise).  Calls
 * on one GPU share the array: calls that may overlap (other streams, other
 * threads) race. */
int32_t pa_decode_noalloc(void* out, const void* q, const void* k_cache, const void* v_cache,
                          const int32_t* block_tables, int32_t max_blocks_per_seq,
                          const int32_t* context_lens, int32_t max_context_len,
                          int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                          int32_t head_dim, int32_t num_blocks, float scale, int32_t dtype,
                          pa_stream_t stream);

/* Bytes of pa_decode_noalloc's fixed split-K scratch.  No reference
 * counterpart. */
size_t pa_decode_noalloc_scratch_bytes(void);

/* pa_decode over a quantised PagedKvCache (int8 values in f32 caches with
 * one scale per block, pa_kv_cache_create_quantized): every K / V element
 * is read as value * block_scales[block], which is what the reference's
 * read_kv returns for such a cache (buffer.rs:320-331) before attention.
 * f32 q / out; block_scales device f32 [num_blocks]. */
int32_t pa_decode_quantized(void* out, const void* q, const float* k_cache, const float* v_cache,
                            const float* block_scales, const int32_t* block_tables,
                            int32_t max_blocks_per_seq, const int32_t* context_lens,
                            int32_t max_context_len, int32_t num_seqs, int32_t num_heads,
                            int32_t num_kv_heads, int32_t head_dim, int32_t num_blocks,
                            float scale, void* workspace, size_t workspace_bytes,
                            pa_stream_t stream);

/* Chunked causal prefill over the paged cache.
 *   out, q        [total_q, Hq, D]; sequence s owns rows
 *                 cu_q_lens[s] .. cu_q_lens[s+1]-1
 *   cu_q_lens     [num_seqs + 1] int32, past_lens [num_seqs] int32
 *   max_q_len     host upper bound of the per-sequence query count
 * Query row i of sequence s sits at absolute position past_lens[s] + i and
 * attends keys j <= past_lens[s] + i, all read from the cache (write the
 * chunk's K/V with pa_reshape_and_cache first).  Table entries outside
 * [0, num_blocks) contribute no keys, as in pa_decode.  cu_q_lens entries
 * outside [0, total_q], sequences of more than max_q_len rows and negative
 * past_lens are caller errors: the rows concerned are unspecified, and no
 * read or write leaves q and out (offsets are clamped on the device).
 * Replaces forward_prefill / forward_prefill_continue's attention
 * (rope_gqa.rs:261-372): tiled_attention (util.rs:188-234) for past = 0 and
 * compute_gqa_attention + prefill_continue_causal_mask
 * (paged_gqa.rs:135-164) for past > 0. */
int32_t pa_prefill(void* out, const void* q, const void* k_cache, const void* v_cache,
                   const int32_t* block_tables, int32_t max_blocks_per_seq,
                   const int32_t* cu_q_lens, const int32_t* past_lens, int32_t num_seqs,
                   int32_t total_q, int32_t max_q_len, int32_t num_heads, int32_t num_kv_heads,
                   int32_t head_dim, int32_t num_blocks, float scale, int32_t dtype,
                   pa_stream_t stream);

/* pa_prefill over a quantised PagedKvCache, reading values as in
 * pa_decode_quantized (f32 q / out). */
int32_t pa_prefill_quantized(void* out, const void* q, const float* k_cache, const float* v_cache,
                             const float* block_scales, const int32_t* block_tables,
                             int32_t max_blocks_per_seq, const int32_t* cu_q_lens,
                             const int32_t* past_lens, int32_t num_seqs, int32_t total_q,
                             int32_t max_q_len, int32_t num_heads, int32_t num_kv_heads,
                             int32_t head_dim, int32_t num_blocks, float scale,
                             pa_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* VLLM_LITE_AMD_PA_H */
