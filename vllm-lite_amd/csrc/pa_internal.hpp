// Launchers shared between translation units of libpa.so (not exported).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pa {

#define PA_HIDDEN __attribute__((visibility("hidden")))

// Quantised (int8-in-f32) block writes: one workgroup per task, see quant.hip.
PA_HIDDEN int32_t launch_quant_write(float* k_cache, float* v_cache, float* scales,
                                     const float* k, const float* v, int H, int D, int num_tasks,
                                     const int32_t* task_block, const int32_t* task_beg,
                                     const int32_t* tok, const int32_t* off, uint64_t* hashes,
                                     hipStream_t stream);
// Block hashes after every token of a (non-quantised) write, before its
// scatter: see cache_ops.hip.
PA_HIDDEN int32_t launch_block_hash_replay(const void* k_cache, const void* key, int32_t dtype,
                                           int H, int D, int num_tasks,
                                           const int32_t* task_block, const int32_t* task_beg,
                                           const int32_t* tok, const int32_t* off,
                                           uint64_t* hashes, hipStream_t stream);
// write_kv of one token (non-quantised caches): block hash + store in one
// launch, the hash into host-mapped *hash_out.
PA_HIDDEN int32_t launch_write_token(void* k_cache, void* v_cache, const void* key,
                                     const void* value, int32_t dtype, int H, int D, int64_t blk,
                                     int off, uint64_t* hash_out, hipStream_t stream);
// read_kv of at most kSmallIds blocks with the ids in the kernel arguments.
constexpr int kSmallIds = 16;
PA_HIDDEN int32_t launch_read_kv_small(const void* k_cache, const void* v_cache, int32_t dtype,
                                       const int32_t* ids, int n_ids, int seq_len, int H, int D,
                                       int num_blocks, void* out_k, void* out_v,
                                       hipStream_t stream);
PA_HIDDEN int32_t launch_quant_read(const float* k_cache, const float* v_cache,
                                    const float* scales, const int32_t* block_ids, int seq_len,
                                    int H, int D, float* out_k, float* out_v, hipStream_t stream);

// pa_decode / pa_prefill with q rows q_row elements apart (a view of a fused
// QKV projection output); pa_batch_attention's path.
PA_HIDDEN int32_t decode_strided(void* out, const void* q, int64_t q_row, const void* k_cache,
                                 const void* v_cache, const int32_t* block_tables,
                                 int32_t max_blocks_per_seq, const int32_t* context_lens,
                                 int32_t max_context_len, int32_t num_seqs, int32_t num_heads,
                                 int32_t num_kv_heads, int32_t head_dim, int32_t num_blocks,
                                 float scale, void* workspace, size_t workspace_bytes,
                                 int32_t dtype, hipStream_t stream);
PA_HIDDEN int32_t prefill_strided(void* out, const void* q, int64_t q_row, const void* k_cache,
                                  const void* v_cache, const int32_t* block_tables,
                                  int32_t max_blocks_per_seq, const int32_t* cu_q_lens,
                                  const int32_t* past_lens, int32_t num_seqs, int32_t total_q,
                                  int32_t max_q_len, int32_t num_heads, int32_t num_kv_heads,
                                  int32_t head_dim, int32_t num_blocks, float scale,
                                  int32_t dtype, hipStream_t stream);

}  // namespace pa
