/*
 * pa_dense.h -- the dense side around the paged-attention path, for an
 * end-to-end decoder step: RMSNorm or LayerNorm (with the residual add fused
 * in), the SwiGLU activation, and the linear projections (skinny-M for
 * decode steps, a tiled GEMM for prompt chunks).  Conventions as pa.h (device
 * pointers, stream-ordered, PA_OK or a negative pa_status); dtype
 * PA_DTYPE_F32 or PA_DTYPE_BF16, math in f32.
 */
#ifndef VLLM_LITE_AMD_PA_DENSE_H
#define VLLM_LITE_AMD_PA_DENSE_H

#include "pa.h"

#ifdef __cplusplus
extern "C" {
#endif

/* RmsNorm::forward (crates/model/src/components/norm/rms_norm.rs:26-50) with
 * the decoder block's residual add fused in front
 * (crates/model/src/components/decoder_block/mod.rs:157-198):
 *   if add != NULL:  residual[r] += add[r]        (rounded to dtype, in place)
 *   out[r] = residual[r] / sqrt(mean(residual[r]^2) + eps) * weight
 * residual / add / out [rows, hidden] (contiguous), weight [hidden]. */
int32_t pa_rms_norm(void* out, void* residual, const void* add, const void* weight,
                    int32_t rows, int32_t hidden, float eps, int32_t dtype, pa_stream_t stream);

/* LnLayerNorm::forward (crates/model/src/components/norm/layer_norm.rs:26-39,
 * candle_nn::LayerNorm with the mean removed and an affine bias), the norm the
 * reference's decoder blocks are built with
 * (crates/model/src/components/decoder_block/factory.rs:42-46), with the
 * residual add fused in front as in pa_rms_norm:
 *   if add != NULL:  residual[r] += add[r]        (rounded to dtype, in place)
 *   mu = mean(residual[r]);  var = mean((residual[r] - mu)^2)
 *   out[r] = (residual[r] - mu) / sqrt(var + eps) * weight + bias
 * bias may be NULL (the zero bias).  Shapes as pa_rms_norm. */
int32_t pa_layer_norm(void* out, void* residual, const void* add, const void* weight,
                      const void* bias, int32_t rows, int32_t hidden, float eps, int32_t dtype,
                      pa_stream_t stream);

/* The SwiGLU activation of swiglu_forward
 * (crates/model/src/components/mlp/swiglu.rs:18-31) on a fused gate|up
 * projection output:  out[r][i] = silu(gate_up[r][i]) * gate_up[r][inter + i],
 * silu(x) = x / (1 + e^-x).  gate_up [rows, 2 * inter], out [rows, inter]. */
int32_t pa_silu_mul(void* out, const void* gate_up, int32_t rows, int32_t inter, int32_t dtype,
                    pa_stream_t stream);

/* Activation epilogues and flags of pa_linear. */
enum { PA_ACT_NONE = 0, PA_ACT_SILU_MUL = 1 };
enum { PA_LINEAR_RMS_IN = 1, PA_LINEAR_ADD_OUT = 2 };

/* The decoder's linear projections for the few-row batches of a decode step
 * (candle_nn::Linear as the reference's attention and MLP use it: the QKV
 * projection with bias, crates/model/src/components/attention/rope_gqa.rs:261-302,
 * the output projection, and the MLP's gate/up/down projections,
 * crates/model/src/components/mlp/swiglu.rs:18-31), plus the tied LM head:
 *   act PA_ACT_NONE:      out[r][n] = sum_k x[r][k] * weight[n][k] (+ bias[n])
 *   act PA_ACT_SILU_MUL:  weight is the fused gate|up matrix [2 N, K] and
 *                         out[r][n] = silu(g) * u with g, u the gate / up
 *                         outputs of column n rounded to bf16 (pa_silu_mul on
 *                         the unfused projection's output); bias must be NULL.
 * x [rows, K], weight [N or 2 N, K], out [rows, N], all contiguous bf16 and
 * 16-byte aligned, bias [N] or NULL; K (in_features) and N (out_features)
 * as the kernel below needs.  f32 accumulation.
 * packed = 1: weight is in the layout of pa_linear_pack (rows N or 2 N).
 * flags (0 or a combination):
 *   PA_LINEAR_RMS_IN   the rows of x are RMS-normalised on the fly: the result
 *                      is multiplied by 1 / sqrt(mean_k(x[r][k]^2) + eps) (the
 *                      decoder's RMSNorm, crates/model/src/components/norm/
 *                      rms_norm.rs:26-50, in front of the projection); the
 *                      norm weight is folded into the weight's columns by
 *                      pa_linear_pack's col_scale;
 *   PA_LINEAR_ADD_OUT  out is the residual stream and is updated in place,
 *                      out[r][n] = bf16(out[r][n] + bf16(y[r][n])) (the
 *                      decoder block's residual add); not with SwiGLU.
 * workspace: NULL, or pa_linear_workspace_size() bytes (256-byte aligned)
 * whose first bytes hold counters that must be ZERO before the first call
 * that uses it (e.g. hipMemset once after allocating it); every call leaves
 * them zero again.  With it, long-K projections over few output tiles (the
 * MLP down projection of a decode step) split K over several workgroups per
 * tile, the last to finish summing the partial tiles in a fixed order (the
 * result does not depend on their timing).  Calls that may run at the same
 * time need distinct workspaces.  Without it one workgroup takes each tile.
 * Three kernels behind the one entry point:
 *  - rows <= 64 (decode steps), packed or row-major weights: the skinny
 *    kernel, where the weights dominate the traffic (they are re-read once
 *    per 32 rows); K a multiple of 32, N of 16;
 *  - rows <= 32, packed weights of at least 65,536 rows (the LM head), no
 *    bias, activation or residual add, K <= 992: a persistent kernel that
 *    holds X in LDS and streams the weight tiles over all CUs (the
 *    workspace is not used);
 *  - rows > 64 (prompt chunks), or an N the skinny tiles do not divide, with
 *    row-major weights, no PA_LINEAR_RMS_IN and K a multiple of 64: a tiled
 *    GEMM on the matrix cores (128 x 128 output tiles, K staged through LDS
 *    in steps of 64; any N, with SwiGLU a multiple of 64; the workspace is
 *    not used).
 * Other shapes return PA_ERR_UNSUPPORTED, as does any dtype but bf16. */
int32_t pa_linear(void* out, const void* x, const void* weight, const void* bias, int32_t rows,
                  int32_t out_features, int32_t in_features, int32_t act, int32_t packed,
                  int32_t flags, float eps, void* workspace, size_t workspace_bytes,
                  int32_t dtype, pa_stream_t stream);

/* Workspace bytes pa_linear's K split uses for this shape (0: none; the call
 * then needs no workspace).  No reference counterpart. */
size_t pa_linear_workspace_size(int32_t rows, int32_t out_features, int32_t in_features,
                                int32_t act);

/* Repacks a row-major bf16 weight [rows, cols] (rows a multiple of 16, cols
 * of 32) into the fragment order pa_linear reads with packed = 1: every
 * 16-row x 32-column MFMA operand fragment becomes one contiguous kilobyte,
 * the fragments of a 16-row tile consecutive along the columns.  col_scale
 * [cols] (bf16) or NULL: each column is multiplied by it (rounded to bf16),
 * which folds a norm weight in front of the projection.  Same size as the
 * input; packed and weight must not overlap.  No reference counterpart: a
 * load-time layout step for the weights pa_linear streams. */
int32_t pa_linear_pack(void* packed, const void* weight, const void* col_scale, int32_t rows,
                       int32_t cols, int32_t dtype, pa_stream_t stream);

/* The decode step's QKV projection with RoPE and the KV-cache write fused
 * into its epilogue: pa_linear (bf16, act none, optional PA_LINEAR_RMS_IN and
 * bias) over a weight packed by pa_linear_pack_qkv, followed in the same pass
 * by what pa_rope_reshape_and_cache does to its output
 * (crates/model/src/components/attention/rope_gqa.rs:280-302,
 * crates/model/src/components/positional/rope.rs:335-568):
 *   out [rows, (num_heads + 2 num_kv_heads) head_dim]: the projection, q and k
 *       columns rotated by position (inv_freq [head_dim / 2], positions [rows]),
 *       v columns as projected; identical to pa_linear followed by
 *       pa_rope_reshape_and_cache on the q / k / v views of its output;
 *   k_cache / v_cache: token r's rotated k and its v written to slot
 *       slot_mapping[r] (skipped when outside [0, num_blocks * 16)).
 * head_dim and in_features multiples of 32; flags 0 or PA_LINEAR_RMS_IN.
 * weight, bias: the fused QKV weight [(Hq + 2 Hkv) head_dim, in_features]
 * (bias in the original row order).  No reference counterpart as one call. */
int32_t pa_linear_rope_cache(void* out, const void* x, const void* weight, const void* bias,
                             int32_t rows, int32_t num_heads, int32_t num_kv_heads,
                             int32_t head_dim, int32_t in_features, int32_t flags, float eps,
                             const int64_t* positions, const int64_t* slot_mapping,
                             const float* inv_freq, void* k_cache, void* v_cache,
                             int32_t num_blocks, int32_t dtype, pa_stream_t stream);

/* pa_linear_pack for pa_linear_rope_cache's weight: the fused QKV weight
 * [(num_heads + 2 num_kv_heads) head_dim, cols], with the rows of each query
 * and key head reordered so that the two members (i, i + head_dim / 2) of
 * each rotation pair land in the same wavefront; col_scale as pa_linear_pack.
 * No reference counterpart: a load-time layout step. */
int32_t pa_linear_pack_qkv(void* packed, const void* weight, const void* col_scale,
                           int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                           int32_t cols, int32_t dtype, pa_stream_t stream);

/* Greedy sampling's argmax_logits (crates/traits/src/sampling.rs:439-453) on
 * every row of a logit matrix: out[r] = the first column holding the row's
 * largest value, comparing with `>` from -inf, so NaN never wins and a row
 * with no value above -inf (or cols == 0) gives 0.  logits [rows, cols] with
 * row_stride elements between rows (0 = cols); out [rows] int64 (device). */
int32_t pa_argmax(int64_t* out, const void* logits, int32_t rows, int32_t cols,
                  int64_t row_stride, int32_t dtype, pa_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* VLLM_LITE_AMD_PA_DENSE_H */
