/*
 * pa_dense.h -- the dense side around the paged-attention path, for an
 * end-to-end decoder step: RMSNorm or LayerNorm (with the residual add fused
 * in) and the SwiGLU activation.  The projections themselves are plain GEMMs and run in
 * hipBLASLt.  Conventions as pa.h (device pointers, stream-ordered, PA_OK or
 * a negative pa_status); dtype PA_DTYPE_F32 or PA_DTYPE_BF16, math in f32.
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

#ifdef __cplusplus
}
#endif

#endif /* VLLM_LITE_AMD_PA_DENSE_H */
