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
                                     const int32_t* tok, const int32_t* off, hipStream_t stream);
PA_HIDDEN int32_t launch_quant_read(const float* k_cache, const float* v_cache,
                                    const float* scales, const int32_t* block_ids, int seq_len,
                                    int H, int D, float* out_k, float* out_v, hipStream_t stream);

}  // namespace pa
