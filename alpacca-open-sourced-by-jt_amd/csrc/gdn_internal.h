// GDN step launcher shared by the step entry point and the fused
// recurrent-layer step (no timing bracket of its own).
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>

namespace alpx {

// Output scale 1 / sqrt(Dk) of the GDN read-out o = S q / sqrt(Dk).
inline float gdn_output_scale(int key_dim) { return 1.0f / sqrtf((float)key_dim); }

int gdn_step_launch(float* state, const void* q, const void* k, const void* v, const float* beta,
                    const float* log_decay, void* out, int batch, int key_heads,
                    int value_heads, int key_dim, int value_dim, int dtype, int out_dtype,
                    hipStream_t s);

}  // namespace alpx
