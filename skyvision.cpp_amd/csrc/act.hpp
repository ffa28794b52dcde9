// act.hpp - the GLU element formulas between the two expert products
// (ggml_vec_swiglu_f32 / ggml_vec_geglu_erf_f32 / ggml_vec_geglu_f32):
//   SILU          silu(a) * b                    qwen3omni_model.cpp:771
//   GELU_ERF_GP1  gelu_erf(h) * (g + 1)          moondream.cpp:534-535
//   GELU_TANH     gelu_tanh(a) * b
//   GELU_ERF      gelu_erf(a) * b                moe_compute.cpp:127-129
#pragma once

#include <hip/hip_runtime.h>

namespace mimoe {

__device__ inline float act_pair(int act, float a, float b) {
    const float SQRT_2_INV = 0.70710678118654752440084436210484f;
    const float SQRT_2_OVER_PI = 0.79788456080286535587989211986876f;
    const float GELU_COEF_A = 0.044715f;
    switch (act) {
    case 0: return (a / (1.0f + expf(-a))) * b;
    case 1: {
        const float g1 = b + 1.0f;
        return 0.5f * a * (1.0f + erff(a * SQRT_2_INV)) * g1;
    }
    case 2: return 0.5f * a * (1.0f + tanhf(SQRT_2_OVER_PI * a * (1.0f + GELU_COEF_A * a * a))) * b;
    case 3: return 0.5f * a * (1.0f + erff(a * SQRT_2_INV)) * b;
    default: return 0.f;
    }
}

}  // namespace mimoe
