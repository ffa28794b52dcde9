// act.hpp - the GLU element formulas between the two expert products
// (ggml_vec_swiglu_f32 / ggml_vec_geglu_erf_f32 / ggml_vec_geglu_f32):
//   SILU          silu(a) * b                    qwen3omni_model.cpp:771
//   GELU_ERF_GP1  gelu_erf(h) * (g + 1)          moondream.cpp:534-535
//   GELU_TANH     gelu_tanh(a) * b
//   GELU_ERF      gelu_erf(a) * b                moe_compute.cpp:127-129
//   RELU_SQR      relu(a)^2 (b unused)           nemotronomni_model.cpp:366-367
#pragma once

#include <hip/hip_runtime.h>

namespace mimoe {

constexpr int ACT_RELU_SQR = 4;   // mi_act: non-gated experts, one product
// ggml_sqr(ggml_relu(u)): relu keeps u > 0, else 0
__device__ inline float relu_sqr(float a) {
    const float r = a > 0.f ? a : 0.f;
    return r * r;
}

// libm-accurate forms (GEMV path: a few values per token)
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
    case 4: return relu_sqr(a);
    default: return 0.f;
    }
}

// Branch-free forms for the GEMM epilogue (32 values per lane).  exp via
// v_exp_f32 (2^x), reciprocals via v_rcp_f32 (1 ulp).  erf through the
// complementary function of Abramowitz & Stegun 7.1.26 (Hastings):
//   erfc(z) = t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) exp(-z^2),
//   t = 1 / (1 + p z), z >= 0, |error of erf| <= 1.5e-7,
// so 1 + erf(x) = 2 - erfc(z) for x >= 0 and erfc(z) for x < 0 keeps
// relative accuracy on the negative tail.  Against the libm forms the
// results differ by ~1e-7 absolute, far below one Q8_K step of the
// activations that follow.
__device__ inline float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ inline float rcp_fast(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ inline float one_plus_erf_fast(float x) {
    const float z = fabsf(x);
    const float t = rcp_fast(fmaf(0.3275911f, z, 1.0f));
    float p = fmaf(t, 1.061405429f, -1.453152027f);
    p = fmaf(t, p, 1.421413741f);
    p = fmaf(t, p, -0.284496736f);
    p = fmaf(t, p, 0.254829592f);
    const float c = t * p * exp_fast(-z * z);   // erfc(z)
    return x >= 0.f ? 2.0f - c : c;
}
// ACT is a template argument: callers branch once per tile, not per value
// (a runtime switch over branch-free bodies gets if-converted, evaluating
// every form)
template <int ACT>
__device__ inline float act_pair_fast(float a, float b) {
    const float SQRT_2_INV = 0.70710678118654752440084436210484f;
    const float SQRT_2_OVER_PI = 0.79788456080286535587989211986876f;
    const float GELU_COEF_A = 0.044715f;
    if constexpr (ACT == 0) {
        return a * rcp_fast(1.0f + exp_fast(-a)) * b;
    } else if constexpr (ACT == 1) {
        return 0.5f * a * one_plus_erf_fast(a * SQRT_2_INV) * (b + 1.0f);
    } else if constexpr (ACT == 2) {
        // (1 + tanh(u)) / 2 = 1 / (1 + exp(-2u)): one exp2 with the constants
        // folded, -2 sqrt(2/pi) log2(e) * a * (1 + c a^2)
        const float k = -2.0f * SQRT_2_OVER_PI * 1.4426950408889634f;
        const float e = __builtin_amdgcn_exp2f(k * a * (1.0f + GELU_COEF_A * a * a));
        return a * b * rcp_fast(1.0f + e);
    } else if constexpr (ACT == 3) {
        return 0.5f * a * one_plus_erf_fast(a * SQRT_2_INV) * b;
    } else {
        return relu_sqr(a);
    }
}

}  // namespace mimoe
