// norm.hpp - the row norms in front of the MoE block (k_norm_rows in
// k_data.hip; mi_norm and mi_moe_forward_norm).
//
// Reference norms (applied to the layer stream before the MoE block):
//   RMS    y = (x * s) [* w]               s = 1 / sqrtf(fl32(sum x^2 / D) + eps)
//          ggml_rms_norm then ggml_mul by ffn_norm (qwen3omni_model.cpp:756-757)
//   LAYER  y = ((x - m) * s) [* w] [+ b]   m = fl32(sum x / D),
//                                          s = 1 / sqrtf(fl32(sum (x - m)^2 / D) + eps)
//          ggml_norm then ggml_mul / ggml_add (moondream.cpp:405-407)
// ggml sums the fp32 products x*x and (x-m)*(x-m) in double; so does this
// (k_norm_rows: one work-group per row, a fixed order).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mimoe {

enum { NORM_NONE = 0, NORM_RMS = 1, NORM_LAYER = 2 };

// k_norm_rows' fixed summation order (also run inside the fused single-token
// kernel): thread t < NORM_T holds elements 1024 k + 4 t + j (k < NORM_PIECES,
// j < 4), sums them in that order in fp64, and the NORM_T partials are added
// pairwise, red[t] += red[t + o] for o = NORM_T / 2 .. 1.
constexpr int NORM_T = 256, NORM_PIECES = 4;   // rows up to 4096

struct NormParams {
    int kind = NORM_NONE;
    float eps = 0.f;
    const float *w = nullptr;   // [D] or null
    const float *b = nullptr;   // [D] or null (LAYER only)
};

// the normalized value of element i (value v) of a row with stats (m, s)
__device__ inline float norm_apply(const NormParams &p, float v, int64_t i, float m, float s) {
    float y = p.kind == NORM_RMS ? v * s : (v - m) * s;
    if (p.w) y = y * p.w[i];
    if (p.kind == NORM_LAYER && p.b) y = y + p.b[i];
    return y;
}

}  // namespace mimoe
