// wave_ops.hpp - wave-level pieces shared by the routing kernels and the
// fused decode kernels: one implementation, so every path that quantizes an
// activation row or selects experts produces the same bits.
#pragma once

#include "common.hpp"

namespace mimoe {

// Q8_K of one 256-value block held by one wave, lane l holding the values at
// 4l .. 4l+3 (ggml quantize_row_q8_K_ref): the first value with the largest
// |x| sets iscale = -127 / x, q = min(127, nearest_int(iscale * v)),
// d = 1 / iscale; an all-zero block gives q = 0 and d = 0.  Returns d.
__device__ inline float q8k_wave(const float (&v)[4], int lane, int (&q)[4]) {
    AmaxIdx a{-1.f, 1 << 30, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) a = amax_better(a, AmaxIdx{fabsf(v[j]), 4 * lane + j, v[j]});
    a = wave_amax_idx(a);
#pragma unroll
    for (int j = 0; j < 4; ++j) q[j] = 0;
    if (a.ax == 0.f) return 0.f;
    const float iscale = -127.f / a.val;
#pragma unroll
    for (int j = 0; j < 4; ++j) q[j] = imin(127, nearest_int(iscale * v[j]));
    return 1 / iscale;
}

// sum of the 16 codes of lane group lane / 4 (the ggml bsums entry), valid in
// every lane of the group
__device__ inline int q8k_bsum16(const int (&q)[4]) {
    int s = q[0] + q[1] + q[2] + q[3];
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    return s;
}

__device__ inline uint32_t pack_i8x4(const int (&q)[4]) {
    return (uint32_t)(uint8_t)q[0] | ((uint32_t)(uint8_t)q[1] << 8) | ((uint32_t)(uint8_t)q[2] << 16) |
           ((uint32_t)(uint8_t)q[3] << 24);
}

// softmax over the K selected logits held by lanes k < K (ggml_soft_max on
// the get_rows view): max, expf(v - max), sum in fp64 in slot order, scale
// by (float)(1.0 / sum).  Every lane of the wave must call it; lane k < K
// gets its weight.
__device__ inline float softmax_selected_wave(float myval, int K, int lane) {
    float mx = lane < K ? myval : -INFINITY;
    mx = wave_max(mx);
    const float val = lane < K ? expf(myval - mx) : 0.f;
    double sum = 0.0;
    for (int k = 0; k < K; ++k) sum = sum + (double)__shfl(val, k, 64);
    sum = 1.0 / sum;
    const float s = (float)sum;
    return val * s;
}

// Top-k of one token's E logits by one wave (E <= 64 * TOPK_MAX_PER_LANE,
// K <= 64): K rounds of a wave arg-max (largest value, lowest id on ties)
// over the experts not yet taken.  Lane k < K gets the k-th id and, when
// want_w, its softmax weight over the K selected logits: max, expf(v - max),
// sum in fp64 in slot order, scale by (float)(1.0 / sum) (ggml_soft_max).
constexpr int TOPK_MAX_PER_LANE = 4;
__device__ inline void topk_softmax_wave(const float *l, int E, int K, int lane, int &mysel, float &myw,
                                         bool want_w) {
    float v[TOPK_MAX_PER_LANE];
    bool avail[TOPK_MAX_PER_LANE];
#pragma unroll
    for (int i = 0; i < TOPK_MAX_PER_LANE; ++i) {
        const int e = lane + 64 * i;
        avail[i] = e < E;
        v[i] = avail[i] ? l[e] : 0.f;
    }
    mysel = 0;
    float myval = 0.f;
    for (int k = 0; k < K; ++k) {
        float bv = 0.f;
        int bi = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < TOPK_MAX_PER_LANE; ++i) {
            const int e = lane + 64 * i;
            if (avail[i] && (bi == 0x7fffffff || v[i] > bv)) {
                bv = v[i];
                bi = e;
            }
        }
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
            const bool take = oi != 0x7fffffff && (bi == 0x7fffffff || ov > bv || (ov == bv && oi < bi));
            if (take) {
                bv = ov;
                bi = oi;
            }
        }
        if (bi != 0x7fffffff && (bi & 63) == lane) {
#pragma unroll
            for (int i = 0; i < TOPK_MAX_PER_LANE; ++i)
                if (lane + 64 * i == bi) avail[i] = false;
        }
        if (lane == k) {
            mysel = bi;
            myval = bv;
        }
    }
    myw = want_w ? softmax_selected_wave(myval, K, lane) : 0.f;
}

}  // namespace mimoe
