// wave_ops.hpp - wave-level pieces shared by the routing kernels and the
// fused decode kernels: one implementation, so every path that quantizes an
// activation row or selects experts produces the same bits.
#pragma once

#include "common.hpp"

namespace mimoe {

// ---------------------------------------------------------------- lane exchange
// DPP moves (no LDS round trip) for reductions inside 16-lane rows.  Each
// control pairs every lane with one partner; applied in this order the four
// reduce groups of 2, 4, 8 and 16 lanes, and every lane of the group ends up
// with the result:
//   0xB1  quad_perm [1,0,3,2]   (lane ^ 1)
//   0x4E  quad_perm [2,3,0,1]   (lane ^ 2)
//   0x141 row_half_mirror       (lane i <-> 7 - i within 8)
//   0x140 row_mirror            (lane i <-> 15 - i within 16)
template <int CTRL>
__device__ inline int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ inline float dpp_f(float v) {
    return __builtin_bit_cast(float, dpp_i<CTRL>(__builtin_bit_cast(int, v)));
}

// sum over aligned groups of `width` lanes (8, 16, 32 or 64), in every lane
__device__ inline float group_sum(float v, int width) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    if (width >= 16) v += dpp_f<0x140>(v);
    if (width >= 32) v += __shfl_xor(v, 16, 64);
    if (width >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

template <int CTRL>
__device__ inline AmaxIdx amax_dpp(AmaxIdx a) {
    AmaxIdx b;
    b.ax = dpp_f<CTRL>(a.ax);
    b.idx = dpp_i<CTRL>(a.idx);
    b.val = dpp_f<CTRL>(a.val);
    return amax_better(a, b);
}
__device__ inline AmaxIdx amax_xor(AmaxIdx a, int o) {
    AmaxIdx b;
    b.ax = __shfl_xor(a.ax, o, 64);
    b.idx = __shfl_xor(a.idx, o, 64);
    b.val = __shfl_xor(a.val, o, 64);
    return amax_better(a, b);
}
// (|x| max, first index) over the wave.  amax_better is a total order (ties
// in |x| go to the lower index), so the result does not depend on the
// reduction tree.
__device__ inline AmaxIdx wave_amax_idx_fast(AmaxIdx a) {
    a = amax_dpp<0xB1>(a);
    a = amax_dpp<0x4E>(a);
    a = amax_dpp<0x141>(a);
    a = amax_dpp<0x140>(a);
    a = amax_xor(a, 16);
    return amax_xor(a, 32);
}

// Q8_K of one 256-value block held by one wave, lane l holding the values at
// 4l .. 4l+3 (ggml quantize_row_q8_K_ref): the first value with the largest
// |x| sets iscale = -127 / x, q = min(127, nearest_int(iscale * v)),
// d = 1 / iscale; an all-zero block gives q = 0 and d = 0.  Returns d.
__device__ inline float q8k_wave(const float (&v)[4], int lane, int (&q)[4]) {
    AmaxIdx a{-1.f, 1 << 30, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) a = amax_better(a, AmaxIdx{fabsf(v[j]), 4 * lane + j, v[j]});
    a = wave_amax_idx_fast(a);
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
    s += dpp_i<0xB1>(s);
    s += dpp_i<0x4E>(s);
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
