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

// inclusive prefix sum over the 64 lanes: Hillis-Steele inside each 16-lane
// row (row_shr 1, 2, 4, 8; lanes shifted in from outside the row add 0), then
// row_bcast:15 adds the last lane of rows 0 / 2 to rows 1 / 3 and row_bcast:31
// the last lane of row 1 (rows 0-1 by then) to rows 2 and 3
__device__ inline int wave_incl_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);
    return v;
}

// lane k's value, uniform (a scalar read: no LDS round trip)
__device__ inline float lane_f(float v, int k) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), k));
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

// Largest |x| over the wave (lane l holding elements 4l .. 4l+3) and the
// signed value of the first element that attains it, in element order: the
// element ggml's "if (ax > amax)" scan keeps.  The max is reduced alone (one
// exchange and one max per step); the first holder comes from a ballot.
struct AbsMax {
    float ax, val;
};
__device__ inline float absmax4(const float (&v)[4]) {
    return fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
}
__device__ inline AbsMax absmax_first(const float (&v)[4], float m) {
    // m: the wave's largest |x|
    const bool h0 = fabsf(v[0]) == m, h1 = fabsf(v[1]) == m, h2 = fabsf(v[2]) == m, h3 = fabsf(v[3]) == m;
    const unsigned long long holders = __ballot(h0 | h1 | h2 | h3);
    const int first = (int)__builtin_ctzll(holders | (1ull << 63));
    const float mine = h0 ? v[0] : h1 ? v[1] : h2 ? v[2] : v[3];
    AbsMax r;
    r.ax = m;
    r.val = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mine), first));
    return r;
}

// Q8_K of one 256-value block held by one wave, lane l holding the values at
// 4l .. 4l+3 (ggml quantize_row_q8_K_ref): the first value with the largest
// |x| sets iscale = -127 / x, q = min(127, nearest_int(iscale * v)),
// d = 1 / iscale; an all-zero block gives q = 0 and d = 0.  Returns d.
__device__ inline float q8k_wave(const float (&v)[4], int lane, int (&q)[4]) {
    float m = absmax4(v);
    m = fmaxf(m, dpp_f<0xB1>(m));
    m = fmaxf(m, dpp_f<0x4E>(m));
    m = fmaxf(m, dpp_f<0x141>(m));
    m = fmaxf(m, dpp_f<0x140>(m));
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    const AbsMax a = absmax_first(v, m);
#pragma unroll
    for (int j = 0; j < 4; ++j) q[j] = 0;
    if (a.ax == 0.f) return 0.f;
    const float iscale = -127.f / a.val;
#pragma unroll
    for (int j = 0; j < 4; ++j) q[j] = imin(127, nearest_int(iscale * v[j]));
    return 1 / iscale;
}

// Q8_K of N blocks at once (the same arithmetic as q8k_wave; the N reductions
// run in lockstep so their lane exchanges overlap)
template <int N>
__device__ inline void q8k_wave_n(const float (&v)[N][4], int lane, int (&q)[N][4], float (&d)[N]) {
    float m[N];
#pragma unroll
    for (int n = 0; n < N; ++n) m[n] = absmax4(v[n]);
#pragma unroll
    for (int n = 0; n < N; ++n) m[n] = fmaxf(m[n], dpp_f<0xB1>(m[n]));
#pragma unroll
    for (int n = 0; n < N; ++n) m[n] = fmaxf(m[n], dpp_f<0x4E>(m[n]));
#pragma unroll
    for (int n = 0; n < N; ++n) m[n] = fmaxf(m[n], dpp_f<0x141>(m[n]));
#pragma unroll
    for (int n = 0; n < N; ++n) m[n] = fmaxf(m[n], dpp_f<0x140>(m[n]));
#pragma unroll
    for (int n = 0; n < N; ++n) m[n] = fmaxf(m[n], __shfl_xor(m[n], 16, 64));
#pragma unroll
    for (int n = 0; n < N; ++n) m[n] = fmaxf(m[n], __shfl_xor(m[n], 32, 64));
#pragma unroll
    for (int n = 0; n < N; ++n) {
        const AbsMax a = absmax_first(v[n], m[n]);
        const bool zero = a.ax == 0.f;
        const float iscale = zero ? 0.f : -127.f / a.val;
#pragma unroll
        for (int j = 0; j < 4; ++j) q[n][j] = zero ? 0 : imin(127, nearest_int(iscale * v[n][j]));
        d[n] = zero ? 0.f : 1 / iscale;
    }
}

// Q8_K of four blocks by one wave, 16 lanes per block: lane l quantizes
// values 16 (l % 16) .. +15 of block l / 16 (same arithmetic as q8k_wave;
// the four blocks share one instruction stream, and each lane's 16 codes
// form one ggml bsums entry).  Returns this lane's block scale d; bsum is
// the sum of the lane's 16 codes.
__device__ inline float q8k_wave4x16(const float (&v)[16], int lane, int (&q)[16], int &bsum) {
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) m = fmaxf(m, fabsf(v[i]));
    m = fmaxf(m, dpp_f<0xB1>(m));
    m = fmaxf(m, dpp_f<0x4E>(m));
    m = fmaxf(m, dpp_f<0x141>(m));
    m = fmaxf(m, dpp_f<0x140>(m));   // m: largest |x| of the lane's block
    // first element attaining it: first holder lane of the 16-lane group,
    // first position in that lane
    bool has = false;
    float mine = 0.f;
#pragma unroll
    for (int i = 15; i >= 0; --i) {
        const bool hi = fabsf(v[i]) == m;
        has = has | hi;
        mine = hi ? v[i] : mine;
    }
    const unsigned long long holders = __ballot(has);
    float first_val[4];
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
        const unsigned long long gm = (holders >> (16 * gi)) & 0xffffull;
        const int fl = 16 * gi + (int)__builtin_ctzll(gm | 0x8000ull);
        first_val[gi] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mine), fl));
    }
    const int grp = lane >> 4;
    const float val = grp == 0 ? first_val[0] : grp == 1 ? first_val[1] : grp == 2 ? first_val[2] : first_val[3];
    const bool zero = m == 0.f;
    const float iscale = zero ? 0.f : -127.f / val;
    int s = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        q[i] = zero ? 0 : imin(127, nearest_int(iscale * v[i]));
        s += q[i];
    }
    bsum = s;
    return zero ? 0.f : 1 / iscale;
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
    float mx = -INFINITY;
    for (int k = 0; k < K; ++k) mx = fmaxf(mx, lane_f(myval, k));
    const float val = lane < K ? expf(myval - mx) : 0.f;
    double sum = 0.0;
    for (int k = 0; k < K; ++k) sum = sum + (double)lane_f(val, k);
    sum = 1.0 / sum;
    const float s = (float)sum;
    return val * s;
}

// Top-k of one token's E logits by one wave (E <= 64 * TOPK_MAX_PER_LANE,
// K <= 64), largest value first, lower id first on ties: K rounds of the
// wave's largest remaining value (a max reduction), whose id is the lowest
// set bit of a ballot of its holders (ids 64 i + lane, block i = 0 first);
// the winner then leaves the race (NaN: the max skips it, == never holds).
// The order equals ranking every value by the values that come before it
// (larger, or equal with a lower id).  Lane k < K gets the k-th id and, when
// want_w, its softmax weight over the K selected logits: max, expf(v - max),
// sum in fp64 in slot order, scale by (float)(1.0 / sum) (ggml_soft_max).
constexpr int TOPK_MAX_PER_LANE = 4;
__device__ inline void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
// Router gating variants (the layer's mi_gating): kind 0 ranks the logits
// and takes the softmax over the K selected; kind 1 ranks s + sel_bias[e]
// with s = fl32(1 / (1 + exp(-logit))) evaluated in fp64 (one rounding, so
// every implementation ranks the same values) and weights s / (fl32(sum_K
// s in fp64, slot order) + eps) * scaling; kind 2 ranks the probabilities of
// the softmax over all E (ggml_soft_max: max, e = fl32(exp(fl32(l - max)))
// with the exp in fp64, the e summed in fp64 in expert order, p = e *
// fl32(1 / sum)) and weights p / fl32(sum_K p in fp64, slot order);
// expert_scale[e] multiplies the weights of every kind.
struct Gating {
    int kind = 0;
    const float *sel_bias = nullptr;
    const float *expert_scale = nullptr;
    float scaling = 1.f;
    float eps = 0.f;
};

__device__ inline float gating_sigmoid(float x) { return (float)(1.0 / (1.0 + exp(-(double)x))); }

// the wave's largest value, uniform: max within 16-lane rows (DPP), then
// rows 0 -> 1, 2 -> 3 (row_bcast:15) and row 1 -> 2, 3 (row_bcast:31): lane
// 63 holds the maximum of all four rows
__device__ inline float wave_max_uniform(float m) {
    m = fmaxf(m, dpp_f<0xB1>(m));
    m = fmaxf(m, dpp_f<0x4E>(m));
    m = fmaxf(m, dpp_f<0x141>(m));
    m = fmaxf(m, dpp_f<0x140>(m));
    const int mi = __builtin_bit_cast(int, m);
    m = fmaxf(m, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(mi, mi, 0x142, 0xA, 0xF, false)));
    const int mj = __builtin_bit_cast(int, m);
    m = fmaxf(m, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(mj, mj, 0x143, 0xC, 0xF, false)));
    return lane_f(m, 63);
}

// raw[i]: the logit of expert 64 i + lane (any value past E)
__device__ inline void topk_softmax_regs(const float (&raw)[TOPK_MAX_PER_LANE], int E, int K, int lane, int &mysel,
                                         float &myw, bool want_w, const Gating &gt) {
    const int nper = (E + 63) >> 6;
    float v[TOPK_MAX_PER_LANE];
#pragma unroll
    for (int i = 0; i < TOPK_MAX_PER_LANE; ++i) {
        const int e = lane + 64 * i;
        if (e < E) {
            v[i] = raw[i];
            if (gt.kind == 1) v[i] = gating_sigmoid(v[i]) + (gt.sel_bias ? gt.sel_bias[e] : 0.f);
        } else {
            v[i] = -INFINITY;
        }
    }
    if (gt.kind == 2) {
        float mx = v[0];
#pragma unroll
        for (int i = 1; i < TOPK_MAX_PER_LANE; ++i) mx = fmaxf(mx, v[i]);
        mx = wave_max(mx);
        float ex[TOPK_MAX_PER_LANE];
#pragma unroll
        for (int i = 0; i < TOPK_MAX_PER_LANE; ++i)
            ex[i] = lane + 64 * i < E ? (float)exp((double)(v[i] - mx)) : 0.f;
        // the sum in expert order e = 64 i + lane: uniform lane reads
        double sum = 0.0;
#pragma unroll
        for (int i = 0; i < TOPK_MAX_PER_LANE; ++i) {
            if (i >= nper) break;
            const int eb = __builtin_bit_cast(int, ex[i]);
            for (int j = 0; j < 64; ++j) sum = sum + (double)__builtin_bit_cast(float, __builtin_amdgcn_readlane(eb, j));
        }
        const float inv = (float)(1.0 / sum);
#pragma unroll
        for (int i = 0; i < TOPK_MAX_PER_LANE; ++i)
            if (lane + 64 * i < E) v[i] = ex[i] * inv;
    }
    mysel = 0;
    float mys = 0.f;   // lane k: the k-th selected value
    for (int r = 0; r < K; ++r) {
        float m = v[0];
#pragma unroll
        for (int i = 1; i < TOPK_MAX_PER_LANE; ++i)
            if (i < nper) m = fmaxf(m, v[i]);
        const float s = wave_max_uniform(m);
        int e = -1;
#pragma unroll
        for (int i = 0; i < TOPK_MAX_PER_LANE; ++i) {
            if (i >= nper) break;
            const unsigned long long b = __ballot(v[i] == s);
            if (e < 0 && b != 0ull) e = 64 * i + (int)__builtin_ctzll(b);
        }
        e = __builtin_amdgcn_readfirstlane(e);
#pragma unroll
        for (int i = 0; i < TOPK_MAX_PER_LANE; ++i)
            if (e == 64 * i + lane) v[i] = __builtin_nanf("");
        if (lane == r) {
            mysel = e;
            mys = s;
        }
    }
    if (!want_w) {
        myw = 0.f;
        return;
    }
    if (gt.kind == 1) {
        // the logit of the lane's selected expert, from the lane that holds it
        float lsel = 0.f;
#pragma unroll
        for (int i = 0; i < TOPK_MAX_PER_LANE; ++i) {
            const float t = __shfl(raw[i], mysel & 63, 64);
            if (i == (mysel >> 6)) lsel = t;
        }
        const float sg = lane < K ? gating_sigmoid(lsel) : 0.f;
        double sum = 0.0;
        for (int k = 0; k < K; ++k) sum = sum + (double)lane_f(sg, k);
        myw = sg / ((float)sum + gt.eps) * gt.scaling;
    } else if (gt.kind == 2) {
        const float p = lane < K ? mys : 0.f;
        double sum = 0.0;
        for (int k = 0; k < K; ++k) sum = sum + (double)lane_f(p, k);
        myw = p / (float)sum;
    } else {
        myw = softmax_selected_wave(lane < K ? mys : 0.f, K, lane);
    }
    if (gt.expert_scale && lane < K) myw = myw * gt.expert_scale[mysel];
}

// the same, on the E logits at l
__device__ inline void topk_softmax_wave(const float *l, int E, int K, int lane, int &mysel, float &myw, bool want_w,
                                         const Gating &gt = Gating{}) {
    float raw[TOPK_MAX_PER_LANE];
#pragma unroll
    for (int i = 0; i < TOPK_MAX_PER_LANE; ++i) {
        const int e = lane + 64 * i;
        raw[i] = e < E ? l[e] : 0.f;
    }
    topk_softmax_regs(raw, E, K, lane, mysel, myw, want_w, gt);
}

}  // namespace mimoe
