// q8h.hpp - one 256-value Q8_K block as fp16 d*q values in a k-quant
// consumer's 32x32x16 MFMA K order, computed by 16 lanes (k_q8k_rows_h, and
// the GLU epilogue of the 32-row gate/up GEMM).
//
// Lane s of a block owns 16 values: four runs of 4 consecutive values, at
// base(g, s) and base(g, s) + 32 for g = 0, 1 - so each lane loads its values
// straight in the output order and writes 32 bytes at 16 s; no code bytes are
// packed, staged or unpacked.  d and q: ggml's quantize_row_q8_K_ref (d =
// 1 / (127 / m), q = rint(127 / m * x), m the largest |x|); the value d*q does
// not depend on which element of largest |x| fixes the scale's sign (-127 /
// (+-m) = -+(127 / m), a correctly rounded divide is odd; codes round half to
// even, odd; |127 x / m| < 127.5), so d and q change sign together and their
// product keeps its bits - only the sign of a zero product may differ from
// the element-first form, and a zero adds nothing to an MFMA sum that starts
// at +0.
#pragma once

#include "common.hpp"
#include "wave_ops.hpp"

namespace mimoe {

// fp16 orders of Q8_K outputs: XO_Q4 / XO_Q6 the 32x32x16 order of a Q4_K /
// Q6_K consumer, XO_ANY element by element (whatever the output asks for)
enum { XO_ANY = 0, XO_Q4 = 1, XO_Q6 = 2 };

// first of lane s's 4 values A of half g (B: the 4 at + 32); output slot p
// = 0..7 of the half holds Q4_K A0 A2 B0 B2 A1 A3 B1 B3, Q6_K A0..A3 B0..B3
template <int XO>
__device__ __forceinline__ int q8h_base(int s, int g) {
    return XO == XO_Q4 ? 64 * (2 * (s >> 3) + g) + 4 * (s & 7)
                       : 128 * (s >> 3) + 16 * g + 4 * ((s & 7) >> 1) + 64 * (s & 1);
}

// lane s's 16 values of the block at x (fp32 or fp16, 16-byte / 8-byte
// aligned runs) in its output slots
template <int XO, typename ST>
__device__ __forceinline__ void q8h_gather(const ST *x, int s, float (&v)[16]) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {   // run r: half g = r >> 1, A (r even) or B
        const int g = r >> 1, half = r & 1;
        const int start = q8h_base<XO>(s, g) + 32 * half;
        float w[4];
        if constexpr (sizeof(ST) == 2) {
            const uint2 u = *(const uint2 *)(x + start);
            const half2_t h0 = __builtin_bit_cast(half2_t, u.x), h1 = __builtin_bit_cast(half2_t, u.y);
            w[0] = (float)h0[0]; w[1] = (float)h0[1]; w[2] = (float)h1[0]; w[3] = (float)h1[1];
        } else {
            const float4 f = *(const float4 *)(x + start);
            w[0] = f.x; w[1] = f.y; w[2] = f.z; w[3] = f.w;
        }
        // the run's 4 values to their output slots
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int p = XO == XO_Q4 ? (i & 1) * 4 + (i >> 1) + 2 * half : i + 4 * half;
            v[8 * g + p] = w[i];
        }
    }
}

// the block's scale from the 16 lanes' values (every lane of the 16-lane row
// takes part: DPP inside the row), then, when live, lane s's 16 fp16 d*q to
// dst (the block's first value) + 16 s; a scale whose codes leave the fp16
// range is counted in range_total (lane 0 of the block)
__device__ __forceinline__ void q8h_quant_store(const float (&v)[16], bool live, _Float16 *dst, int s,
                                                int32_t *range_total) {
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) m = fmaxf(m, fabsf(v[i]));
    m = fmaxf(m, dpp_f<0xB1>(m));
    m = fmaxf(m, dpp_f<0x4E>(m));
    m = fmaxf(m, dpp_f<0x141>(m));
    m = fmaxf(m, dpp_f<0x140>(m));   // the block's largest |x|
    const bool zero = m == 0.f;
    const float iscale = zero ? 0.f : 127.f / m;
    const float d = zero ? 0.f : 1 / iscale;
    if (!live) return;
    uint32_t h[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        half2_t hh;
        hh[0] = f16_sat(d * __builtin_rintf(iscale * v[2 * k]));
        hh[1] = f16_sat(d * __builtin_rintf(iscale * v[2 * k + 1]));
        h[k] = __builtin_bit_cast(uint32_t, hh);
    }
    if (s == 0 && range_total && f16_over(d)) atomicAdd(range_total, 1);
    uint4 *o = (uint4 *)(dst + 16 * s);
    o[0] = make_uint4(h[0], h[1], h[2], h[3]);
    o[1] = make_uint4(h[4], h[5], h[6], h[7]);
}

}  // namespace mimoe
