// common.hpp - device helpers shared by the MI355X MoE kernels.
//
// Block formats (ggml block_q4_K / block_q6_K / block_q8_K; byte layouts in
// convert/q4k.py:9-10, convert/q6k.py:10-11, scripts/test_q6k.py:41-62):
//   Q4_K  144 B / 256 values: d f16 | dmin f16 | scales[12] (6-bit pairs) | qs[128]
//   Q6_K  210 B / 256 values: ql[128] | qh[64] | scales[16] i8 | d f16
//   Q8_K  (activations)      : d f32 | qs[256] i8 | bsums[16] i16
//
// All kernels are compiled with -ffp-contract=off: an expression rounds as
// written, and fused multiply-adds are requested explicitly (fmaf /
// __builtin_elementwise_fma), so the fp paths that must match the CPU oracle
// bit for bit (RNG, quantizers, router, Q8_K) do.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mimoe {

constexpr int QK = 256;
constexpr int Q4K_BYTES = 144;
constexpr int Q6K_BYTES = 210;
constexpr int WAVE = 64;

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- fp16 bits
// IEEE binary16 <-> binary32 by integer arithmetic (round to nearest even),
// independent of the hardware denormal mode; same code as the CPU oracle.
__device__ __host__ inline float fp16_bits_to_f32(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    const uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            // value = man * 2^-24, normalize
            int e = 0;
            uint32_t m = man;
            while (!(m & 0x400u)) { m <<= 1; e++; }
            m &= 0x3ffu;
            bits = sign | ((uint32_t)(113 - e) << 23) | (m << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    return __builtin_bit_cast(float, bits);
}

__device__ __host__ inline uint32_t f32_to_fp16_bits(float f) {
    const uint32_t x = __builtin_bit_cast(uint32_t, f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u);
    if (ax >= 0x477ff000u) return sign | 0x7c00u;
    if (ax < 0x38800000u) {
        if (ax < 0x33000000u) return sign;
        const uint32_t e = ax >> 23;
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - e;
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return sign | q;
    }
    const uint32_t e = (ax >> 23) - 112u;
    const uint32_t m = ax & 0x7fffffu;
    uint32_t q = (e << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return sign | q;
}

// hardware conversion for hot paths (exact for normal and subnormal fp16)
__device__ inline float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// Work-group barrier for LDS hand-offs: this wave's LDS accesses complete,
// then s_barrier.  Outstanding global loads and stores stay in flight
// (__syncthreads also waits for them, vmcnt(0), which costs a memory round
// trip where a kernel has just issued loads or stores it does not need yet).
// The asm memory clobber keeps the compiler from moving memory accesses across
// the barrier.  Not for global data that other threads of the work-group read.
__device__ inline void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");
}

// This wave's global loads and stores complete (vmcnt(0); on gfx9 the
// counter covers stores too), as an asm statement with a memory clobber: the
// compiler neither sinks earlier memory accesses below it nor hoists later
// ones above it (__builtin_amdgcn_s_waitcnt alone is not a compiler barrier).
// A completion word stored after it is seen only after the data stored
// before it.
__device__ inline void vm_drain() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __host__ inline int imin(int a, int b) { return a < b ? a : b; }
__device__ __host__ inline int imax(int a, int b) { return a > b ? a : b; }

// ggml nearest_int: round half to even through the 1.5*2^23 constant
__device__ __host__ inline int nearest_int(float fval) {
    const float val = fval + 12582912.f;
    const int i = __builtin_bit_cast(int, val);
    return (i & 0x007fffff) - 0x00400000;
}

// 6-bit scale / min of sub-block j (convert/q4k.py:107-110)
__device__ __host__ inline void scale_min_k4(int j, const uint8_t *q, int &d, int &m) {
    if (j < 4) {
        d = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4);
    }
}

// the same unpack from the three packed dwords w0..w2 = scales[0..12) held in
// registers (j may vary per lane; no local-memory array, no branch)
__device__ inline void scale_min_k4_reg(int j, uint32_t w0, uint32_t w1, uint32_t w2, int &d, int &m) {
    const uint32_t sh = 8u * (uint32_t)(j & 3);
    const int b0 = (int)((w0 >> sh) & 0xffu), b1 = (int)((w1 >> sh) & 0xffu), b2 = (int)((w2 >> sh) & 0xffu);
    const int d_lo = b0 & 63, m_lo = b1 & 63;
    const int d_hi = (b2 & 0xF) | ((b0 >> 6) << 4), m_hi = (b2 >> 4) | ((b1 >> 6) << 4);
    const bool lo = j < 4;
    d = lo ? d_lo : d_hi;
    m = lo ? m_lo : m_hi;
}

// fp16 operand d*q of the GEMM path, saturated at the largest finite fp16:
// a Q8_K block whose scale puts 127 d beyond it (|x| > 65504) is counted by
// its producer (range_total) instead of turning into inf.
constexpr float kF16Max = 65504.f;
__device__ inline _Float16 f16_sat(float v) { return (_Float16)fminf(fmaxf(v, -kF16Max), kF16Max); }
__device__ inline bool f16_over(float d) { return fabsf(d) * 127.f > kF16Max; }

// Offset of a Q4_K sub-block dequantized from centred codes: with s = d*sc,
// w = s q - dmin m = s (q - 8) + (8 s - dmin m).  Both products are exact in
// fp32 (11-bit d times a 6-bit integer), so the offset is rounded once.
__device__ inline float q4k_center(float d, int sc, float dmin, int m) {
    return 8.0f * (d * (float)sc) - dmin * (float)m;
}

// ---------------------------------------------------------------- MFMA K order
// The prefill GEMM feeds v_mfma_f32_16x16x32_f16 with 8 fp16 values per lane.
// Inside a 256-value super-block, MFMA step s (0..7), lane group g (lane/16,
// 0..3) and operand slot p (0..7) address K position pos = 32*s + 8*g + p.
// The weight side dequantizes straight from the GGUF block layout, so each
// (s, g, p) names one element of the block; activations are stored in the
// same order so both operands agree.
//
// Q4_K: lane group g owns qs[32g .. 32g+32) (elements 64g..64g+63); step s
// uses the dword qs[32g+4s .. +4): low nibbles are elements 64g+4s+{0..3},
// high nibbles 64g+32+4s+{0..3}.  The dequant emits pairs (n0,n4) (n1,n5)
// (n2,n6) (n3,n7) of that dword's nibbles.
__device__ __host__ inline int q4k_elem(int pos) {
    const int s = pos >> 5, g = (pos >> 3) & 3, p = pos & 7;
    const int off[8] = {0, 2, 32, 34, 1, 3, 33, 35};
    return 64 * g + 4 * s + off[p];
}
// Q6_K: lane group g covers half h = g/2, l in 16*(g%2) .. +16; step s = 2j+w
// covers l0 = 16*(g%2) + 4j and, for w = 0, quarters q1 (l0..l0+3) and q2
// (32+l0..); for w = 1, quarters q3 (64+l0..) and q4 (96+l0..).
__device__ __host__ inline int q6k_elem(int pos) {
    const int s = pos >> 5, g = (pos >> 3) & 3, p = pos & 7;
    return 128 * (g >> 1) + 16 * (g & 1) + 4 * (s >> 1) + 64 * (s & 1) + 32 * (p >> 2) + (p & 3);
}
__device__ __host__ inline int mfma_elem(int wtype, int pos) {
    return wtype == 14 ? q6k_elem(pos) : q4k_elem(pos);
}

// v_mfma_f32_32x32x16_f16 order: step s (0..15), lane group g (lane/32, 0..1),
// slot p (0..7), pos = 16*s + 8*g + p.
// Q4_K: steps 8 h .. 8 h + 7 cover half h of the block (qs[64h..64h+64));
// lane group g takes chunk c = 2 h + g (qs[32c..32c+32)); step s uses dword
// s&7 of that chunk: elements 64c + 4(s&7) + {0..3} (low nibbles, sub-block
// 2c) and 64c + 32 + 4(s&7) + {0..3} (high, 2c+1), in the operand order of
// q4k_elem.
__device__ __host__ inline int q4k_elem32(int pos) {
    const int s = pos >> 4, g = (pos >> 3) & 1, p = pos & 7;
    const int off[8] = {0, 2, 32, 34, 1, 3, 33, 35};
    return 64 * (2 * (s >> 3) + g) + 4 * (s & 7) + off[p];
}
// Q6_K: steps 8 h .. 8 h + 7 cover half h of the block (ql[64h..64h+64),
// qh[32h..32h+32), scales[8h..8h+8)); lane group g takes the quarter-row
// positions l = 16 g .. 16 g + 15; step s = 8 h + 2 jj + w covers
// l = 16 g + 4 jj .. + 3 of quarters (q1, q2) for w = 0 or (q3, q4) for w = 1;
// slots 0..3 the first quarter, 4..7 the second.
__device__ __host__ inline int q6k_elem32(int pos) {
    const int s = pos >> 4, g = (pos >> 3) & 1, p = pos & 7;
    return 128 * (s >> 3) + 16 * g + 4 * ((s & 7) >> 1) + (p & 3) + 32 * (p >> 2) + 64 * (s & 1);
}
__device__ __host__ inline int q4k_pos32(int e) {
    const int c = e >> 6, r = e & 63, hi = r >> 5, r2 = r & 31, j = r2 >> 2, lo = r2 & 3;
    const int g = c & 1, s = 8 * (c >> 1) + j, p = (lo & 1) * 4 + hi * 2 + (lo >> 1);
    return 16 * s + 8 * g + p;
}
__device__ __host__ inline int q6k_pos32(int e) {
    const int h = e >> 7, r = e & 127, qq = r >> 5, l = r & 31;
    const int s = 8 * h + 2 * ((l >> 2) & 3) + (qq >> 1), p = 4 * (qq & 1) + (l & 3);
    return 16 * s + 8 * (l >> 4) + p;
}
__device__ __host__ inline int mfma32_elem(int wtype, int pos) {
    return wtype == 14 ? q6k_elem32(pos) : q4k_elem32(pos);
}
__device__ __host__ inline int mfma32_pos(int wtype, int e) {
    return wtype == 14 ? q6k_pos32(e) : q4k_pos32(e);
}

// ---------------------------------------------------------------- wave helpers
__device__ inline float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ inline int wave_sum_i(int v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ inline float wave_sum_f(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// (|x| max, first index) reduction used by Q8_K: ggml keeps the first element
// with the largest magnitude (strict '>'), whose signed value sets the scale.
struct AmaxIdx {
    float ax;
    int idx;
    float val;
};
__device__ inline AmaxIdx amax_better(AmaxIdx a, AmaxIdx b) {
    // selects, not branches (non-short-circuit operators)
    const bool t = (b.ax > a.ax) | ((b.ax == a.ax) & (b.idx < a.idx));
    AmaxIdx r;
    r.ax = t ? b.ax : a.ax;
    r.idx = t ? b.idx : a.idx;
    r.val = t ? b.val : a.val;
    return r;
}
__device__ inline AmaxIdx wave_amax_idx(AmaxIdx a, int width = 64) {
    for (int o = width >> 1; o > 0; o >>= 1) {
        AmaxIdx b;
        b.ax = __shfl_xor(a.ax, o, 64);
        b.idx = __shfl_xor(a.idx, o, 64);
        b.val = __shfl_xor(a.val, o, 64);
        a = amax_better(a, b);
    }
    return a;
}

}  // namespace mimoe
