// k_b32.hip - expert tables in the 32-value block formats (Q4_0, Q5_0, Q8_0)
// and in F16: the types the reference's converters write by default (Q8_0:
// convert/convert_hf_to_gguf.py:55-57, convert/convert_qwen3omni.py:60-61,135;
// Q5_0: convert/convert_nemotronomni.py:113-114; F16 / Q4_0:
// convert/convert_diffusiongemma.py:62).
//
// ggml-cpu semantics (ggml_mul_mat_id with these tables): the activation rows
// are converted to the weight type's vec_dot_type first, Q8_0 (32-value blocks,
// d = amax / 127 stored as fp16) for Q4_0 / Q5_0 / Q8_0 and fp16 (round to
// nearest even) for F16; each block then contributes an exact integer dot
// times the two fp16 scales, F16 rows exact fp16 x fp16 products.
//
//  * quantizers of weight rows (mi_quantize; ggml quantize_row_*_ref),
//  * the activation pass: Q8_0 codes + fp16 scales (GEMV), fp16(d q) or fp16(x)
//    rows (GEMM, and F16's GEMV),
//  * the grouped GEMV (decode): 8 lanes per weight row, each lane one 32-value
//    block per 256 values, integer dots on v_dot4_i32_i8 / fp16 pairs on
//    v_dot2_f32_f16,
//  * the grouped GEMM (prefill) on v_mfma_f32_32x32x16_f16: a work-group owns
//    a balanced tile of up to 192 dispatched rows of one expert and 128 weight
//    rows (GLU: 64 gate and the 64 matching up rows), each wave 32 of them
//    against all the tile's rows (6 MFMA tiles, one dequantized weight operand
//    feeds all of them); activations staged through LDS 64 K values at a
//    time (double buffered, 16-byte chunks swizzled by row), weights loaded
//    into registers one stage ahead and dequantized to fp16 in registers.
//
// Block layouts (ggml block_q4_0 / q5_0 / q8_0, no padding, so blocks start
// at any even byte):
//   Q4_0 18 B: d f16 | qs[16]            value j < 16: low nibble of qs[j], 16 + j: high; x = d (q - 8)
//   Q5_0 22 B: d f16 | qh u32 | qs[16]   5th bit of value j: bit j of qh;                 x = d (q - 16)
//   Q8_0 34 B: d f16 | qs[32] i8                                                          x = d q
#include "act.hpp"
#include "common.hpp"
#include "launch.hpp"

namespace mimoe {

typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int WT> struct B32Fmt;
template <> struct B32Fmt<2> { static constexpr int BYTES = 18, WORDS = 5, OFF = 8; };    // Q4_0
template <> struct B32Fmt<6> { static constexpr int BYTES = 22, WORDS = 6, OFF = 16; };   // Q5_0
template <> struct B32Fmt<8> { static constexpr int BYTES = 34, WORDS = 9, OFF = 0; };    // Q8_0

// ------------------------------------------------------------------ block loads
// The WORDS aligned dwords that intersect the block at p (an even address; a
// block spans WORDS dwords at either alignment).  Every dword read holds at
// least one byte of the block, so no read leaves the table's pages.
template <int WT>
__device__ inline void b32_words(const uint8_t *p, uint32_t (&w)[B32Fmt<WT>::WORDS], uint32_t &mis) {
    const uintptr_t a = (uintptr_t)p;
    mis = (uint32_t)(a & 2u);
    const uint32_t *q = (const uint32_t *)(a - mis);
#pragma unroll
    for (int i = 0; i < B32Fmt<WT>::WORDS; ++i) w[i] = q[i];
}
// the 4 block bytes from byte offset OFF (even): bytes [mis + OFF, ...) of
// the words (compile-time word indices keep the words in registers)
template <int OFF, int N>
__device__ inline uint32_t b32_dword(const uint32_t (&w)[N], uint32_t mis) {
    constexpr int k = OFF >> 2;   // OFF % 4 is 0 or 2
    if constexpr ((OFF & 2) == 0) return mis ? __builtin_amdgcn_alignbyte(w[k + 1], w[k], 2) : w[k];
    else return mis ? w[k + 1] : __builtin_amdgcn_alignbyte(w[k + 1], w[k], 2);
}
__device__ inline float b32_d(uint32_t w0, uint32_t mis) {
    return fp16_bits_to_f32(mis ? (w0 >> 16) : (w0 & 0xffffu));
}

// signed codes of values 4i .. 4i + 3 of the block as bytes, i < 8 (Q8_0:
// the codes; Q4_0 / Q5_0: the unsigned codes q, the offset is applied by the
// caller through the block's activation sum)
template <int WT, int I>
__device__ inline uint32_t b32_codes4(const uint32_t (&w)[B32Fmt<WT>::WORDS], uint32_t mis) {
    if constexpr (WT == 8) {
        return b32_dword<2 + 4 * I>(w, mis);
    } else {
        constexpr int QS = WT == 2 ? 2 : 6;
        const uint32_t qs = b32_dword<QS + 4 * (I & 3)>(w, mis);
        uint32_t v = I < 4 ? (qs & 0x0F0F0F0Fu) : ((qs >> 4) & 0x0F0F0F0Fu);
        if constexpr (WT == 6) {
            const uint32_t qh = b32_dword<2>(w, mis);
            const uint32_t b = (qh >> (4 * I)) & 0xFu;   // 5th bits of values 4I .. 4I + 3
            v |= ((b & 1u) << 4) | ((b & 2u) << 11) | ((b & 4u) << 18) | ((b & 8u) << 25);
        }
        return v;
    }
}
template <int WT, int I = 0>
__device__ inline void b32_codes_all(const uint32_t (&w)[B32Fmt<WT>::WORDS], uint32_t mis, uint32_t (&c)[8]) {
    c[I] = b32_codes4<WT, I>(w, mis);
    if constexpr (I < 7) b32_codes_all<WT, I + 1>(w, mis, c);
}

// ------------------------------------------------------------------ quantizers
// One thread per 32-value block, the oracle's statement order (the scale and
// codes bit for bit; fp16 by integer rounding, independent of denormal mode).
template <int WT>
__global__ void __launch_bounds__(256) k_quantize_b32(const float *src, uint8_t *dst, int64_t nblocks) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const float *x = src + i * 32;
    if constexpr (WT == 1) {
        uint32_t *o = (uint32_t *)(dst + i * 64);
#pragma unroll
        for (int j = 0; j < 16; ++j) o[j] = f32_to_fp16_bits(x[2 * j]) | (f32_to_fp16_bits(x[2 * j + 1]) << 16);
        return;
    }
    uint8_t *y = dst + i * B32Fmt<WT == 1 ? 8 : WT>::BYTES;
    if constexpr (WT == 8) {
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint32_t dh = f32_to_fp16_bits(d);
        y[0] = (uint8_t)dh;
        y[1] = (uint8_t)(dh >> 8);
        for (int j = 0; j < 32; ++j) y[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
    } else {
        constexpr float NEG = WT == 2 ? -8.0f : -16.0f;
        constexpr float ADD = WT == 2 ? 8.5f : 16.5f;
        constexpr int TOP = WT == 2 ? 15 : 31;
        float amax = 0.0f, mx = 0.0f;
        for (int j = 0; j < 32; ++j) {
            const float v = x[j];
            if (amax < fabsf(v)) {
                amax = fabsf(v);
                mx = v;
            }
        }
        const float d = mx / NEG;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint32_t dh = f32_to_fp16_bits(d);
        y[0] = (uint8_t)dh;
        y[1] = (uint8_t)(dh >> 8);
        uint32_t qh = 0;
        uint8_t *qs = y + (WT == 2 ? 2 : 6);
        for (int j = 0; j < 16; ++j) {
            const float x0 = x[j] * id, x1 = x[16 + j] * id;
            const int8_t t0 = (int8_t)(x0 + ADD), t1 = (int8_t)(x1 + ADD);
            const uint32_t c0 = (uint32_t)(uint8_t)(t0 < TOP ? t0 : TOP);
            const uint32_t c1 = (uint32_t)(uint8_t)(t1 < TOP ? t1 : TOP);
            qs[j] = (uint8_t)((c0 & 0x0Fu) | ((c1 & 0x0Fu) << 4));
            qh |= ((c0 & 0x10u) >> 4) << j;
            qh |= ((c1 & 0x10u) >> 4) << (j + 16);
        }
        if constexpr (WT == 6)
            for (int b = 0; b < 4; ++b) y[2 + b] = (uint8_t)(qh >> (8 * b));
    }
}

int launch_quantize_b32(int type, const float *src, void *dst, int64_t nblocks, hipStream_t st) {
    if (nblocks <= 0) return 0;
    const dim3 grid((unsigned)((nblocks + 255) / 256));
    uint8_t *o = (uint8_t *)dst;
    switch (type) {
    case 1: hipLaunchKernelGGL(k_quantize_b32<1>, grid, dim3(256), 0, st, src, o, nblocks); break;
    case 2: hipLaunchKernelGGL(k_quantize_b32<2>, grid, dim3(256), 0, st, src, o, nblocks); break;
    case 6: hipLaunchKernelGGL(k_quantize_b32<6>, grid, dim3(256), 0, st, src, o, nblocks); break;
    case 8: hipLaunchKernelGGL(k_quantize_b32<8>, grid, dim3(256), 0, st, src, o, nblocks); break;
    default: return -3;
    }
    return hip_check_launch();
}

// ------------------------------------------------------------------ activations
// Rows of K values (K % 32 == 0, row r at src + r * ld) into the operand form
// of a consumer weight type (B32Prep): Q8_0 codes [r][K] and fp16 scales
// [r][K/32] (GEMV of Q4_0 / Q5_0 / Q8_0), fp16(d q) rows [r][K] (their GEMM),
// or fp16(x) rows [r][K] (F16, both paths).  One block per 32 lanes; the Q8_0
// scale and codes are the oracle's bit for bit.
template <typename S>
__global__ void __launch_bounds__(256) k_prep_b32(const S *src, int64_t ld, int64_t nrows, int64_t K, B32Prep o) {
    const int64_t nbr = K / 32;
    const int64_t blk = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 5;
    const int j = threadIdx.x & 31;
    if (blk >= nrows * nbr) return;   // a whole half-wave leaves together
    const int64_t r = blk / nbr, b = blk - r * nbr;
    float v = (float)src[r * ld + 32 * b + j];
    if (o.pre_act == 4) {   // ggml_sqr(ggml_relu(u)) before the quantization
        const float t = v > 0.f ? v : 0.f;
        v = t * t;
    }
    const int64_t at = r * K + 32 * b + j;
    if (o.mode == B32_PREP_F16) {
        o.xh[at] = __builtin_bit_cast(_Float16, (uint16_t)f32_to_fp16_bits(v));
        return;
    }
    float amax = fabsf(v);
#pragma unroll
    for (int s = 1; s < 32; s <<= 1) amax = fmaxf(amax, __shfl_xor(amax, s, 32));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const int q = (int)roundf(v * id);
    const uint32_t dh = f32_to_fp16_bits(d);
    if (o.mode == B32_PREP_CODES) {
        o.q8[at] = (int8_t)q;
        if (j == 0) o.dh[r * nbr + b] = (uint16_t)dh;
    } else {
        o.xh[at] = (_Float16)(fp16_bits_to_f32(dh) * (float)q);
    }
}

int launch_prep_b32(const float *src, int64_t ld, int64_t nrows, int64_t K, const B32Prep &o, hipStream_t st) {
    if (nrows <= 0) return 0;
    if (K % 32) return -6;
    const int64_t threads = nrows * K;
    hipLaunchKernelGGL(k_prep_b32<float>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, src, ld, nrows,
                       K, o);
    return hip_check_launch();
}

// ------------------------------------------------------------------ GEMV
// dot of one 32-value block (this lane's) with the activation row's block
template <int WT>
__device__ inline float b32_block_dot(const uint8_t *wblk, const int8_t *xq, float dx) {
    uint32_t w[B32Fmt<WT>::WORDS], mis;
    b32_words<WT>(wblk, w, mis);
    const uint4 xa = *(const uint4 *)xq, xb = *(const uint4 *)(xq + 16);
    const uint32_t xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
    uint32_t cw[8];
    b32_codes_all<WT>(w, mis, cw);
    int isum = 0, xsum = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        isum = __builtin_amdgcn_sdot4((int)cw[i], (int)xv[i], isum, false);
        if constexpr (WT != 8) xsum = __builtin_amdgcn_sdot4(0x01010101, (int)xv[i], xsum, false);
    }
    const float dw = b32_d(w[0], mis);
    // the expression orders of ggml_vec_dot_q{4,5,8}_0_q8_0
    if constexpr (WT == 8) return (float)isum * (dw * dx);
    else if constexpr (WT == 6) return (dw * dx) * (float)(isum - 16 * xsum);
    else return (float)(isum - 8 * xsum) * dw * dx;
}

__device__ inline float f16_block_dot(const uint8_t *wblk, const _Float16 *xh) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint4 wv = *(const uint4 *)(wblk + 16 * c);
        const uint4 xv = *(const uint4 *)(xh + 8 * c);
        const uint32_t wa[4] = {wv.x, wv.y, wv.z, wv.w}, xa[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
            acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, wa[i]), __builtin_bit_cast(half2_t, xa[i]),
                                         acc, false);
    }
    return acc;
}

// Grid (column blocks, active experts), 4 waves of 8 row groups x 8 lanes; a
// row group owns one weight row (GLU: groups 0-3 the gate rows, 4-7 the
// matching up rows), lane sl takes blocks sl, sl + 8, ... of it for every
// token of the expert (the row's bytes come from HBM once, from the caches
// for the later tokens).
template <int WT>
__global__ void __launch_bounds__(256) k_gemv_b32(B32Args g) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rs = lane >> 3, sl = lane & 7;
    const int j = blockIdx.y;
    if (j >= *g.n_active) return;
    const int e = g.active_e[j];
    const int cnt = g.counts[e], off = g.offsets[e];
    const bool glu = g.glu != 0;
    const int64_t col0 = ((int64_t)blockIdx.x * 4 + wave) * (glu ? 4 : 8);
    int64_t col = col0 + (glu ? (rs & 3) : rs);
    const bool col_ok = col < g.ncols;
    if (!col_ok) col = 0;
    const ExpertMat *M = &g.a;
    int64_t wrow = col;
    if (glu && rs >= 4) {
        if (g.fused) wrow = g.I + col;
        else M = &g.b;
    }
    const uint8_t *rowp = M->data + (int64_t)e * M->mat_bytes + wrow * M->row_bytes;
    const int64_t Kin = M->K, nbr = Kin / 32;
    for (int m = 0; m < cnt; ++m) {
        const int p = g.perm[off + m];
        const int64_t arow = g.ne11 == 1 ? p / g.K : p;
        float acc = 0.f;
        for (int64_t b = sl; b < nbr; b += 8) {
            if constexpr (WT == 1) {
                acc += f16_block_dot(rowp + 64 * b, g.xh + arow * Kin + 32 * b);
            } else {
                const float dx = fp16_bits_to_f32(g.dh[arow * nbr + b]);
                acc += b32_block_dot<WT>(rowp + (int64_t)B32Fmt<WT>::BYTES * b, g.q8 + arow * Kin + 32 * b, dx);
            }
        }
        acc += __shfl_xor(acc, 1, 64);
        acc += __shfl_xor(acc, 2, 64);
        acc += __shfl_xor(acc, 4, 64);
        if (glu) {
            const float other = __shfl(acc, lane + 32 < 64 ? lane + 32 : lane, 64);
            if (rs < 4 && sl == 0 && col_ok) g.y[(int64_t)p * g.ldy + col] = act_pair(g.act, acc, other);
        } else {
            if (sl == 0 && col_ok) g.y[(int64_t)p * g.ldy + col] = acc;
        }
    }
}

// ------------------------------------------------------------------ GEMM
constexpr int GB_BM = G4_BM;        // rows per tile (balanced dispatch tiles)
constexpr int GB_RT = GB_BM / 32;   // row tiles of 32
constexpr int GB_BK = 64;           // K values per stage
constexpr int GB_ACH = GB_BM * (GB_BK / 8) / 256;   // 16-byte activation chunks per thread per stage

// this lane's weight operands of one stage: for K16 step s, K values
// k0 + 16 s + 8 h + (0..7) of its row (h = lane / 32), as fp16
template <int WT> struct GBRaw { uint32_t w0[B32Fmt<WT>::WORDS], w1[B32Fmt<WT>::WORDS]; uint32_t mis0, mis1; };
template <> struct GBRaw<1> { uint4 v[4]; };

template <int WT>
__device__ inline void gb_load(const uint8_t *row, int64_t k0, int64_t Kin, int h, GBRaw<WT> &r) {
    if constexpr (WT == 1) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int64_t k = k0 + 16 * s + 8 * h;
            r.v[s] = k < Kin ? *(const uint4 *)(row + 2 * k) : make_uint4(0, 0, 0, 0);
        }
    } else {
        const int64_t blk = k0 / 32;
        b32_words<WT>(row + (int64_t)B32Fmt<WT>::BYTES * blk, r.w0, r.mis0);
        if (blk + 1 < Kin / 32) {
            b32_words<WT>(row + (int64_t)B32Fmt<WT>::BYTES * (blk + 1), r.w1, r.mis1);
        } else {
#pragma unroll
            for (int i = 0; i < B32Fmt<WT>::WORDS; ++i) r.w1[i] = 0u;   // d = 0: zero weights
            r.mis1 = 0u;
        }
    }
}

// 4 unsigned byte codes (+ bias making them unsigned) -> 2 half2 of (q - off) * d
__device__ inline void gb_bytes_h(uint32_t x, float off, half2_t d2, half2_t &lo, half2_t &hi) {
    // bytes b0..b3 into fp16 1024 + b (exact), then - (1024 + off), then * d
    const uint32_t p01 = __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u);
    const uint32_t p23 = __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u);
    const _Float16 c = (_Float16)(1024.0f + off);
    const half2_t cc = {c, c};
    lo = (__builtin_bit_cast(half2_t, p01) - cc) * d2;
    hi = (__builtin_bit_cast(half2_t, p23) - cc) * d2;
}

template <int WT, int S>
__device__ inline half8_t gb_operand(const GBRaw<WT> &r, int h) {
    if constexpr (WT == 1) {
        return __builtin_bit_cast(half8_t, r.v[S]);
    } else {
        const auto &w = S < 2 ? r.w0 : r.w1;
        const uint32_t mis = S < 2 ? r.mis0 : r.mis1;
        const _Float16 dh = (_Float16)b32_d(w[0], mis);
        const half2_t d2 = {dh, dh};
        // values v0 .. v0 + 7 of the block, v0 = 16 (S & 1) + 8 h: groups of 4
        // i0 = 4 (S & 1) + 2 h and i0 + 1
        constexpr int J = 4 * (S & 1);
        uint32_t c0 = h ? b32_codes4<WT, J + 2>(w, mis) : b32_codes4<WT, J>(w, mis);
        uint32_t c1 = h ? b32_codes4<WT, J + 3>(w, mis) : b32_codes4<WT, J + 1>(w, mis);
        float off;
        if constexpr (WT == 8) {
            c0 ^= 0x80808080u;   // signed -> q + 128
            c1 ^= 0x80808080u;
            off = 128.0f;
        } else {
            off = WT == 2 ? 8.0f : 16.0f;
        }
        half2_t a0, a1, a2, a3;
        gb_bytes_h(c0, off, d2, a0, a1);
        gb_bytes_h(c1, off, d2, a2, a3);
        const u32x4 o = {__builtin_bit_cast(uint32_t, a0), __builtin_bit_cast(uint32_t, a1),
                         __builtin_bit_cast(uint32_t, a2), __builtin_bit_cast(uint32_t, a3)};
        return __builtin_bit_cast(half8_t, o);
    }
}

template <int WT, bool GLU>
__global__ void __launch_bounds__(256) k_gemm_b32(B32Args g) {
    __shared__ __attribute__((aligned(16))) _Float16 As[2][GB_BM * GB_BK];   // 2 x 24 KB
    __shared__ int s_row[GB_BM];   // activation row of each tile row
    __shared__ int s_p[GB_BM];     // output row (slot index) of each tile row, -1 past the tile
    const int tile = blockIdx.y;
    if (tile >= *g.n_tiles) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
    const int e = g.tile_e[tile], start = g.tile_start[tile], mrows = g.tile_rows[tile];
    const int nrt = (mrows + 31) >> 5;
    // this lane's weight row and output column
    int64_t col;
    const ExpertMat *M = &g.a;
    int64_t wrow;
    if (GLU) {
        col = (int64_t)blockIdx.x * 64 + 32 * (wave & 1) + l32;
        wrow = col;
        if (wave >= 2) {
            if (g.fused) wrow = g.I + col;
            else M = &g.b;
        }
    } else {
        col = (int64_t)blockIdx.x * 128 + 32 * wave + l32;
        wrow = col;
    }
    const bool col_ok = col < g.ncols;
    if (!col_ok) wrow = 0;   // a valid row; its results are not stored
    const uint8_t *row = M->data + (int64_t)e * M->mat_bytes + wrow * M->row_bytes;
    const int64_t Kin = M->K;
    if (tid < GB_BM) {
        const int p = tid < mrows ? g.perm[start + tid] : -1;
        s_p[tid] = p;
        s_row[tid] = p < 0 ? 0 : (g.ne11 == 1 ? p / g.K : p);
    }
    __syncthreads();

    // activation chunks of this thread: chunk q = tid + 256 i -> tile row q / 8, K chunk q % 8
    uint4 areg[GB_ACH];
    auto load_a = [&](int64_t k0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < GB_ACH; ++i) {
            const int q = tid + 256 * i, r = q >> 3, c = q & 7;
            const int64_t k = k0 + 8 * c;
            areg[i] = (r < 32 * nrt && k < Kin) ? *(const uint4 *)(g.xh + (int64_t)s_row[r] * Kin + k)
                                               : make_uint4(0, 0, 0, 0);
        }
    };
    auto store_a = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < GB_ACH; ++i) {
            const int q = tid + 256 * i, r = q >> 3, c = q & 7;
            *(uint4 *)(&As[buf][(r * 8 + (c ^ (r & 7))) * 8]) = areg[i];
        }
    };

    f32x16 acc[GB_RT];
#pragma unroll
    for (int t = 0; t < GB_RT; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[t][i] = 0.f;

    const int nk = (int)((Kin + GB_BK - 1) / GB_BK);
    GBRaw<WT> cur, nxt;
    load_a(0);
    gb_load<WT>(row, 0, Kin, h, cur);
    store_a(0);
    __syncthreads();
    for (int kb = 0; kb < nk; ++kb) {
        const bool more = kb + 1 < nk;
        if (more) {
            load_a((int64_t)(kb + 1) * GB_BK);
            gb_load<WT>(row, (int64_t)(kb + 1) * GB_BK, Kin, h, nxt);
        }
        const _Float16 *A = As[kb & 1];
        auto step = [&](const half8_t bop, int s) __attribute__((always_inline)) {
            const int c = 2 * s + h;
#pragma unroll
            for (int t = 0; t < GB_RT; ++t) {
                if (t < nrt) {
                    const int r = 32 * t + l32;
                    const half8_t aop = *(const half8_t *)(&A[(r * 8 + (c ^ (r & 7))) * 8]);
                    acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(aop, bop, acc[t], 0, 0, 0);
                }
            }
        };
        step(gb_operand<WT, 0>(cur, h), 0);
        step(gb_operand<WT, 1>(cur, h), 1);
        step(gb_operand<WT, 2>(cur, h), 2);
        step(gb_operand<WT, 3>(cur, h), 3);
        if (more) {
            store_a((kb + 1) & 1);
            cur = nxt;
        }
        __syncthreads();
    }

    // rows 32 t + 8 (i / 4) + 4 h + i % 4, column col
    if (GLU) {
        float *G = (float *)&As[0][0];   // [GB_BM][64] up-product values (48 KB)
        const int cc = 32 * (wave & 1) + l32;
        if (wave >= 2) {
#pragma unroll
            for (int t = 0; t < GB_RT; ++t)
                if (t < nrt)
#pragma unroll
                    for (int i = 0; i < 16; ++i) G[(32 * t + 8 * (i >> 2) + 4 * h + (i & 3)) * 64 + cc] = acc[t][i];
        }
        __syncthreads();
        if (wave < 2 && col_ok) {
#pragma unroll
            for (int t = 0; t < GB_RT; ++t)
                if (t < nrt)
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int m = 32 * t + 8 * (i >> 2) + 4 * h + (i & 3);
                        if (m < mrows) g.y[(int64_t)s_p[m] * g.ldy + col] = act_pair(g.act, acc[t][i], G[m * 64 + cc]);
                    }
        }
    } else if (col_ok) {
#pragma unroll
        for (int t = 0; t < GB_RT; ++t)
            if (t < nrt)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int m = 32 * t + 8 * (i >> 2) + 4 * h + (i & 3);
                    if (m < mrows) g.y[(int64_t)s_p[m] * g.ldy + col] = acc[t][i];
                }
    }
}

// ------------------------------------------------------------------ launch
template <template <int> class KF>
static int b32_dispatch_type(int type, dim3 grid, const B32Args &g, hipStream_t st);

int launch_gemv_b32(const B32Args &g, hipStream_t st) {
    if (g.max_active <= 0) return 0;
    if (g.a.K % 32) return -6;
    const int64_t per_block = (g.glu ? 4 : 8) * 4;
    const dim3 grid((unsigned)((g.ncols + per_block - 1) / per_block), (unsigned)g.max_active);
    switch (g.a.type) {
    case 1: hipLaunchKernelGGL(k_gemv_b32<1>, grid, dim3(256), 0, st, g); break;
    case 2: hipLaunchKernelGGL(k_gemv_b32<2>, grid, dim3(256), 0, st, g); break;
    case 6: hipLaunchKernelGGL(k_gemv_b32<6>, grid, dim3(256), 0, st, g); break;
    case 8: hipLaunchKernelGGL(k_gemv_b32<8>, grid, dim3(256), 0, st, g); break;
    default: return -3;
    }
    return hip_check_launch();
}

int launch_gemm_b32(const B32Args &g, hipStream_t st) {
    if (g.max_tiles <= 0) return 0;
    if (g.a.K % 32) return -6;
    const dim3 grid((unsigned)(g.glu ? (g.ncols + 63) / 64 : (g.ncols + 127) / 128), (unsigned)g.max_tiles);
#define GB_LAUNCH(T)                                                                                    \
    if (g.glu) hipLaunchKernelGGL((k_gemm_b32<T, true>), grid, dim3(256), 0, st, g);                   \
    else hipLaunchKernelGGL((k_gemm_b32<T, false>), grid, dim3(256), 0, st, g);
    switch (g.a.type) {
    case 1: GB_LAUNCH(1) break;
    case 2: GB_LAUNCH(2) break;
    case 6: GB_LAUNCH(6) break;
    case 8: GB_LAUNCH(8) break;
    default: return -3;
    }
#undef GB_LAUNCH
    return hip_check_launch();
}

}  // namespace mimoe
