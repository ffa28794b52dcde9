// k_gemm.hip - grouped k-quant GEMM on fp16 MFMA for prefill.
//
// One work-group computes a 64-row tile of one expert's token list (rows are
// the dispatched (token, slot) pairs, gathered through the permutation) against
// 256 GLU columns (gate/up: 256 h rows + 256 g rows) or 512 output columns
// (down).  Weights stream from the GGUF Q4_K / Q6_K blocks straight into
// registers and are dequantized in-register to fp16 (packed fp16 math on
// exact small-integer codes); activations are Q8_K-quantized rows stored as
// fp16(d * q) in the MFMA K order of the weight type, staged through LDS.
// v_mfma_f32_16x16x32_f16 accumulates in fp32.
//
// GLU epilogue: act(h, g) per (row, column), then the row's 256 columns are
// quantized to Q8_K (ggml: the down mul_mat_id quantizes its F32 input) and
// written as fp16 in the K order of the down weights, so the down GEMM reads
// it directly.
#include "act.hpp"
#include "common.hpp"
#include "launch.hpp"

namespace mimoe {

constexpr int GM_BM = 64;
constexpr int GM_WAVES = 8;
constexpr int GM_THREADS = GM_WAVES * 64;
constexpr int GM_LDA = QK + 8;   // halfs per LDS row (pad: 528 B rows spread LDS banks)

__device__ inline half2_t u2h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ inline uint32_t h22u(half2_t h) { return __builtin_bit_cast(uint32_t, h); }
__device__ inline half2_t splat(float f) {
    const _Float16 h = (_Float16)f;
    half2_t r = {h, h};
    return r;
}

// 16 bytes from a 2-byte-aligned address, touching only the dwords that
// intersect [p, p + 16)
__device__ inline uint4 load16_a2(const uint8_t *p) {
    const uintptr_t a = (uintptr_t)p;
    const uint32_t mis = (uint32_t)(a & 3u);
    const uint32_t *w = (const uint32_t *)(a - mis);
    const uint32_t w0 = w[0], w1 = w[1], w2 = w[2], w3 = w[3];
    const uint32_t w4 = mis ? w[4] : 0u;
    uint4 r;
    r.x = __builtin_amdgcn_alignbyte(w1, w0, mis);
    r.y = __builtin_amdgcn_alignbyte(w2, w1, mis);
    r.z = __builtin_amdgcn_alignbyte(w3, w2, mis);
    r.w = __builtin_amdgcn_alignbyte(w4, w3, mis);
    return r;
}

// Q4_K: dword v holds nibbles n0..n7 = (a0,b0,a1,b1,a2,b2,a3,b3), a = sub-block
// 2g (elements 64g+4s+i), b = sub-block 2g+1 (64g+32+4s+i).  Output operand
// order (a0,a2,b0,b2,a1,a3,b1,b3).  Codes become exact fp16 integers q - 8
// through the 1024 (bits 0-3) and 64 (bits 4-7) exponent tricks; one packed
// fma per pair applies s = d*sc and c = 8 d*sc - dmin*m (q4k_center):
// w = (q - 8) s + c.  Centring the codes halves the weight of s's rounding
// and leaves c small, so w lands close to the fp16 rounding of the exact
// d*sc*q - dmin*m.
__device__ inline half8_t dq_q4k(uint32_t v, half2_t sA, half2_t nmA, half2_t sB, half2_t nmB) {
    const half2_t c1032 = {(_Float16)1032.f, (_Float16)1032.f};
    const half2_t c72 = {(_Float16)72.f, (_Float16)72.f};
    const uint32_t v8 = v >> 8;
    const half2_t t0 = u2h2((v & 0x000F000Fu) | 0x64006400u) - c1032;
    const half2_t t1 = u2h2((v & 0x00F000F0u) | 0x54005400u) - c72;
    const half2_t t2 = u2h2((v8 & 0x000F000Fu) | 0x64006400u) - c1032;
    const half2_t t3 = u2h2((v8 & 0x00F000F0u) | 0x54005400u) - c72;
    const half2_t w0 = __builtin_elementwise_fma(t0, sA, nmA);
    const half2_t w1 = __builtin_elementwise_fma(t1, sB, nmB);
    const half2_t w2 = __builtin_elementwise_fma(t2, sA, nmA);
    const half2_t w3 = __builtin_elementwise_fma(t3, sB, nmB);
    const u32x4 r = {h22u(w0), h22u(w1), h22u(w2), h22u(w3)};
    return __builtin_bit_cast(half8_t, r);
}

// 4 bytes of 6-bit codes -> two half2 of (q - 32) * s
__device__ inline void q6_bytes_to_h2(uint32_t x, half2_t s, half2_t &lo, half2_t &hi) {
    const half2_t c1056 = {(_Float16)1056.f, (_Float16)1056.f};
    const uint32_t p01 = (x & 0x000000FFu) | ((x << 8) & 0x00FF0000u) | 0x64006400u;
    const uint32_t p23 = ((x >> 16) & 0x000000FFu) | ((x >> 8) & 0x00FF0000u) | 0x64006400u;
    lo = (u2h2(p01) - c1056) * s;
    hi = (u2h2(p23) - c1056) * s;
}

// Q6_K step s = 2*jj + w: dword jj of the lane's ql/qh vectors; w = 0 gives
// quarters q1 (p 0..3) and q2 (p 4..7), w = 1 gives q3 and q4.
__device__ inline half8_t dq_q6k(uint32_t qla, uint32_t qlb, uint32_t qh, int w, half2_t s_first,
                                 half2_t s_second) {
    uint32_t qa, qb;
    if (w == 0) {
        qa = (qla & 0x0F0F0F0Fu) | ((qh << 4) & 0x30303030u);
        qb = (qlb & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u);
    } else {
        qa = ((qla >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u);
        qb = ((qlb >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u);
    }
    half2_t a01, a23, b01, b23;
    q6_bytes_to_h2(qa, s_first, a01, a23);
    q6_bytes_to_h2(qb, s_second, b01, b23);
    const u32x4 r = {h22u(a01), h22u(a23), h22u(b01), h22u(b23)};
    return __builtin_bit_cast(half8_t, r);
}

// K position of element e inside a 256 block (inverse of q4k_elem / q6k_elem)
__device__ inline int mfma_pos(int wtype, int e) {
    if (wtype == 14) {
        const int h = e >> 7, r = e & 127, qq = r >> 5, l = r & 31;
        const int g = 2 * h + (l >> 4), jj = (l & 15) >> 2, i = l & 3;
        const int s = 2 * jj + (qq >> 1), p = 4 * (qq & 1) + i;
        return 32 * s + 8 * g + p;
    }
    const int g = e >> 6, r = e & 63, hi = r >> 5, r2 = r & 31, s = r2 >> 2, lo = r2 & 3;
    const int p = (lo & 1) * 4 + hi * 2 + (lo >> 1);
    return 32 * s + 8 * g + p;
}

struct WRegsQ4 {
    uint32_t qs[8];
    half2_t sA, nmA, sB, nmB;
};
struct WRegsQ6 {
    uint32_t qla[4], qlb[4], qh[4];
    half2_t sq[4];
};

template <int WT, bool GLU, int NEXT>
__global__ void __launch_bounds__(GM_THREADS) k_gemm(GemmArgs g) {
    __shared__ __attribute__((aligned(16))) _Float16 As[GM_BM * GM_LDA];
    __shared__ int s_p[GM_BM];
    __shared__ int64_t s_arow[GM_BM];
    __shared__ AmaxIdx s_red[GM_BM][GM_WAVES];
    __shared__ float s_is[GM_BM], s_d[GM_BM];

    const int tile = blockIdx.y;
    if (tile >= *g.n_tiles) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int l16 = lane & 15, g4 = lane >> 4;
    const int e = g.tile_e[tile], r0 = g.tile_r0[tile];
    const int cnt = g.counts[e], off = g.offsets[e];
    const int mrows = imin(GM_BM, cnt - r0);
    const int64_t Kin = g.a.K;
    const int nb = (int)(Kin / QK);

    if (tid < GM_BM) {
        const int p = tid < mrows ? g.perm[off + r0 + tid] : -1;
        s_p[tid] = p;
        s_arow[tid] = p < 0 ? 0 : (g.ne11 == 1 ? (int64_t)(p / g.K) : (int64_t)p);
    }

    // weight rows of this lane's four 16-row subtiles
    const uint8_t *rowp[4];
    int64_t ncol[4];
    bool nok[4];
    for (int nt = 0; nt < 4; ++nt) {
        int64_t n;
        const ExpertMat *M = &g.a;
        int64_t wrow;
        if (GLU) {
            n = (int64_t)blockIdx.x * 256 + 32 * wave + 16 * (nt & 1) + l16;
            wrow = n;
            if (nt >= 2) {
                if (g.fused) wrow = g.I + n;
                else M = &g.b;
            }
        } else {
            n = (int64_t)blockIdx.x * 512 + 64 * wave + 16 * nt + l16;
            wrow = n;
        }
        ncol[nt] = n;
        nok[nt] = n < g.ncols;
        if (!nok[nt]) wrow = 0;
        rowp[nt] = M->data + (int64_t)e * M->mat_bytes + wrow * M->row_bytes;
    }

    float4_t acc[4][4];
    for (int mt = 0; mt < 4; ++mt)
        for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = (float4_t){0.f, 0.f, 0.f, 0.f};
    __syncthreads();

    for (int b = 0; b < nb; ++b) {
        // activation tile: 64 rows x 512 B
        uint4 av[4];
        for (int it = 0; it < 4; ++it) {
            const int idx = tid + GM_THREADS * it;
            const int r = idx >> 5, c16 = idx & 31;
            av[it] = *(const uint4 *)(g.xh + s_arow[r] * Kin + (int64_t)b * QK + c16 * 8);
        }
        // weights of block b
        WRegsQ4 w4[WT == 12 ? 4 : 1];
        WRegsQ6 w6[WT == 14 ? 4 : 1];
        for (int nt = 0; nt < 4; ++nt) {
            if constexpr (WT == 12) {
                const uint8_t *blk = rowp[nt] + (int64_t)b * Q4K_BYTES;
                const uint4 h = *(const uint4 *)blk;
                const uint4 q0 = *(const uint4 *)(blk + 16 + 32 * g4);
                const uint4 q1 = *(const uint4 *)(blk + 16 + 32 * g4 + 16);
                w4[nt].qs[0] = q0.x; w4[nt].qs[1] = q0.y; w4[nt].qs[2] = q0.z; w4[nt].qs[3] = q0.w;
                w4[nt].qs[4] = q1.x; w4[nt].qs[5] = q1.y; w4[nt].qs[6] = q1.z; w4[nt].qs[7] = q1.w;
                const float d = h2f((uint16_t)(h.x & 0xffff)), dmin = h2f((uint16_t)(h.x >> 16));
                int scA, mA, scB, mB;
                scale_min_k4_reg(2 * g4, h.y, h.z, h.w, scA, mA);
                scale_min_k4_reg(2 * g4 + 1, h.y, h.z, h.w, scB, mB);
                w4[nt].sA = splat(d * (float)scA);
                w4[nt].nmA = splat(q4k_center(d, scA, dmin, mA));
                w4[nt].sB = splat(d * (float)scB);
                w4[nt].nmB = splat(q4k_center(d, scB, dmin, mB));
            } else {
                const uint8_t *blk = rowp[nt] + (int64_t)b * Q6K_BYTES;
                const int h = g4 >> 1, lo16 = 16 * (g4 & 1);
                const uint4 a = load16_a2(blk + 64 * h + lo16);
                const uint4 bq = load16_a2(blk + 64 * h + 32 + lo16);
                const uint4 hq = load16_a2(blk + 128 + 32 * h + lo16);
                w6[nt].qla[0] = a.x; w6[nt].qla[1] = a.y; w6[nt].qla[2] = a.z; w6[nt].qla[3] = a.w;
                w6[nt].qlb[0] = bq.x; w6[nt].qlb[1] = bq.y; w6[nt].qlb[2] = bq.z; w6[nt].qlb[3] = bq.w;
                w6[nt].qh[0] = hq.x; w6[nt].qh[1] = hq.y; w6[nt].qh[2] = hq.z; w6[nt].qh[3] = hq.w;
                const uint4 s16 = load16_a2(blk + 192);
                const uint32_t sv[4] = {s16.x, s16.y, s16.z, s16.w};
                const uint8_t *pd = blk + 208;
                const float d = h2f((uint16_t)((uint32_t)pd[0] | ((uint32_t)pd[1] << 8)));
                for (int qq = 0; qq < 4; ++qq) {
                    const int idx = 8 * h + (g4 & 1) + 2 * qq;
                    const int sc = (int)(int8_t)(sv[idx >> 2] >> (8 * (idx & 3)));
                    w6[nt].sq[qq] = splat(d * (float)sc);
                }
            }
        }
        for (int it = 0; it < 4; ++it) {
            const int idx = tid + GM_THREADS * it;
            const int r = idx >> 5, c16 = idx & 31;
            *(uint4 *)(As + r * GM_LDA + c16 * 8) = av[it];
        }
        __syncthreads();

#pragma unroll
        for (int s = 0; s < 8; ++s) {
            half8_t A[4];
            for (int mt = 0; mt < 4; ++mt)
                A[mt] = *(const half8_t *)(As + (16 * mt + l16) * GM_LDA + 32 * s + 8 * g4);
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) {
                half8_t B;
                if constexpr (WT == 12) {
                    B = dq_q4k(w4[nt].qs[s], w4[nt].sA, w4[nt].nmA, w4[nt].sB, w4[nt].nmB);
                } else {
                    const int jj = s >> 1, wsel = s & 1;
                    B = dq_q6k(w6[nt].qla[jj], w6[nt].qlb[jj], w6[nt].qh[jj], wsel, w6[nt].sq[2 * wsel],
                               w6[nt].sq[2 * wsel + 1]);
                }
                for (int mt = 0; mt < 4; ++mt)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[mt], B, acc[mt][nt], 0, 0, 0);
            }
        }
        __syncthreads();
    }

    if constexpr (!GLU) {
        // rows m = 16mt + 4*g4 + i, column ncol[nt]
        for (int mt = 0; mt < 4; ++mt)
            for (int i = 0; i < 4; ++i) {
                const int m = 16 * mt + 4 * g4 + i;
                if (m >= mrows) continue;
                float *yrow = g.y + (int64_t)s_p[m] * g.ldy;
                for (int nt = 0; nt < 4; ++nt)
                    if (nok[nt]) yrow[ncol[nt]] = acc[mt][nt][i];
            }
    } else {
        // act for columns c = 32*wave + 16*j + l16 (j = 0, 1) of this 256 tile
        float v[4][2][4];
        for (int mt = 0; mt < 4; ++mt)
            for (int j = 0; j < 2; ++j)
                for (int i = 0; i < 4; ++i) v[mt][j][i] = act_pair(g.act, acc[mt][j][i], acc[mt][2 + j][i]);
        // Q8_K over each row's 256 columns: first column with the largest |v|
        for (int mt = 0; mt < 4; ++mt)
            for (int i = 0; i < 4; ++i) {
                AmaxIdx a{-1.f, 1 << 30, 0.f};
                for (int j = 0; j < 2; ++j) {
                    AmaxIdx c{fabsf(v[mt][j][i]), 32 * wave + 16 * j + l16, v[mt][j][i]};
                    a = amax_better(a, c);
                }
                a = wave_amax_idx(a, 16);
                if (l16 == 0) s_red[16 * mt + 4 * g4 + i][wave] = a;
            }
        __syncthreads();
        if (tid < GM_BM) {
            AmaxIdx a = s_red[tid][0];
            for (int w = 1; w < GM_WAVES; ++w) a = amax_better(a, s_red[tid][w]);
            if (a.ax != 0.f) {
                const float iscale = -127.f / a.val;
                s_is[tid] = iscale;
                s_d[tid] = 1 / iscale;
                if (g.range_total && tid < mrows && f16_over(1 / iscale)) atomicAdd(g.range_total, 1);
            } else {
                s_is[tid] = 0.f;
                s_d[tid] = 0.f;
            }
        }
        __syncthreads();
        for (int mt = 0; mt < 4; ++mt)
            for (int i = 0; i < 4; ++i) {
                const int m = 16 * mt + 4 * g4 + i;
                const float is = s_is[m], d = s_d[m];
                for (int j = 0; j < 2; ++j) {
                    const int c = 32 * wave + 16 * j + l16;
                    const int q = d != 0.f ? imin(127, nearest_int(is * v[mt][j][i])) : 0;
                    As[m * GM_LDA + mfma_pos(NEXT, c)] = f16_sat(d * (float)q);
                }
            }
        __syncthreads();
        for (int it = 0; it < 4; ++it) {
            const int idx = tid + GM_THREADS * it;
            const int r = idx >> 5, c16 = idx & 31;
            if (r < mrows)
                *(uint4 *)(g.acth + (int64_t)s_p[r] * g.I + (int64_t)blockIdx.x * QK + c16 * 8) =
                    *(const uint4 *)(As + r * GM_LDA + c16 * 8);
        }
    }
}

int launch_gemm(const GemmArgs &g, hipStream_t st) {
    if (g.max_tiles <= 0) return 0;
    if (g.a.K % QK) return -6;
    const bool glu = g.epi == EPI_GLU;
    if (glu && (g.I % QK)) return -6;
    const unsigned gx = glu ? (unsigned)(g.I / QK) : (unsigned)((g.ncols + 511) / 512);
    const dim3 grid(gx, (unsigned)g.max_tiles);
    const dim3 block(GM_THREADS);
    if (g.a.type == 12) {
        if (!glu) hipLaunchKernelGGL((k_gemm<12, false, 12>), grid, block, 0, st, g);
        else if (g.next_type == 14) hipLaunchKernelGGL((k_gemm<12, true, 14>), grid, block, 0, st, g);
        else hipLaunchKernelGGL((k_gemm<12, true, 12>), grid, block, 0, st, g);
    } else if (g.a.type == 14) {
        if (!glu) hipLaunchKernelGGL((k_gemm<14, false, 12>), grid, block, 0, st, g);
        else if (g.next_type == 14) hipLaunchKernelGGL((k_gemm<14, true, 14>), grid, block, 0, st, g);
        else hipLaunchKernelGGL((k_gemm<14, true, 12>), grid, block, 0, st, g);
    } else {
        return -3;
    }
    return hip_check_launch();
}

}  // namespace mimoe
