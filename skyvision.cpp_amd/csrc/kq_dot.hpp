// kq_dot.hpp - one lane's 32-value piece of a Q4_K / Q6_K super-block
// against a Q8_K activation block: the integer form of ggml's
// ggml_vec_dot_q4_K_q8_K / ggml_vec_dot_q6_K_q8_K, split so that 8 lanes cover
// a block (the grouped GEMV and the batched decode kernel).
#pragma once

#include "common.hpp"

namespace mimoe {

// 8 bytes from a 2-byte-aligned address (Q6_K blocks are 210 bytes), reading
// only the aligned dwords that intersect [p, p + 8).
__device__ inline uint2 load8_a2(const uint8_t *p) {
    const uintptr_t a = (uintptr_t)p;
    const uint32_t mis = (uint32_t)(a & 3u);
    const uint32_t *w = (const uint32_t *)(a - mis);
    const uint32_t w0 = w[0], w1 = w[1];
    const uint32_t w2 = mis ? w[2] : 0u;
    uint2 r;
    r.x = __builtin_amdgcn_alignbyte(w1, w0, mis);
    r.y = __builtin_amdgcn_alignbyte(w2, w1, mis);
    return r;
}

struct Q4Piece {      // one lane's 32 values of a Q4_K super-block
    uint32_t qs[4];
    float d, dmin;
    int scA, mA, scB, mB;
};

__device__ inline void load_q4_piece(const uint8_t *blk, int sl, Q4Piece &w) {
    const uint4 h = *(const uint4 *)blk;   // d, dmin, scales[12]
    const uint4 q = *(const uint4 *)(blk + 16 + 16 * sl);
    w.qs[0] = q.x; w.qs[1] = q.y; w.qs[2] = q.z; w.qs[3] = q.w;
    w.d = h2f((uint16_t)(h.x & 0xffff));
    w.dmin = h2f((uint16_t)(h.x >> 16));
    const int c = sl >> 1;
    scale_min_k4_reg(2 * c, h.y, h.z, h.w, w.scA, w.mA);
    scale_min_k4_reg(2 * c + 1, h.y, h.z, h.w, w.scB, w.mB);
}

// lane piece: chunk c = sl/2, l0 = 16*(sl%2); low nibbles = elements 64c+l0+i
// (sub-block 2c), high nibbles = 64c+32+l0+i (sub-block 2c+1), i < 16.
__device__ inline float dot_q4_piece(const Q4Piece &w, int sl, const int8_t *q8blk, float dx,
                                     const int16_t *bsblk) {
    const int c = sl >> 1, l0 = 16 * (sl & 1);
    const uint4 xa = *(const uint4 *)(q8blk + 64 * c + l0);
    const uint4 xb = *(const uint4 *)(q8blk + 64 * c + 32 + l0);
    const uint32_t xav[4] = {xa.x, xa.y, xa.z, xa.w};
    const uint32_t xbv[4] = {xb.x, xb.y, xb.z, xb.w};
    int sa = 0, sb = 0;
    for (int i = 0; i < 4; ++i) {
        sa = __builtin_amdgcn_sdot4((int)(w.qs[i] & 0x0F0F0F0Fu), (int)xav[i], sa, false);
        sb = __builtin_amdgcn_sdot4((int)((w.qs[i] >> 4) & 0x0F0F0F0Fu), (int)xbv[i], sb, false);
    }
    const int bsa = bsblk[4 * c + (sl & 1)];
    const int bsb = bsblk[4 * c + 2 + (sl & 1)];
    const int isum = w.scA * sa + w.scB * sb;
    const int msum = w.mA * bsa + w.mB * bsb;
    return (w.d * dx) * (float)isum - (w.dmin * dx) * (float)msum;
}

struct Q6Piece {      // one lane's 32 values of a Q6_K super-block
    uint2 qla, qlb, qh;
    float d;
    int sc[4];
};

// lane piece: half h = sl/4, l0 = 8*(sl%4); quarters qq = 0..3 are elements
// 128h + 32qq + l0 + i, i < 8, with scale sc[8h + l0/16 + 2qq].
__device__ inline void load_q6_piece(const uint8_t *blk, int sl, Q6Piece &w) {
    const int h = sl >> 2, l0 = 8 * (sl & 3);
    w.qla = load8_a2(blk + 64 * h + l0);
    w.qlb = load8_a2(blk + 64 * h + 32 + l0);
    w.qh = load8_a2(blk + 128 + 32 * h + l0);
    const uint2 s8 = load8_a2(blk + 192 + 8 * h);
    const int is = l0 >> 4;
    for (int qq = 0; qq < 4; ++qq) {
        const int idx = is + 2 * qq;
        const uint32_t word = (idx >> 2) ? s8.y : s8.x;
        w.sc[qq] = (int)(int8_t)(word >> (8 * (idx & 3)));
    }
    const uint8_t *pd = blk + 208;
    w.d = h2f((uint16_t)((uint32_t)pd[0] | ((uint32_t)pd[1] << 8)));
}

__device__ inline float dot_q6_piece(const Q6Piece &w, int sl, const int8_t *q8blk, float dx) {
    const int h = sl >> 2, l0 = 8 * (sl & 3);
    const uint32_t la[2] = {w.qla.x, w.qla.y}, lb[2] = {w.qlb.x, w.qlb.y}, hh[2] = {w.qh.x, w.qh.y};
    int isum = 0;
    for (int qq = 0; qq < 4; ++qq) {
        const uint2 xq = *(const uint2 *)(q8blk + 128 * h + 32 * qq + l0);
        const uint32_t xv[2] = {xq.x, xq.y};
        int s = 0;
        for (int i = 0; i < 2; ++i) {
            uint32_t lo, hi2;
            if (qq == 0) { lo = la[i] & 0x0F0F0F0Fu; hi2 = (hh[i] << 4) & 0x30303030u; }
            else if (qq == 1) { lo = lb[i] & 0x0F0F0F0Fu; hi2 = (hh[i] << 2) & 0x30303030u; }
            else if (qq == 2) { lo = (la[i] >> 4) & 0x0F0F0F0Fu; hi2 = hh[i] & 0x30303030u; }
            else { lo = (lb[i] >> 4) & 0x0F0F0F0Fu; hi2 = (hh[i] >> 2) & 0x30303030u; }
            // bytes q in 0..63 -> q - 32 as signed bytes: q ^ 0x20 is the 6-bit
            // two's complement of q - 32; copy bit 5 into bits 6-7 (per byte,
            // 0x20 * 6 = 0xC0, so nothing carries across bytes)
            const uint32_t x6 = (lo | hi2) ^ 0x20202020u;
            const uint32_t sq = x6 | ((x6 & 0x20202020u) * 6u);
            s = __builtin_amdgcn_sdot4((int)sq, (int)xv[i], s, false);
        }
        isum += w.sc[qq] * s;
    }
    return (w.d * dx) * (float)isum;
}

}  // namespace mimoe
