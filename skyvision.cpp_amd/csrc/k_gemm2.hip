// k_gemm2.hip - grouped k-quant GEMM on v_mfma_f32_32x32x16_f16 (prefill).
//
// A work-group owns a 64-row tile of one expert's dispatched rows (tokens
// gathered through the permutation) and 8 waves; each wave owns 64 rows x 64
// weight rows as 2 x 2 MFMA tiles of 32 x 32.  Activation tiles are staged in
// LDS, double buffered; weights stream straight from the GGUF blocks into
// registers (the next super-block's bytes are fetched while the current one
// is consumed) and are expanded in-register with packed fp16 math.
//
// Gate/up (GLU) on Q4_K is computed exactly like ggml-cpu's Q4_K x Q8_K dot
// (ggml_vec_dot_q4_K_q8_K): the MFMA operands are exact small integers - the
// activation codes q8 and sc_j * q4 (<= 63 * 15) - so the fp32 accumulator holds
// the integer sum  P = sum_j sc_j sum_i q4 q8  of each 256-value super-block,
// and a second MFMA gives the min term  Q = sum_j m_j bsum_j  from the Q8_K
// block sums.  Per super-block the fp32 epilogue adds
//     d_x * (d_w * P - dmin_w * Q)
// which is the ggml formula up to fp32 summation order.  The GLU output is then
// quantized to Q8_K per 256 columns (ggml: the down mul_mat_id quantizes its
// F32 input) and stored as fp16(d * q) in the down weight's K order.
//
// Down (STORE) dequantizes Q4_K / Q6_K to fp16 in-register and multiplies the
// fp16 Q8_K activations, accumulating in fp32.
#include "act.hpp"
#include "common.hpp"
#include "launch.hpp"

namespace mimoe {

constexpr int G2_BM = 64;
constexpr int G2_WAVES = 8;
constexpr int G2_THREADS = G2_WAVES * 64;
constexpr int G2_LDA = QK + 8;          // halfs per LDS row: 528 B rows spread the LDS banks

typedef float float16_t __attribute__((ext_vector_type(16)));

__device__ inline half2_t u2h2_(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ inline uint32_t h22u_(half2_t h) { return __builtin_bit_cast(uint32_t, h); }
__device__ inline half2_t splat_(float f) {
    const _Float16 h = (_Float16)f;
    half2_t r = {h, h};
    return r;
}
__device__ inline uint32_t dword_of(const uint4 &v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

__device__ inline uint4 load16_a2_(const uint8_t *p) {
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

// exact integer operand: nibbles of dword v -> (a0,a2,b0,b2,a1,a3,b1,b3) * sc,
// a = low nibbles (sub-block lo), b = high nibbles (sub-block hi).
// fma((1024 + a), sc, -1024 sc) = a * sc exactly (<= 945 is an fp16 integer).
// v_and_or_b32 (src0 & src1) | src2 in one instruction; the compiler splits
// it in two when both constants are literals (gfx9 VOP3 takes no literal)
__device__ __forceinline__ uint32_t and_or_(uint32_t v, uint32_t mask, uint32_t orv) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(mask), "v"(orv));
    return r;
}
// 8 nibbles of one qs dword -> 8 exact fp16 values sc * q (pairs (n0,n4)
// (n1,n5) (n2,n6) (n3,n7); low nibbles scaled by sc_lo, high by sc_hi):
// 1024 + q via the 0x6400 exponent (64 + q via 0x5400 for bits 4-7), then
// fma(1024 + q, sc, -1024 sc) = q * sc exactly (|q sc| < 2048).
// m64 / m54 hold 0x64006400 / 0x54005400 in VGPRs.
__device__ inline half8_t dq4_exact(uint32_t v, half2_t sc_lo, half2_t nc_lo, half2_t sc_hi, half2_t nc_hi,
                                    uint32_t m64, uint32_t m54) {
    const uint32_t v8 = v >> 8;
    const half2_t t0 = u2h2_(and_or_(v, 0x000F000Fu, m64));
    const half2_t t1 = u2h2_(and_or_(v, 0x00F000F0u, m54));
    const half2_t t2 = u2h2_(and_or_(v8, 0x000F000Fu, m64));
    const half2_t t3 = u2h2_(and_or_(v8, 0x00F000F0u, m54));
    const u32x4 r = {h22u_(__builtin_elementwise_fma(t0, sc_lo, nc_lo)), h22u_(__builtin_elementwise_fma(t1, sc_hi, nc_hi)),
                     h22u_(__builtin_elementwise_fma(t2, sc_lo, nc_lo)), h22u_(__builtin_elementwise_fma(t3, sc_hi, nc_hi))};
    return __builtin_bit_cast(half8_t, r);
}

// fp16 weights: q exact, then one packed fma with s = d*sc, nm = -dmin*m
__device__ inline half8_t dq4_f16(uint32_t v, half2_t s_lo, half2_t nm_lo, half2_t s_hi, half2_t nm_hi) {
    const half2_t c1024 = {(_Float16)1024.f, (_Float16)1024.f};
    const half2_t c64 = {(_Float16)64.f, (_Float16)64.f};
    const uint32_t v8 = v >> 8;
    const half2_t t0 = u2h2_((v & 0x000F000Fu) | 0x64006400u) - c1024;
    const half2_t t1 = u2h2_((v & 0x00F000F0u) | 0x54005400u) - c64;
    const half2_t t2 = u2h2_((v8 & 0x000F000Fu) | 0x64006400u) - c1024;
    const half2_t t3 = u2h2_((v8 & 0x00F000F0u) | 0x54005400u) - c64;
    const u32x4 r = {h22u_(__builtin_elementwise_fma(t0, s_lo, nm_lo)), h22u_(__builtin_elementwise_fma(t1, s_hi, nm_hi)),
                     h22u_(__builtin_elementwise_fma(t2, s_lo, nm_lo)), h22u_(__builtin_elementwise_fma(t3, s_hi, nm_hi))};
    return __builtin_bit_cast(half8_t, r);
}

// 4 Q6_K values (6-bit codes q in the bytes of x) -> fp16 (q - 32) * s:
// v_perm_b32 puts each byte under the 0x64 exponent byte (1024 + q), then
// (1024 + q) - 1056 is exact and one rounding happens in the multiply
__device__ inline void q6b_to_h2(uint32_t x, half2_t s, half2_t &lo, half2_t &hi) {
    const half2_t c1056 = {(_Float16)1056.f, (_Float16)1056.f};
    const uint32_t p01 = __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u);
    const uint32_t p23 = __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u);
    lo = (u2h2_(p01) - c1056) * s;
    hi = (u2h2_(p23) - c1056) * s;
}
__device__ inline half8_t dq6_f16(uint32_t qla, uint32_t qlb, uint32_t qh, int w, half2_t s_first, half2_t s_second) {
    uint32_t qa, qb;
    if (w == 0) {
        qa = (qla & 0x0F0F0F0Fu) | ((qh << 4) & 0x30303030u);
        qb = (qlb & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u);
    } else {
        qa = ((qla >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u);
        qb = ((qlb >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u);
    }
    half2_t a01, a23, b01, b23;
    q6b_to_h2(qa, s_first, a01, a23);
    q6b_to_h2(qb, s_second, b01, b23);
    const u32x4 r = {h22u_(a01), h22u_(a23), h22u_(b01), h22u_(b23)};
    return __builtin_bit_cast(half8_t, r);
}

// XCD-aware tile order.  Work-groups are dealt to the 8 XCDs round robin, so
// the linear id is remapped XCD-major: each XCD walks a contiguous range of
// v = nt * max_tiles + mt, i.e. the M tiles of one expert's weight slab (same
// weights, consecutive in the tile list) run back to back on one XCD and
// re-read the slab from that XCD's L2.  The grid is a multiple of 8; padding
// blocks and tiles past n_tiles exit.
__device__ inline void tile_coords(int max_tiles, int &mt, int &nt) {
    const int lin = blockIdx.x;
    const int per = gridDim.x >> 3;
    const int v = (lin & 7) * per + (lin >> 3);   // a bijection on [0, gridDim.x)
    nt = v / max_tiles;
    mt = v - nt * max_tiles;
}

// ------------------------------------------------------------------ GLU
// 8 waves (2 per SIMD).  Wave w owns act columns 32w .. 32w+31 of the
// 256-column tile: col tile 0 holds their h (gate) rows, col tile 1 their g
// (up) rows; each wave covers all 64 token rows (row tiles 0, 1).
//
// Every operand reaches LDS by MUBUF loads that write LDS directly (lane i
// of a load writes the 16 bytes at +16i of a 1 KB span); no global load
// targets a register inside the K loop.
//  * activation codes (two stages): rows of 256 fp16 padded to 264 (528 B),
//    so an MFMA operand read of 32 rows at one K chunk touches 32 distinct
//    bank groups at the lane's row base plus a constant.  The 64 padded rows
//    are 33 KB = 33 loads; slot q = 64*k + lane of load k holds row q / 33,
//    chunk q % 33 (chunk 32 is the pad: it reloads chunk 0).  Block sums
//    (64 rows x 32 B) and row scales (64 x 4 B) ride in the same stage.
//  * weights (one stage per wave): the wave's 32 h rows and 32 g rows, each
//    row's whole 144-byte block (header + qs) at a 144-byte stride (a read
//    of 32 rows at one chunk is bank-conflict free), 32 rows = 4.5 KB padded
//    to 5 loads.  Rows are whole lines in global memory, so the loads are
//    coalesced.  The wave reads its block into registers right after the
//    block's barrier and only then loads the next block over it.
constexpr int G2G_WAVES = 8;
constexpr int G2G_THREADS = G2G_WAVES * 64;
constexpr int G2G_LDA = QK + 8;                       // padded row (halfs)
constexpr int G2G_ALOADS = G2_BM * (QK / 8 + 1) / 64; // 33
constexpr int G2G_LDV = QK + 4;                       // fp32 GLU row in the epilogue
constexpr int G2G_WGRP = 5 * 1024;                    // 32 rows x 144 B, padded
typedef __attribute__((address_space(3))) void lds_void_t;

// one stage of the activation double buffer; the two stages are separate
// LDS variables so the compiler can tell the loads into one from the reads
// of the other
struct G2GBuf {
    _Float16 As[G2_BM * G2G_LDA];        // 33 KB activation codes
    _Float16 Bs[G2_BM * 16];             // 2 KB block sums of 16 codes
    float Dx[G2_BM];                     // row scales
};

struct G2GLane {
    int wave, lane, l32, g2;
    __amdgpu_buffer_rsrc_t rx, rbs, rd, rw[2];   // xh, xbs, xd, weight matrices of col tiles 0 / 1
    uint32_t kin2;                               // activation row bytes
    uint32_t nb;                                 // K blocks
    uint32_t w0;                                 // byte offset of the wave's first weight row
    uint32_t rowb;                               // weight row bytes
    uint32_t wct;                                // col tile 1 offset when it shares col tile 0's matrix
    const int *arow;                             // LDS: activation row of each tile row
};

// buffer resource of a raw byte range (bounds-checked: reads past nbytes return 0)
__device__ inline __amdgpu_buffer_rsrc_t g2_rsrc(const void *p, int64_t nbytes) {
    const int n = nbytes > 0x7fffffff ? 0x7fffffff : (int)nbytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, n, 0x00020000);
}

// loads of block b: activation stage st (5 loads per wave, the 33rd issued
// by every wave with identical bytes; waves 0-1 block sums, wave 2 row
// scales) and the wave's weight region W (10 loads).  The per-lane offsets
// are recomputed here each block from the lane index and the tile's row
// table (a dozen registers less across the K loop); the opaque copy of the
// lane index keeps the compiler from hoisting them back out of the loop.
__device__ __forceinline__ void g2g_issue(const G2GLane &L, int b, G2GBuf &st, uint8_t *W) {
    int lane;
    asm volatile("v_mov_b32 %0, %1" : "=v"(lane) : "v"(L.lane));
#pragma unroll
    for (int j = 0; j < 5; ++j) {
        // slot q = 64k + lane of the padded activation tile: row q / 33, chunk q % 33
        const int k = j < 4 ? L.wave + 8 * j : G2G_ALOADS - 1;
        const int q = 64 * k + lane;
        const int row = q / 33, ch = q % 33;
        const uint32_t aoff = (uint32_t)L.arow[row] * L.kin2 + 16u * (uint32_t)(ch == 32 ? 0 : ch);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(L.rx, (lds_void_t *)&st.As[k * 512], 16, aoff, b * (QK * 2), 0, 0);
    }
    if (L.wave < 2) {
        const uint32_t bsoff = (uint32_t)L.arow[32 * L.wave + (lane >> 1)] * (L.nb * 32u) + 16u * (lane & 1);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(L.rbs, (lds_void_t *)&st.Bs[L.wave * 512], 16, bsoff, b * 32, 0, 0);
    } else if (L.wave == 2) {
        const uint32_t dxoff = (uint32_t)L.arow[lane] * (L.nb * 4u);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(L.rd, (lds_void_t *)&st.Dx[0], 4, dxoff, b * 4, 0, 0);
    }
    // weight load j of col tile ct: slot 64j + lane of the 32-row group =
    // row slot / 9, 16-byte chunk slot % 9 (slots past 32 rows x 9 chunks
    // reload the last chunk: identical bytes into the padding)
#pragma unroll
    for (int j = 0; j < 5; ++j) {
        const int slot = imin(64 * j + lane, 32 * 9 - 1);
        const int r = slot / 9, c = slot - 9 * r;
        const uint32_t woff = L.w0 + (uint32_t)r * L.rowb + 16u * (uint32_t)c;
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(L.rw[ct], (lds_void_t *)(W + ct * G2G_WGRP + j * 1024), 16,
                                                     woff + ct * L.wct, b * Q4K_BYTES, 0, 0);
    }
}

// one K block: wait for every load of block b, read this wave's weights
// into registers, start the loads of block b+1 (weights over the region just
// read, activations into stage nxt), accumulate block b
__device__ __forceinline__ void g2g_block(const G2Args &g, const G2GLane &L, int b, int nb, G2GBuf &cur,
                                          G2GBuf &nxt, uint8_t *W, float16_t (&acc)[2][2]) {
    const int l32 = L.l32, g2 = L.g2;
    // all of this wave's loads have landed (vmcnt(0)); after the barrier,
    // every wave's have.  A raw barrier: the asm memory clobber keeps the
    // compiler from moving LDS accesses across it.
    __builtin_amdgcn_s_waitcnt(0x0F70);
    asm volatile("s_barrier" ::: "memory");
    // weights of block b: header (chunk 0) and the lane's 64 qs bytes
    // (chunks 1 + 4*g2 .. 4 + 4*g2) of row (ct, l32)
    u32x4 hvs[2], qv[2][4];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
        const u32x4 *rw = (const u32x4 *)(W + ct * G2G_WGRP + l32 * Q4K_BYTES);
        hvs[ct] = rw[0];
#pragma unroll
        for (int q = 0; q < 4; ++q) qv[ct][q] = rw[1 + 4 * g2 + q];
    }
    // the weight loads of block b+1 overwrite the region: wait for the reads
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
    __builtin_amdgcn_sched_barrier(0);
    if (b + 1 < nb) g2g_issue(L, b + 1, nxt, W);
    __builtin_amdgcn_sched_barrier(0);
    // ---- per-block constants from the headers
    half2_t sc_lo[2][2], nc_lo[2][2], sc_hi[2][2], nc_hi[2][2];
    half8_t mins[2];
    float dw[2], dmw[2];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
        const u32x4 hv = hvs[ct];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int sc_, m_;
            scale_min_k4_reg(4 * g2 + j, hv.y, hv.z, hv.w, sc_, m_);
            mins[ct][2 * j] = (_Float16)(float)m_;
            mins[ct][2 * j + 1] = (_Float16)(float)m_;
        }
        dw[ct] = h2f((uint16_t)(hv.x & 0xffff));
        dmw[ct] = h2f((uint16_t)(hv.x >> 16));
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {   // steps 0-7: sub-blocks (4g2, 4g2+1); 8-15: (4g2+2, 4g2+3)
            int sc0, sc1, m_;
            scale_min_k4_reg(4 * g2 + 2 * hf, hv.y, hv.z, hv.w, sc0, m_);
            scale_min_k4_reg(4 * g2 + 2 * hf + 1, hv.y, hv.z, hv.w, sc1, m_);
            sc_lo[ct][hf] = splat_((float)sc0);
            nc_lo[ct][hf] = splat_(-1024.f * (float)sc0);
            sc_hi[ct][hf] = splat_((float)sc1);
            nc_hi[ct][hf] = splat_(-64.f * (float)sc1);
        }
    }
    // ---- main term: P = sum_j sc_j sum_i q4 q8, 16 MFMA steps of K = 16
    float16_t P[2][2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int i = 0; i < 16; ++i) P[rt][ct][i] = 0.f;
    const _Float16 *Ab = &cur.As[l32 * G2G_LDA + 8 * g2];
    const uint32_t m64 = 0x64006400u, m54 = 0x54005400u;
#pragma unroll
    for (int s = 0; s < 16; ++s) {
        const half8_t A0 = *(const half8_t *)(Ab + 16 * s);
        const half8_t A1 = *(const half8_t *)(Ab + 32 * G2G_LDA + 16 * s);
        const int hf = s >> 3;
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            const half8_t B = dq4_exact(qv[ct][s >> 2][s & 3], sc_lo[ct][hf], nc_lo[ct][hf], sc_hi[ct][hf],
                                        nc_hi[ct][hf], m64, m54);
            P[0][ct] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A0, B, P[0][ct], 0, 0, 0);
            P[1][ct] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A1, B, P[1][ct], 0, 0, 0);
        }
    }
    // ---- min term Q = sum_j m_j * bsum16_j (one MFMA per tile), then
    // acc += dx * (dw * P - dmin * Q); row scales of rows 32rt + 8a + 4g2 + {0..3}
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            const half8_t Abs = *(const half8_t *)(&cur.Bs[(32 * rt + l32) * 16 + 8 * g2]);
            float16_t q = {};
            q = __builtin_amdgcn_mfma_f32_32x32x16_f16(Abs, mins[ct], q, 0, 0, 0);
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const float4_t dxv = *(const float4_t *)(&cur.Dx[32 * rt + 8 * a + 4 * g2]);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float t = fmaf(-dmw[ct], q[4 * a + i], dw[ct] * P[rt][ct][4 * a + i]);
                    acc[rt][ct][4 * a + i] = fmaf(dxv[i], t, acc[rt][ct][4 * a + i]);
                }
            }
        }
    }
}

template <int ACT>
__device__ __forceinline__ void g2g_glu_rows(const float16_t (&acc)[2][2], float *V0, float *V1, int col, int g2) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int r = (8 * (i >> 2) + 4 * g2 + (i & 3)) * G2G_LDV + col;
        V0[r] = act_pair_fast<ACT>(acc[0][0][i], acc[0][1][i]);
        V1[r] = act_pair_fast<ACT>(acc[1][0][i], acc[1][1][i]);
    }
}

template <int NEXT>
__global__ void __launch_bounds__(G2G_THREADS) k_g2_glu(G2Args g) {
    __shared__ __attribute__((aligned(1024))) G2GBuf st0;
    __shared__ __attribute__((aligned(1024))) G2GBuf st1;
    __shared__ __attribute__((aligned(1024))) uint8_t s_w[G2G_WAVES][2 * G2G_WGRP];
    __shared__ int s_p[G2_BM], s_arow[G2_BM];
    const int nx = (int)(g.I / QK);
    int tile, ctile;
    tile_coords(g.max_tiles, tile, ctile);
    if (tile >= *g.n_tiles || ctile >= nx) return;
    G2GLane L;
    const int tid = threadIdx.x;
    L.wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: scalar branches
    L.lane = tid & 63;
    L.l32 = L.lane & 31;
    L.g2 = L.lane >> 5;
    const int wave = L.wave, lane = L.lane, l32 = L.l32, g2 = L.g2;
    const int e = g.tile_e[tile], r0 = g.tile_r0[tile];
    const int cnt = g.counts[e], off = g.offsets[e];
    const int mrows = imin(G2_BM, cnt - r0);
    const uint32_t Kin = (uint32_t)g.a.K;
    const int nb = (int)(Kin / QK);

    if (tid < G2_BM) {
        const int p = tid < mrows ? g.perm[off + r0 + tid] : -1;
        s_p[tid] = p;
        s_arow[tid] = p < 0 ? 0 : p / g.K;
    }
    __syncthreads();
    L.kin2 = 2u * Kin;
    L.nb = (uint32_t)nb;
    L.arow = s_arow;
    L.rx = g2_rsrc(g.xh, g.xrows * (int64_t)Kin * 2);
    L.rbs = g2_rsrc(g.xbs, g.xrows * (int64_t)nb * 32);
    L.rd = g2_rsrc(g.xd, g.xrows * (int64_t)nb * 4);
    // weight rows of the wave: h rows n0 + r (col tile 0), g rows I + n0 + r
    // of the fused matrix or up rows n0 + r (col tile 1), n0 = 256 ctile + 32 wave
    {
        const int64_t n0 = (int64_t)ctile * QK + 32 * wave;
        L.rowb = (uint32_t)g.a.row_bytes;
        L.w0 = (uint32_t)(n0 * g.a.row_bytes);
        L.rw[0] = g2_rsrc(g.a.data + (int64_t)e * g.a.mat_bytes, g.a.mat_bytes);
        if (g.fused) {
            L.rw[1] = L.rw[0];
            L.wct = (uint32_t)(g.I * g.a.row_bytes);
        } else {
            L.rw[1] = g2_rsrc(g.b.data + (int64_t)e * g.b.mat_bytes, g.b.mat_bytes);
            L.wct = 0;
        }
    }
    uint8_t *W = &s_w[wave][0];
    g2g_issue(L, 0, st0, W);

    float16_t acc[2][2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[rt][ct][i] = 0.f;

    for (int b = 0; b < nb; b += 2) {
        g2g_block(g, L, b, nb, st0, st1, W, acc);
        if (b + 1 < nb) g2g_block(g, L, b + 1, nb, st1, st0, W, acc);
    }

    // ---- GLU values to LDS as fp32 rows of 256 (+4 pad): rows 0-31 in
    // stage 0, rows 32-63 in stage 1 (all reads of the stages are done)
    __syncthreads();
    {
        const int col = 32 * wave + l32;
        float *V0 = (float *)st0.As, *V1 = (float *)st1.As;
        switch (g.act) {
        case 0: g2g_glu_rows<0>(acc, V0, V1, col, g2); break;
        case 1: g2g_glu_rows<1>(acc, V0, V1, col, g2); break;
        case 2: g2g_glu_rows<2>(acc, V0, V1, col, g2); break;
        default: g2g_glu_rows<3>(acc, V0, V1, col, g2); break;
        }
    }
    __syncthreads();
    // ---- Q8_K of each row (first column with the largest |v| sets the
    // scale), written as fp16(d * q) in the down weight's K order: thread
    // (row, t) owns K positions 32t .. 32t+31, which hold the row elements
    // base_t + f(j) (the two orders are affine in t)
    const int row = tid >> 3, t = tid & 7;
    const float *Vr = (row < 32 ? (const float *)st0.As : (const float *)st1.As) + (row & 31) * G2G_LDV;
    const int base = NEXT == 14 ? 4 * t : 64 * (t >> 2) + 8 * (t & 3);
    float x[32];
    AmaxIdx best{-1.f, 0, 0.f};
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        int f;
        if (NEXT == 14) {
            f = 128 * ((j >> 3) & 1) + 64 * (j >> 4) + 32 * ((j & 7) >> 2) + (j & 3);
        } else {
            constexpr int off4[8] = {0, 2, 32, 34, 1, 3, 33, 35};
            f = 128 * ((j >> 3) & 1) + 4 * (j >> 4) + off4[j & 7];
        }
        x[j] = Vr[base + f];
        best = amax_better(best, AmaxIdx{fabsf(x[j]), base + f, x[j]});
    }
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) {
        AmaxIdx b;
        b.ax = __shfl_xor(best.ax, o, 64);
        b.idx = __shfl_xor(best.idx, o, 64);
        b.val = __shfl_xor(best.val, o, 64);
        best = amax_better(best, b);
    }
    float is = 0.f, d = 0.f;
    if (best.ax != 0.f) {
        is = -127.f / best.val;
        d = 1 / is;
    }
    if (row < mrows) {
        u32x4 o[4];
#pragma unroll
        for (int j = 0; j < 32; j += 2) {
            const int q0 = d != 0.f ? imin(127, nearest_int(is * x[j])) : 0;
            const int q1 = d != 0.f ? imin(127, nearest_int(is * x[j + 1])) : 0;
            const half2_t h = {(_Float16)(d * (float)q0), (_Float16)(d * (float)q1)};
            o[j >> 3][(j >> 1) & 3] = h22u_(h);
        }
        u32x4 *dst = (u32x4 *)(g.acth + (int64_t)s_p[row] * g.I + (int64_t)ctile * QK + 32 * t);
#pragma unroll
        for (int k = 0; k < 4; ++k) dst[k] = o[k];
    }
}

// ------------------------------------------------------------------ STORE
// fp32 rows out: y[p][n] = sum_k x[p][k] w[n][k] for the dispatched rows p of
// one expert.  8 waves; the work-group tile is 64 rows x 256 weight rows,
// wave w owns weight rows 32w .. 32w+31 (one 32-wide col tile) for both
// 32-row row tiles.  Weights and activations are dequantized to fp16 (the
// activations arrive as fp16(d * q) in this weight type's K order).
//
// Staging as in the GLU kernel: MUBUF loads that write LDS.  Activations:
// two stages of 64 rows padded to 264 halfs.  Weights: one region per wave,
// the 32 rows' block b each covered by the 16-byte aligned chunks holding
// it (Q4_K: 9 chunks, 16-byte aligned; Q6_K: a 210-byte block starts at any
// even byte of a chunk, 14 chunks cover it, plus one pad chunk so the row
// stride (240 B) spreads the LDS banks).  Each lane re-aligns its half of
// the block with v_alignbyte after dword-aligned reads.
constexpr int G3_NCOL = 256;

template <int WT> struct G3Fmt;
template <> struct G3Fmt<12> {
    static constexpr int BB = Q4K_BYTES;   // block bytes
    static constexpr int NC = 9;           // 16-byte chunks per staged row
    static constexpr int NLD = 5;          // loads of 1 KB per wave (32 rows x NC chunks)
};
template <> struct G3Fmt<14> {
    static constexpr int BB = Q6K_BYTES;
    static constexpr int NC = 15;
    static constexpr int NLD = 8;
};

struct G3Buf {
    _Float16 As[G2_BM * G2G_LDA];
};

struct G3Lane {
    int wave, lane, l32, g2;
    __amdgpu_buffer_rsrc_t rx, rw;
    uint32_t aoff[5];    // activation loads: per-lane byte offsets (block 0)
    uint32_t wrow[8];    // weight loads: byte offset of block 0 of the slot's row + 16 * chunk... see g3_issue
    uint32_t wchk[8];    // 16 * chunk of the slot
    uint32_t srow;       // byte offset of block 0 of the lane's own row (l32)
};

// loads of block b: activation stage st (5 per wave, the 33rd issued by every
// wave with identical bytes) and the wave's weight region W (NLD per wave):
// slot 64j + lane holds chunk c of row r; the row's block b starts at byte
// wrow + b * BB, its covering chunks at that offset rounded down to 16
template <int WT>
__device__ __forceinline__ void g3_issue(const G3Lane &L, int b, G3Buf &st, uint8_t *W) {
    using F = G3Fmt<WT>;
#pragma unroll
    for (int j = 0; j < 5; ++j) {
        const int k = j < 4 ? L.wave + 8 * j : G2G_ALOADS - 1;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(L.rx, (lds_void_t *)&st.As[k * 512], 16, L.aoff[j], b * (QK * 2), 0,
                                                 0);
    }
#pragma unroll
    for (int j = 0; j < F::NLD; ++j) {
        const uint32_t start = L.wrow[j] + (uint32_t)(b * F::BB);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(L.rw, (lds_void_t *)(W + j * 1024), 16, (start & ~15u) + L.wchk[j], 0,
                                                 0, 0);
    }
}

// the lane's operand bytes of block b from its staged row (row l32):
//   Q4_K: q[0..15] = qs chunks 2g2, 2g2+1, hd = header (d, dmin, scales)
//   Q6_K: q[0..15] = ql half g2, q[16..23] = qh half g2,
//         hd.x/.y = scales[8g2 .. 8g2+8), hd.z = d (fp16 bits)
template <int WT>
__device__ __forceinline__ void g3_read_w(const G3Lane &L, int b, const uint8_t *W, uint32_t (&q)[24], u32x4 &hd) {
    using F = G3Fmt<WT>;
    const uint8_t *row = W + L.l32 * (16 * F::NC);
    if constexpr (WT == 12) {
        hd = *(const u32x4 *)row;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const u32x4 v = *(const u32x4 *)(row + 16 + 64 * L.g2 + 16 * k);
            q[4 * k] = v.x; q[4 * k + 1] = v.y; q[4 * k + 2] = v.z; q[4 * k + 3] = v.w;
        }
    } else {
        // the block starts at byte s0 (even) of the staged row: dword reads
        // from s0 & ~3, then a 0- or 2-byte shift
        const uint32_t s0 = (L.srow + (uint32_t)(b * F::BB)) & 15u;
        const uint32_t sh = s0 & 3u;
        const uint32_t *rw = (const uint32_t *)(row + (s0 & ~3u));
        uint32_t t[17];
#pragma unroll
        for (int k = 0; k < 17; ++k) t[k] = rw[16 * L.g2 + k];            // ql: bytes 64 g2 ..
#pragma unroll
        for (int k = 0; k < 16; ++k) q[k] = __builtin_amdgcn_alignbyte(t[k + 1], t[k], sh);
#pragma unroll
        for (int k = 0; k < 9; ++k) t[k] = rw[32 + 8 * L.g2 + k];         // qh: bytes 128 + 32 g2 ..
#pragma unroll
        for (int k = 0; k < 8; ++k) q[16 + k] = __builtin_amdgcn_alignbyte(t[k + 1], t[k], sh);
#pragma unroll
        for (int k = 0; k < 3; ++k) t[k] = rw[48 + 2 * L.g2 + k];         // scales: bytes 192 + 8 g2 ..
        hd.x = __builtin_amdgcn_alignbyte(t[1], t[0], sh);
        hd.y = __builtin_amdgcn_alignbyte(t[2], t[1], sh);
        hd.z = __builtin_amdgcn_alignbyte(rw[53], rw[52], sh) & 0xffffu;   // d: bytes 208, 209
        hd.w = 0u;
    }
}

// one K block: wait for its loads, read the lane's weights, start the loads
// of block b+1, accumulate block b
template <int WT>
__device__ __forceinline__ void g3_block(const G3Lane &L, int b, int nb, G3Buf &cur, G3Buf &nxt, uint8_t *W,
                                         float16_t (&acc)[2]) {
    const int l32 = L.l32, g2 = L.g2;
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    asm volatile("s_barrier" ::: "memory");
    uint32_t q[24];
    u32x4 hd;
    g3_read_w<WT>(L, b, W, q, hd);
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): the next weight loads overwrite the region
    __builtin_amdgcn_sched_barrier(0);
    if (b + 1 < nb) g3_issue<WT>(L, b + 1, nxt, W);
    __builtin_amdgcn_sched_barrier(0);
    const _Float16 *Ab = &cur.As[l32 * G2G_LDA + 8 * g2];
    if constexpr (WT == 12) {
        half2_t s_lo[2], nm_lo[2], s_hi[2], nm_hi[2];
        const float d = h2f((uint16_t)(hd.x & 0xffff)), dmin = h2f((uint16_t)(hd.x >> 16));
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            int sc, m;
            scale_min_k4_reg(4 * g2 + 2 * hf, hd.y, hd.z, hd.w, sc, m);
            s_lo[hf] = splat_(d * (float)sc);
            nm_lo[hf] = splat_(-(dmin * (float)m));
            scale_min_k4_reg(4 * g2 + 2 * hf + 1, hd.y, hd.z, hd.w, sc, m);
            s_hi[hf] = splat_(d * (float)sc);
            nm_hi[hf] = splat_(-(dmin * (float)m));
        }
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const half8_t A0 = *(const half8_t *)(Ab + 16 * s);
            const half8_t A1 = *(const half8_t *)(Ab + 32 * G2G_LDA + 16 * s);
            const int hf = s >> 3;
            const half8_t B = dq4_f16(q[s], s_lo[hf], nm_lo[hf], s_hi[hf], nm_hi[hf]);
            acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A0, B, acc[0], 0, 0, 0);
            acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A1, B, acc[1], 0, 0, 0);
        }
    } else {
        // step s = 2 jj + w: first quarter scale 4w + jj/4, second + 2
        half2_t sq[8];
        const float d = h2f((uint16_t)hd.z);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t word = k < 4 ? hd.x : hd.y;
            sq[k] = splat_(d * (float)(int)(int8_t)(word >> (8 * (k & 3))));
        }
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const half8_t A0 = *(const half8_t *)(Ab + 16 * s);
            const half8_t A1 = *(const half8_t *)(Ab + 32 * G2G_LDA + 16 * s);
            const int jj = s >> 1, w = s & 1;
            const int k0 = 4 * w + (jj >> 2);
            const half8_t B = dq6_f16(q[jj], q[8 + jj], q[16 + jj], w, sq[k0], sq[k0 + 2]);
            acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A0, B, acc[0], 0, 0, 0);
            acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A1, B, acc[1], 0, 0, 0);
        }
    }
}

template <int WT>
__global__ void __launch_bounds__(G2_THREADS) k_g2_store(G2Args g) {
    using F = G3Fmt<WT>;
    __shared__ __attribute__((aligned(1024))) G3Buf st0;
    __shared__ __attribute__((aligned(1024))) G3Buf st1;
    __shared__ __attribute__((aligned(1024))) uint8_t s_w[G2_WAVES][F::NLD * 1024];
    __shared__ int s_p[G2_BM], s_arow[G2_BM];
    const int nx = (int)((g.ncols + G3_NCOL - 1) / G3_NCOL);
    int tile, ctile;
    tile_coords(g.max_tiles, tile, ctile);
    if (tile >= *g.n_tiles || ctile >= nx) return;
    G3Lane L;
    const int tid = threadIdx.x;
    L.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    L.lane = tid & 63;
    L.l32 = L.lane & 31;
    L.g2 = L.lane >> 5;
    const int wave = L.wave, l32 = L.l32, g2 = L.g2;
    const int e = g.tile_e[tile], r0 = g.tile_r0[tile];
    const int cnt = g.counts[e], off = g.offsets[e];
    const int mrows = imin(G2_BM, cnt - r0);
    const uint32_t Kin = (uint32_t)g.a.K;
    const int nb = (int)(Kin / QK);
    if (tid < G2_BM) {
        const int p = tid < mrows ? g.perm[off + r0 + tid] : -1;
        s_p[tid] = p;
        s_arow[tid] = p < 0 ? 0 : (g.ne11 == 1 ? p / g.K : p);
    }
    __syncthreads();
    L.rx = g2_rsrc(g.xh, g.xrows * (int64_t)Kin * 2);
#pragma unroll
    for (int j = 0; j < 5; ++j) {
        // slot q = 64k + lane of the padded activation tile: row q / 33, chunk q % 33
        const int k = j < 4 ? wave + 8 * j : G2G_ALOADS - 1;
        const int q = 64 * k + L.lane;
        const int row = q / 33, ch = q % 33;
        L.aoff[j] = (uint32_t)s_arow[row] * (2u * Kin) + 16u * (uint32_t)(ch == 32 ? 0 : ch);
    }
    // weight rows n0 + r of the expert matrix (rows past ncols re-read the
    // last row; their outputs are never stored); offsets are relative to the
    // matrix base rounded down to 16 bytes, so 16-byte chunks are aligned
    {
        const uint8_t *mat = g.a.data + (int64_t)e * g.a.mat_bytes;
        const uint32_t mis = (uint32_t)((uintptr_t)mat & 15u);
        L.rw = g2_rsrc(mat - mis, g.a.mat_bytes + mis);
        const int n0 = ctile * G3_NCOL + 32 * wave, nlast = (int)g.ncols - 1;
        const uint32_t rowb = (uint32_t)g.a.row_bytes;
#pragma unroll
        for (int j = 0; j < F::NLD; ++j) {
            const int slot = imin(64 * j + L.lane, 32 * F::NC - 1);
            const int r = slot / F::NC, c = slot - F::NC * r;
            L.wrow[j] = mis + (uint32_t)imin(n0 + r, nlast) * rowb;
            L.wchk[j] = 16u * (uint32_t)c;
        }
        L.srow = mis + (uint32_t)imin(n0 + l32, nlast) * rowb;
    }
    uint8_t *W = &s_w[wave][0];
    g3_issue<WT>(L, 0, st0, W);

    float16_t acc[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[rt][i] = 0.f;
    for (int b = 0; b < nb; b += 2) {
        g3_block<WT>(L, b, nb, st0, st1, W, acc);
        if (b + 1 < nb) g3_block<WT>(L, b + 1, nb, st1, st0, W, acc);
    }
    // rows 32rt + 8(i/4) + 4g2 + i%4, column n
    const int64_t n = (int64_t)ctile * G3_NCOL + 32 * wave + l32;
    if (n < g.ncols) {
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int m = 32 * rt + 8 * (i >> 2) + 4 * g2 + (i & 3);
                if (m < mrows) g.y[(int64_t)s_p[m] * g.ldy + n] = acc[rt][i];
            }
    }
}

int launch_gemm2(const G2Args &g, hipStream_t st) {
    if (g.max_tiles <= 0) return 0;
    if (g.a.K % QK) return -6;
    if (g.glu) {
        if (g.a.type != 12 || (g.I % QK)) return -6;
        // byte offsets of the buffer loads are 32-bit
        const int64_t lim = 0x7fffffff;
        if (g.xrows <= 0 || g.xrows * g.a.K * 2 > lim || g.a.mat_bytes > lim || (!g.fused && g.b.mat_bytes > lim))
            return -6;
        // the weight loads use one row stride for both col tiles
        if (!g.fused && g.b.row_bytes != g.a.row_bytes) return -6;
        const int nx = (int)(g.I / QK);
        const dim3 grid((unsigned)((nx * g.max_tiles + 7) / 8 * 8));
        if (g.next_type == 14) hipLaunchKernelGGL(k_g2_glu<14>, grid, dim3(G2G_THREADS), 0, st, g);
        else hipLaunchKernelGGL(k_g2_glu<12>, grid, dim3(G2G_THREADS), 0, st, g);
    } else {
        const int nx = (int)((g.ncols + G3_NCOL - 1) / G3_NCOL);
        const int64_t lim = 0x7fffffff;
        if (g.xrows <= 0 || g.xrows * g.a.K * 2 > lim || g.a.mat_bytes + 16 > lim) return -6;
        const dim3 grid((unsigned)((nx * g.max_tiles + 7) / 8 * 8));
        if (g.a.type == 12) hipLaunchKernelGGL(k_g2_store<12>, grid, dim3(G2_THREADS), 0, st, g);
        else if (g.a.type == 14) hipLaunchKernelGGL(k_g2_store<14>, grid, dim3(G2_THREADS), 0, st, g);
        else return -3;
    }
    return hip_check_launch();
}

}  // namespace mimoe
