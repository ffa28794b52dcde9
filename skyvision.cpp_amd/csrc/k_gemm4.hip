// k_gemm4.hip - grouped k-quant GEMMs of the prefill on v_mfma_f32_32x32x16_f16:
// gate/up with the GLU and the Q8_K of its output fused in (k_g4_glu), and
// the down product (k_g4_store).
//
// One work-group of 4 waves per CU, one wave per SIMD with up to 512
// registers.  A work-group owns a tile of up to 128 dispatched rows of one
// expert (tokens gathered through the permutation) and 512 weight rows; each
// wave owns all of the tile's rows and 128 weight rows as 4 x 4 MFMA tiles of
// 32 x 32 (256 fp32 accumulators per lane).  Every dequantized weight operand
// feeds 4 MFMAs (one per 32-row tile) and every activation operand 4 (one per
// 32-column weight tile).  Row tiles past the tile's rows are skipped.
//
// The K loop runs in stages of half a super-block (128 K values = 8 MFMA
// steps of K 16):
//  * activations are fp16 d*q of the Q8_K rows, stored in the weight type's
//    MFMA K order (common.hpp); buffer loads that write LDS directly bring
//    each stage in, double buffered.  Row r of a stage is 16 chunks of 16 B;
//    LDS slot c of the row holds K chunk c ^ (r & 15), so the rows an MFMA
//    operand read touches at one K chunk spread over all banks.
//  * weights: each wave stages its rows' bytes for the next stage in a
//    private LDS region (coalesced loads that write LDS directly), copies its
//    operands into registers at the stage start and dequantizes them to fp16
//    in-register: Q4_K d*sc*q - dmin*m, Q6_K d*sc*(q - 32).
//
// Tile order: the dispatch lists full 128-row tiles first, then the partial
// tiles by decreasing row count; work-group 8q + x (x = XCD) runs tile
// 8 (q / nct) + x, column tile q % nct, so the column tiles of one row tile
// share that XCD's L2 for the activations and tiles start in list order.
#include "act.hpp"
#include "common.hpp"
#include "launch.hpp"

namespace mimoe {

constexpr int G4_WAVES = 4;
constexpr int G4_THREADS = G4_WAVES * 64;
constexpr int G4_NWG = 512;            // weight rows per work-group
constexpr int G4_SK = 128;             // K values per stage
constexpr int G4_AST = G4_BM * G4_SK;  // halfs per activation stage (32 KB)

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ inline half2_t g4_u2h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ inline uint32_t g4_h22u(half2_t h) { return __builtin_bit_cast(uint32_t, h); }
__device__ inline half2_t g4_splat(float f) {
    const _Float16 h = (_Float16)f;
    half2_t r = {h, h};
    return r;
}

// (v & mask) | orv in one v_and_or_b32 (mask in an SGPR)
__device__ __forceinline__ uint32_t g4_and_or(uint32_t v, uint32_t mask, uint32_t orv) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(mask), "v"(orv));
    return r;
}

// 8 nibbles of one Q4_K qs dword -> 8 fp16 weights, pairs (n0,n4) (n1,n5)
// (n2,n6) (n3,n7) (the q4k_elem32 operand order): low nibbles belong to
// sub-block lo, high nibbles to hi.  1024 + q via the 0x6400 exponent (64 + q
// for bits 4-7 via 0x5400), minus the offset (exact), then one fma with the
// block's s = d*sc, nm = -dmin*m.
__device__ __forceinline__ half8_t g4_dq4(uint32_t v, half2_t s_lo, half2_t nm_lo, half2_t s_hi, half2_t nm_hi,
                                          uint32_t m64, uint32_t m54) {
    const half2_t c1024 = {(_Float16)1024.f, (_Float16)1024.f};
    const half2_t c64 = {(_Float16)64.f, (_Float16)64.f};
    const uint32_t v8 = v >> 8;
    const half2_t t0 = g4_u2h2(g4_and_or(v, 0x000F000Fu, m64)) - c1024;
    const half2_t t1 = g4_u2h2(g4_and_or(v, 0x00F000F0u, m54)) - c64;
    const half2_t t2 = g4_u2h2(g4_and_or(v8, 0x000F000Fu, m64)) - c1024;
    const half2_t t3 = g4_u2h2(g4_and_or(v8, 0x00F000F0u, m54)) - c64;
    const u32x4 r = {g4_h22u(__builtin_elementwise_fma(t0, s_lo, nm_lo)),
                     g4_h22u(__builtin_elementwise_fma(t1, s_hi, nm_hi)),
                     g4_h22u(__builtin_elementwise_fma(t2, s_lo, nm_lo)),
                     g4_h22u(__builtin_elementwise_fma(t3, s_hi, nm_hi))};
    return __builtin_bit_cast(half8_t, r);
}

// 4 six-bit Q6_K codes in the bytes of x -> fp16 (q - 32) * s: v_perm_b32
// puts each byte under the 0x64 exponent byte (1024 + q), (1024 + q) - 1056 is
// exact, one rounding in the multiply
__device__ __forceinline__ void g4_q6b(uint32_t x, half2_t s, half2_t &lo, half2_t &hi) {
    const half2_t c1056 = {(_Float16)1056.f, (_Float16)1056.f};
    lo = (g4_u2h2(__builtin_amdgcn_perm(0x64646464u, x, 0x04010400u)) - c1056) * s;
    hi = (g4_u2h2(__builtin_amdgcn_perm(0x64646464u, x, 0x04030402u)) - c1056) * s;
}
// w = 0: quarters (q1, q2) from the low ql nibbles and qh bits 0-1 / 2-3;
// w = 1: quarters (q3, q4) from the high nibbles and qh bits 4-5 / 6-7
__device__ __forceinline__ half8_t g4_dq6(uint32_t qla, uint32_t qlb, uint32_t qh, int w, half2_t s_a, half2_t s_b) {
    uint32_t qa, qb;
    if (w == 0) {
        qa = (qla & 0x0F0F0F0Fu) | ((qh << 4) & 0x30303030u);
        qb = (qlb & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u);
    } else {
        qa = ((qla >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u);
        qb = ((qlb >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u);
    }
    half2_t a01, a23, b01, b23;
    g4_q6b(qa, s_a, a01, a23);
    g4_q6b(qb, s_b, b01, b23);
    const u32x4 r = {g4_h22u(a01), g4_h22u(a23), g4_h22u(b01), g4_h22u(b23)};
    return __builtin_bit_cast(half8_t, r);
}

// buffer resource of a byte range (reads past nbytes return 0)
__device__ inline rsrc_t g4_rsrc(const void *p, int64_t nbytes) {
    const int n = nbytes > 0x7fffffff ? 0x7fffffff : (int)nbytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, n, 0x00020000);
}
__device__ __forceinline__ u32x4 g4_ld4(rsrc_t r, uint32_t off, uint32_t soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, (int)soff, 0));
}
__device__ __forceinline__ uint32_t g4_ld1(rsrc_t r, uint32_t off, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, (int)soff, 0);
}

// ------------------------------------------------------------------ weights
// Each wave stages the weight bytes of its 128 rows for one stage in a
// private LDS region with buffer loads that write LDS directly (16 bytes per
// lane; one load covers 8 or 16 whole rows, so the loads are coalesced),
// copies its lanes' operand bytes into registers at the start of the stage
// and then loads the next stage over the region.  Slot k of row r sits at
// position k ^ swz(r), so the 8 rows an operand read touches at one slot fall
// into distinct bank groups.
//
// Q4_K (dword-aligned blocks): stage h covers half h of the block (qs bytes
// 64 h ..); 5 slots per row = the contiguous 80 bytes 64 h .. of the block
// (stage 0: header + qs[0..64); stage 1: qs[48..128), the first 16 unused),
// so lane group g2's 32 qs bytes sit in slots 1 + 2 g2, 2 + 2 g2 in both
// stages; the row stride of 5 slots spreads 8 rows over all bank groups.
// Q6_K (210-byte blocks start at any even byte): stage h covers half h of the
// block; 8 slots per row: slots 0-4 the 64 ql bytes 64 h .. and slots 5-7 the
// 32 qh bytes 128 + 32 h .., each run fetched from the dword at or below its
// start (the run begins sh = start & 3 bytes into its first slot);
// swz(r) = r & 7.
// The per-block header (Q4_K d, dmin, scales; Q6_K scales and d) is loaded
// straight into registers, one block ahead.
template <int WT> struct G4Fmt;
template <> struct G4Fmt<12> {
    static constexpr int SLOTS = 5, RPL = 0, NLD = 10;   // slots per row, rows per load (Q6_K), loads per stage
};
template <> struct G4Fmt<14> {
    static constexpr int SLOTS = 8, RPL = 8, NLD = 16;
};
template <int WT> constexpr int g4_wregion() { return 128 * G4Fmt<WT>::SLOTS * 16; }
template <int WT> __device__ __forceinline__ int g4_swz(int r) { return WT == 12 ? 0 : r & 7; }

// operand bytes of the stage in registers, per column tile
template <int WT> struct G4W;
template <> struct G4W<12> {
    u32x4 q[4][2];   // the lane group's 32 qs bytes (step sp uses dword sp)
};
template <> struct G4W<14> {
    uint32_t a[4][5], b[4][5], c[4][5];   // ql 64 h + 16 g2 .., ql 64 h + 32 + 16 g2 .., qh 128 + 32 h + 16 g2 .. (5 dwords, sh-shifted)
};
template <int WT> struct G4Hdr;
template <> struct G4Hdr<12> {
    u32x4 h[4];
};
template <> struct G4Hdr<14> {
    uint32_t sc[4][5], d[4];   // 16 scales from the dword at or below byte 192 (sh-shifted); d
};

// the next stage's weight loads of one wave.  Q4_K: load j covers slots
// 64 j .. 64 j + 63 of the wave's 128 rows x 5 (row q / 5, slot q % 5: one
// offset per load and lane); Q6_K: load j covers rows RPL (j % 8) + lane / 8
// of the wave's first (j < 8) or second 64 rows, slot (lane % 8) ^ swz(row).
template <int WT> struct G4WDma;
template <> struct G4WDma<12> {
    rsrc_t r0, r1;          // resources of the first / second 64 rows
    uint32_t off[10];       // lane's byte offset of load j at block 0, stage 0
};
template <> struct G4WDma<14> {
    rsrc_t r0, r1;
    uint32_t base0, base1;  // lane's run start at block 0, stage 0, before the dword rounding
    uint32_t inc_h;         // run start advance for stage 1 (64 ql, 32 qh)
    uint32_t kk16;          // 16 * slot index within the run
    uint32_t rstride;       // bytes between the rows of consecutive loads (8 rows)
};

template <int WT>
__device__ __forceinline__ void g4_issue_w(const G4WDma<WT> &dm, uint8_t *W, int j, int b, int h) {
    using F = G4Fmt<WT>;
    const rsrc_t r = j < F::NLD / 2 ? dm.r0 : dm.r1;
    if constexpr (WT == 12) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t *)(W + 1024 * j), 16, (int)dm.off[j],
                                                 b * Q4K_BYTES + 64 * h, 0, 0);
    } else {
        const int jj = j % (F::NLD / 2);
        const uint32_t base = j < F::NLD / 2 ? dm.base0 : dm.base1;
        const uint32_t x = base + (uint32_t)jj * dm.rstride + (uint32_t)(b * Q6K_BYTES) + (h ? dm.inc_h : 0u);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t *)(W + 1024 * j), 16, (int)((x & ~3u) + dm.kk16), 0, 0,
                                                 0);
    }
}

// the lane's operand bytes of the stage from the wave's region (Q4_K stage
// 0 also holds the block header)
template <int WT>
__device__ __forceinline__ void g4_copy_w(const uint8_t *W, int l32, int g2, int h, G4W<WT> &w, G4Hdr<WT> &k) {
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
        const int r = 32 * ct + l32;
        const uint8_t *row = W + r * (G4Fmt<WT>::SLOTS * 16);
        const int z = g4_swz<WT>(r);
        if constexpr (WT == 12) {
            if (h == 0) k.h[ct] = *(const u32x4 *)row;
            w.q[ct][0] = *(const u32x4 *)(row + 16 * (1 + 2 * g2));
            w.q[ct][1] = *(const u32x4 *)(row + 16 * (2 + 2 * g2));
        } else {
            const u32x4 a4 = *(const u32x4 *)(row + 16 * (g2 ^ z));
            const u32x4 b4 = *(const u32x4 *)(row + 16 * ((2 + g2) ^ z));
            const u32x4 c4 = *(const u32x4 *)(row + 16 * ((5 + g2) ^ z));
            w.a[ct][0] = a4.x; w.a[ct][1] = a4.y; w.a[ct][2] = a4.z; w.a[ct][3] = a4.w;
            w.b[ct][0] = b4.x; w.b[ct][1] = b4.y; w.b[ct][2] = b4.z; w.b[ct][3] = b4.w;
            w.c[ct][0] = c4.x; w.c[ct][1] = c4.y; w.c[ct][2] = c4.z; w.c[ct][3] = c4.w;
            w.a[ct][4] = *(const uint32_t *)(row + 16 * ((1 + g2) ^ z));
            w.b[ct][4] = *(const uint32_t *)(row + 16 * ((3 + g2) ^ z));
            w.c[ct][4] = *(const uint32_t *)(row + 16 * ((6 + g2) ^ z));
        }
    }
}

// Q6_K per-block scales and d of the lane's own rows (woff[ct]: byte offset
// of the row in rw[ct], including the matrix's misalignment)
template <int WT>
__device__ __forceinline__ void g4_load_hdr(const rsrc_t (&rw)[4], const uint32_t (&woff)[4], int b, G4Hdr<WT> &k) {
    if constexpr (WT == 14) {
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
            const uint32_t bs = woff[ct] + (uint32_t)(b * Q6K_BYTES);
            const uint32_t o = (bs + 192u) & ~3u;
            const u32x4 s4 = g4_ld4(rw[ct], o, 0u);
            k.sc[ct][0] = s4.x; k.sc[ct][1] = s4.y; k.sc[ct][2] = s4.z; k.sc[ct][3] = s4.w;
            k.sc[ct][4] = g4_ld1(rw[ct], o + 16u, 0u);
            k.d[ct] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rw[ct], (int)(bs + 208u), 0, 0);
        }
    }
}

// ------------------------------------------------------------------ activations
struct G4Tile {
    int e, mrows, nrt;
};

// rows of the tile: s_p = flat slot index (t*K + k) or -1, s_arow = activation row
__device__ __forceinline__ G4Tile g4_tile(const G2Args &g, int tile, int *s_p, int *s_arow) {
    G4Tile t;
    t.e = g.tile_e[tile];
    const int r0 = g.tile_r0[tile];
    const int cnt = g.counts[t.e], off = g.offsets[t.e];
    t.mrows = imin(G4_BM, cnt - r0);
    t.nrt = (t.mrows + 31) >> 5;
    const int tid = threadIdx.x;
    if (tid < G4_BM) {
        const int p = tid < t.mrows ? g.perm[off + r0 + tid] : -1;
        s_p[tid] = p;
        s_arow[tid] = p < 0 ? 0 : (g.ne11 == 1 ? p / g.K : p);
    }
    __syncthreads();
    return t;
}

// Activation loads of a stage: the 8 NRT loads of 4 rows (1 KB each) of the
// tile's NRT row tiles are dealt to the 4 waves, 2 NRT each.  Load j of wave w
// writes rows 4 L .. 4 L + 3, L = 2 NRT w + j; lane i fetches row 4 L + i / 16,
// K chunk (i % 16) ^ (row % 16) into LDS slot i % 16 of the row.
template <int NRT>
__device__ __forceinline__ void g4_aoffsets(const int *s_arow, int wave, int lane, uint32_t rowbytes,
                                            uint32_t (&aoff)[2 * NRT]) {
#pragma unroll
    for (int j = 0; j < 2 * NRT; ++j) {
        const int r = 4 * (2 * NRT * wave + j) + (lane >> 4);
        const int c = (lane & 15) ^ (r & 15);
        aoff[j] = (uint32_t)s_arow[r] * rowbytes + 16u * (uint32_t)c;
    }
}

// load j of stage (b, h) (the stage's bytes start at 2 (256 b + 128 h) in a row)
template <int NRT>
__device__ __forceinline__ void g4_issue_a(rsrc_t rx, const uint32_t (&aoff)[2 * NRT], int wave, int j, _Float16 *st,
                                           int b, int h) {
    const int L = 2 * NRT * wave + j;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void_t *)(st + 4 * L * G4_SK), 16, (int)aoff[j],
                                             512 * b + 256 * h, 0, 0);
}

// all of this wave's loads have landed, then every wave's (raw barrier: the
// asm memory clobber keeps the compiler from moving memory accesses across it)
__device__ __forceinline__ void g4_stage_sync() {
    __builtin_amdgcn_s_waitcnt(0);
    asm volatile("s_barrier" ::: "memory");
}

// ------------------------------------------------------------------ scales
// Per stage h and column tile: Q4_K s = d*sc and nm = -dmin*m of the lane's
// two sub-blocks 4 h + 2 g2 (low nibbles) and + 1 (high); Q6_K d*scale of the
// four scales the lane's quarter-rows use in half h: 8 h + g2 + {0, 2, 4, 6}
// (steps with w = 0 use the first two, w = 1 the last two).
template <int WT> struct G4Sc;
template <> struct G4Sc<12> {
    half2_t s_lo[4], nm_lo[4], s_hi[4], nm_hi[4];
};
template <> struct G4Sc<14> {
    half2_t sq[4][4];
};

template <int WT>
__device__ __forceinline__ void g4_scales(const G4Hdr<WT> &k, int ct, int g2, int h, uint32_t sh, G4Sc<WT> &s) {
    if constexpr (WT == 12) {
        const u32x4 hv = k.h[ct];
        const float d = h2f((uint16_t)(hv.x & 0xffffu)), dmin = h2f((uint16_t)(hv.x >> 16));
        int sc, m;
        scale_min_k4_reg(4 * h + 2 * g2, hv.y, hv.z, hv.w, sc, m);
        s.s_lo[ct] = g4_splat(d * (float)sc);
        s.nm_lo[ct] = g4_splat(-(dmin * (float)m));
        scale_min_k4_reg(4 * h + 2 * g2 + 1, hv.y, hv.z, hv.w, sc, m);
        s.s_hi[ct] = g4_splat(d * (float)sc);
        s.nm_hi[ct] = g4_splat(-(dmin * (float)m));
    } else {
        const float d = h2f((uint16_t)(k.d[ct] & 0xffffu));
        const uint32_t w0 = __builtin_amdgcn_alignbyte(k.sc[ct][2 * h + 1], k.sc[ct][2 * h], sh);
        const uint32_t w1 = __builtin_amdgcn_alignbyte(k.sc[ct][2 * h + 2], k.sc[ct][2 * h + 1], sh);
        const uint32_t sg = 8u * (uint32_t)g2;
        s.sq[ct][0] = g4_splat(d * (float)(int)(int8_t)(w0 >> sg));
        s.sq[ct][1] = g4_splat(d * (float)(int)(int8_t)(w0 >> (sg + 16u)));
        s.sq[ct][2] = g4_splat(d * (float)(int)(int8_t)(w1 >> sg));
        s.sq[ct][3] = g4_splat(d * (float)(int)(int8_t)(w1 >> (sg + 16u)));
    }
}

// ------------------------------------------------------------------ operands
// dword p of the weight operand of step sp, column tile ct: one quarter of a
// dequantization, so that it can sit between two MFMAs
template <int WT>
__device__ __forceinline__ uint32_t g4_piece(const G4W<WT> &w, const G4Sc<WT> &s, uint32_t sh, int sp, int ct, int p) {
    if constexpr (WT == 12) {
        const half2_t c1024 = {(_Float16)1024.f, (_Float16)1024.f};
        const half2_t c64 = {(_Float16)64.f, (_Float16)64.f};
        const uint32_t v = w.q[ct][sp >> 2][sp & 3];
        const uint32_t x = p < 2 ? v : v >> 8;
        half2_t t;
        if (p & 1) t = g4_u2h2(g4_and_or(x, 0x00F000F0u, 0x54005400u)) - c64;
        else t = g4_u2h2(g4_and_or(x, 0x000F000Fu, 0x64006400u)) - c1024;
        return g4_h22u((p & 1) ? __builtin_elementwise_fma(t, s.s_hi[ct], s.nm_hi[ct])
                               : __builtin_elementwise_fma(t, s.s_lo[ct], s.nm_lo[ct]));
    } else {
        const half2_t c1056 = {(_Float16)1056.f, (_Float16)1056.f};
        const int m = sp >> 1, ww = sp & 1;
        const uint32_t qh = __builtin_amdgcn_alignbyte(w.c[ct][m + 1], w.c[ct][m], sh);
        uint32_t q;
        if (p < 2) {
            const uint32_t ql = __builtin_amdgcn_alignbyte(w.a[ct][m + 1], w.a[ct][m], sh);
            q = ww == 0 ? (ql & 0x0F0F0F0Fu) | ((qh << 4) & 0x30303030u) : ((ql >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u);
        } else {
            const uint32_t ql = __builtin_amdgcn_alignbyte(w.b[ct][m + 1], w.b[ct][m], sh);
            q = ww == 0 ? (ql & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u)
                        : ((ql >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u);
        }
        const uint32_t sel = (p & 1) ? 0x04030402u : 0x04010400u;
        const half2_t sc = s.sq[ct][2 * ww + (p >> 1)];
        return g4_h22u((g4_u2h2(__builtin_amdgcn_perm(0x64646464u, q, sel)) - c1056) * sc);
    }
}

// activation operand of step sp, row tile rt: lane (l32, g2) reads row
// 32 rt + l32, K chunk 2 sp + g2, at slot chunk ^ (l32 % 16); abase =
// 256 l32 + 16 (g2 ^ (l32 % 16)) bytes, so the step's offset is abase ^ 32 sp
__device__ __forceinline__ half8_t g4_read_a(const char *stb, uint32_t abase, int sp, int rt) {
    return *(const half8_t *)(stb + (abase ^ (uint32_t)(32 * sp)) + rt * 32 * 256);
}

// ------------------------------------------------------------------ one stage
// 8 steps x 4 column tiles x NRT row tiles = 32 NRT MFMA slots in a fixed
// interleave: slot (sp, ct, rt) issues the MFMA of row tile rt on the current
// weight operand, its share of the dequantization of the next operand, during
// column tile 0 the activation operand of row tile rt for the next step, and
// extra(slot) (the next stage's loads and scales).  sched_barrier fences keep
// the order: one wave per SIMD hides ~4 VALU instructions behind an MFMA, but
// only between MFMAs.
template <int WT, int NRT, typename Extra>
__device__ __forceinline__ void g4_stage(const _Float16 *st, uint32_t abase, const G4W<WT> &w, const G4Sc<WT> &sc,
                                         uint32_t sh, f32x16 (&acc)[4][4], Extra &&extra) {
    const char *stb = (const char *)st;
    half8_t A[2][NRT];
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) A[0][rt] = g4_read_a(stb, abase, 0, rt);
    u32x4 Bc;
#pragma unroll
    for (int p = 0; p < 4; ++p) Bc[p] = g4_piece<WT>(w, sc, sh, 0, 0, p);
    int slot = 0;
#pragma unroll
    for (int sp = 0; sp < 8; ++sp) {
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
            const int nsp = ct == 3 ? sp + 1 : sp, nct = (ct + 1) & 3;
            u32x4 Bn = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt) {
                acc[rt][ct] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[sp & 1][rt], __builtin_bit_cast(half8_t, Bc),
                                                                     acc[rt][ct], 0, 0, 0);
                if (nsp < 8) {
#pragma unroll
                    for (int p = 0; p < 4; ++p)
                        if (p * NRT / 4 == rt) Bn[p] = g4_piece<WT>(w, sc, sh, nsp, nct, p);
                }
                if (ct == 0 && sp < 7) A[(sp + 1) & 1][rt] = g4_read_a(stb, abase, sp + 1, rt);
                extra(slot);
                ++slot;
                __builtin_amdgcn_sched_barrier(0);
            }
            Bc = Bn;
        }
    }
}

// the whole K loop for NRT row tiles: nb blocks = 2 nb stages.  At the start
// of stage (b, h) the wave copies its weight operands out of its region; the
// stage then loads, between its MFMAs, the activations (other LDS buffer) and
// weights (own region, after the copy has landed) of the next stage and
// computes the next stage's scales.  Q4_K headers arrive with the stage-0
// weights; Q6_K scales are loaded during (b, 1) for block b + 1.  Past the
// last block the loads repeat the last block (valid addresses, unused data;
// the epilogue waits for them).
template <int WT, int NRT>
__device__ __forceinline__ void g4_kloop_n(rsrc_t rx, const int *s_arow, uint32_t arowbytes, const rsrc_t (&rw)[4],
                                           const uint32_t (&woff)[4], const G4WDma<WT> &dm, uint8_t *W, int nb,
                                           int wave, int lane, _Float16 *As0, _Float16 *As1, f32x16 (&acc)[4][4]) {
    using F = G4Fmt<WT>;
    const int l32 = lane & 31, g2 = lane >> 5;
    const uint32_t abase = 256u * (uint32_t)l32 + 16u * (uint32_t)(g2 ^ (l32 & 15));
    uint32_t aoff[2 * NRT];
    g4_aoffsets<NRT>(s_arow, wave, lane, arowbytes, aoff);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[rt][ct][i] = 0.f;
    G4W<WT> w;
    G4Hdr<WT> k0;
    G4Sc<WT> s0, s1;
#pragma unroll
    for (int j = 0; j < 2 * NRT; ++j) g4_issue_a<NRT>(rx, aoff, wave, j, As0, 0, 0);
#pragma unroll
    for (int j = 0; j < F::NLD; ++j) g4_issue_w<WT>(dm, W, j, 0, 0);
    if constexpr (WT == 14) {
        g4_load_hdr<WT>(rw, woff, 0, k0);
        const uint32_t sh0 = woff[0] & 3u;
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) g4_scales<WT>(k0, ct, g2, 0, sh0, s0);
    }
    // slots of the extra work: the region's copy has landed at slot 1; then
    // NLD weight loads, 2 NRT activation loads, the Q6_K scales, and in the
    // last 4 slots the next stage's scales
    constexpr int XW = 1, XA = XW + F::NLD, XH = XA + 2 * NRT, XS = 32 * NRT - 4;
    for (int b = 0; b < nb; ++b) {
        const int bn = b + 1 < nb ? b + 1 : b;
        const uint32_t sh = WT == 14 ? ((woff[0] + (uint32_t)(b * Q6K_BYTES)) & 3u) : 0u;
        const uint32_t shn = WT == 14 ? ((woff[0] + (uint32_t)(bn * Q6K_BYTES)) & 3u) : 0u;
        g4_stage_sync();
        g4_copy_w<WT>(W, l32, g2, 0, w, k0);
        if constexpr (WT == 12) {
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) g4_scales<WT>(k0, ct, g2, 0, 0u, s0);
        }
        g4_stage<WT, NRT>(As0, abase, w, s0, sh, acc, [&](int i) __attribute__((always_inline)) {
            if (i == XW) __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): the copy is in registers
            if (i >= XW && i < XA) g4_issue_w<WT>(dm, W, i - XW, b, 1);
            if (i >= XA && i < XH) g4_issue_a<NRT>(rx, aoff, wave, i - XA, As1, b, 1);
            if (i >= XS) g4_scales<WT>(k0, i - XS, g2, 1, sh, s1);
        });
        // the header of block b is dead once the scales of (b, 1) are made
        g4_stage_sync();
        g4_copy_w<WT>(W, l32, g2, 1, w, k0);
        g4_stage<WT, NRT>(As1, abase, w, s1, sh, acc, [&](int i) __attribute__((always_inline)) {
            if (i == XW) __builtin_amdgcn_s_waitcnt(0xC07F);
            if (i >= XW && i < XA) g4_issue_w<WT>(dm, W, i - XW, bn, 0);
            if (i >= XA && i < XH) g4_issue_a<NRT>(rx, aoff, wave, i - XA, As0, bn, 0);
            if constexpr (WT == 14) {
                if (i == XH) g4_load_hdr<WT>(rw, woff, bn, k0);
                if (i >= XS) g4_scales<WT>(k0, i - XS, g2, 0, shn, s0);
            }
        });
    }
}

// one specialization per row-tile count (branch once per work-group)
template <int WT>
__device__ __forceinline__ void g4_kloop(rsrc_t rx, const int *s_arow, uint32_t arowbytes, const rsrc_t (&rw)[4],
                                         const uint32_t (&woff)[4], const G4WDma<WT> &dm, uint8_t *W, int nb, int wave,
                                         int lane, int nrt, _Float16 *As0, _Float16 *As1, f32x16 (&acc)[4][4]) {
    switch (nrt) {
    case 1: g4_kloop_n<WT, 1>(rx, s_arow, arowbytes, rw, woff, dm, W, nb, wave, lane, As0, As1, acc); break;
    case 2: g4_kloop_n<WT, 2>(rx, s_arow, arowbytes, rw, woff, dm, W, nb, wave, lane, As0, As1, acc); break;
    case 3: g4_kloop_n<WT, 3>(rx, s_arow, arowbytes, rw, woff, dm, W, nb, wave, lane, As0, As1, acc); break;
    default: g4_kloop_n<WT, 4>(rx, s_arow, arowbytes, rw, woff, dm, W, nb, wave, lane, As0, As1, acc); break;
    }
}

// per-lane weight-load descriptors; row0 / row1: the weight row of the wave's
// first / second 64 rows (rows row0 + r, r < 64, and row1 + r - 64)
template <int WT>
__device__ __forceinline__ G4WDma<WT> g4_wdma(rsrc_t r0, rsrc_t r1, int64_t row0, int64_t row1, uint32_t rb,
                                              uint32_t mis, int lane) {
    G4WDma<WT> dm;
    dm.r0 = r0;
    dm.r1 = r1;
    if constexpr (WT == 12) {
#pragma unroll
        for (int j = 0; j < 10; ++j) {
            const int q = 64 * j + lane, r = q / 5, k = q - 5 * r;
            const int64_t row = r < 64 ? row0 + r : row1 + (r - 64);
            dm.off[j] = (uint32_t)(row * rb) + 16u * (uint32_t)k;
        }
    } else {
        const int rl = lane >> 3, k = (lane & 7) ^ (lane >> 3);
        const uint32_t r0off = k < 5 ? 0u : 128u;
        dm.base0 = mis + (uint32_t)((row0 + rl) * rb) + r0off;
        dm.base1 = mis + (uint32_t)((row1 + rl) * rb) + r0off;
        dm.inc_h = k < 5 ? 64u : 32u;
        dm.kk16 = 16u * (uint32_t)(k < 5 ? k : k - 5);
        dm.rstride = 8u * rb;
    }
    return dm;
}

// ------------------------------------------------------------------ GLU
// Wave w owns act columns 64 w .. 64 w + 63 of the work-group's 256: column
// tiles 0, 1 are their h (gate) rows, 2, 3 their g (up) rows.
template <int ACT>
__device__ __forceinline__ void g4_glu_rows(const f32x16 (&acc)[4][4], int rt, float *V, int wave, int lane) {
    const int l32 = lane & 31, g2 = lane >> 5;
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = 8 * (i >> 2) + 4 * g2 + (i & 3);
            V[r * 256 + 64 * wave + 32 * ct + l32] = act_pair_fast<ACT>(acc[rt][ct][i], acc[rt][ct + 2][i]);
        }
}

// Q8_K of the 32 act rows of V (fp32, 256 columns), written as fp16(d * q) in
// the K order of the down weight type NEXT: thread (row, t) owns the K
// positions 32 t .. 32 t + 31 of the row's block, which hold the row elements
// base_t + f(j) (the two orders are affine in t)
template <int NEXT>
__device__ __forceinline__ void g4_q8k_rows(const float *V, int row0, int mrows, const int *s_p, _Float16 *acth,
                                            int64_t I, int ctile) {
    const int tid = threadIdx.x;
    const int row = tid >> 3, t = tid & 7;
    const float *Vr = V + row * 256;
    const int base = NEXT == 14 ? 128 * (t >> 2) + 4 * (t & 3) : 128 * (t >> 2) + 8 * (t & 3);
    float x[32];
    AmaxIdx best{-1.f, 0, 0.f};
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        int f;
        if (NEXT == 14) {
            f = 16 * ((j >> 3) & 1) + 64 * (j >> 4) + 32 * ((j & 7) >> 2) + (j & 3);
        } else {
            constexpr int off4[8] = {0, 2, 32, 34, 1, 3, 33, 35};
            f = 64 * ((j >> 3) & 1) + 4 * (j >> 4) + off4[j & 7];
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
    if (row0 + row < mrows) {
        u32x4 o[4];
#pragma unroll
        for (int j = 0; j < 32; j += 2) {
            const int q0 = d != 0.f ? imin(127, nearest_int(is * x[j])) : 0;
            const int q1 = d != 0.f ? imin(127, nearest_int(is * x[j + 1])) : 0;
            const half2_t h = {(_Float16)(d * (float)q0), (_Float16)(d * (float)q1)};
            o[j >> 3][(j >> 1) & 3] = g4_h22u(h);
        }
        u32x4 *dst = (u32x4 *)(acth + (int64_t)s_p[row0 + row] * I + (int64_t)ctile * QK + 32 * t);
#pragma unroll
        for (int k = 0; k < 4; ++k) dst[k] = o[k];
    }
}

template <int ACT, int NEXT>
__device__ __forceinline__ void g4_glu_epilogue(const G2Args &g, const f32x16 (&acc)[4][4], const G4Tile &t,
                                                int ctile, int wave, int lane, _Float16 *As0, _Float16 *As1,
                                                const int *s_p) {
    __syncthreads();   // every wave is done reading the last stage
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
        if (rt >= t.nrt) break;
        float *V = (float *)(rt & 1 ? As1 : As0);
        g4_glu_rows<ACT>(acc, rt, V, wave, lane);
        __syncthreads();
        g4_q8k_rows<NEXT>(V, 32 * rt, t.mrows, s_p, g.acth, g.I, ctile);
    }
}

template <int NEXT>
__global__ void __launch_bounds__(G4_THREADS) __attribute__((amdgpu_waves_per_eu(1, 1))) k_g4_glu(G2Args g) {
    __shared__ __attribute__((aligned(1024))) _Float16 As0[G4_AST];
    __shared__ __attribute__((aligned(1024))) _Float16 As1[G4_AST];
    __shared__ __attribute__((aligned(1024))) uint8_t Ws[G4_WAVES][g4_wregion<12>()];
    __shared__ int s_p[G4_BM], s_arow[G4_BM];
    const int nct = (int)(g.I / QK);
    int tile, ctile;
    {
        const int lin = blockIdx.x, q = lin >> 3, x = lin & 7;
        const int kk = q / nct;
        ctile = q - kk * nct;
        tile = 8 * kk + x;
        if (tile >= *g.n_tiles) return;
    }
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int l32 = lane & 31;
    const G4Tile t = g4_tile(g, tile, s_p, s_arow);
    const int nrt = __builtin_amdgcn_readfirstlane(t.nrt);
    const uint32_t Kin = (uint32_t)g.a.K;
    const int nb = (int)(Kin / QK);
    const rsrc_t rx = g4_rsrc(g.xh, g.xrows * (int64_t)Kin * 2);
    // weight rows: h rows n0 + 32 ct + l32 (ct 0, 1), g rows (ct 2, 3) at
    // I + n0 + ... of the fused matrix or n0 + ... of the up matrix
    rsrc_t rw[4];
    uint32_t woff[4];
    {
        const int64_t n0 = (int64_t)ctile * QK + 64 * wave;
        const uint32_t rb = (uint32_t)g.a.row_bytes;
        const rsrc_t ra = g4_rsrc(g.a.data + (int64_t)t.e * g.a.mat_bytes, g.a.mat_bytes);
        const rsrc_t rg = g.fused ? ra : g4_rsrc(g.b.data + (int64_t)t.e * g.b.mat_bytes, g.b.mat_bytes);
        const int64_t gbase = g.fused ? g.I + n0 : n0;
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
            rw[ct] = ct < 2 ? ra : rg;
            const int64_t row = (ct < 2 ? n0 + 32 * ct : gbase + 32 * (ct - 2)) + l32;
            woff[ct] = (uint32_t)(row * rb);
        }
    }
    const G4WDma<12> dm = g4_wdma<12>(rw[0], rw[2], (int64_t)ctile * QK + 64 * wave,
                                      g.fused ? g.I + (int64_t)ctile * QK + 64 * wave : (int64_t)ctile * QK + 64 * wave,
                                      (uint32_t)g.a.row_bytes, 0u, lane);
    f32x16 acc[4][4];
    g4_kloop<12>(rx, s_arow, 2u * Kin, rw, woff, dm, Ws[wave], nb, wave, lane, nrt, As0, As1, acc);
    switch (g.act) {
    case 0: g4_glu_epilogue<0, NEXT>(g, acc, t, ctile, wave, lane, As0, As1, s_p); break;
    case 1: g4_glu_epilogue<1, NEXT>(g, acc, t, ctile, wave, lane, As0, As1, s_p); break;
    case 2: g4_glu_epilogue<2, NEXT>(g, acc, t, ctile, wave, lane, As0, As1, s_p); break;
    default: g4_glu_epilogue<3, NEXT>(g, acc, t, ctile, wave, lane, As0, As1, s_p); break;
    }
}

// ------------------------------------------------------------------ STORE
// y[p][n] = sum_k x[p][k] w[n][k] for the tile's rows p; wave w owns weight
// rows 512 ctile + 128 w + 32 ct + l32 (rows past ncols are not stored).
template <int WT>
__global__ void __launch_bounds__(G4_THREADS) __attribute__((amdgpu_waves_per_eu(1, 1))) k_g4_store(G2Args g) {
    __shared__ __attribute__((aligned(1024))) _Float16 As0[G4_AST];
    __shared__ __attribute__((aligned(1024))) _Float16 As1[G4_AST];
    __shared__ __attribute__((aligned(1024))) uint8_t Ws[G4_WAVES][g4_wregion<WT>()];
    __shared__ int s_p[G4_BM], s_arow[G4_BM];
    const int nct = (int)((g.ncols + G4_NWG - 1) / G4_NWG);
    int tile, ctile;
    {
        const int lin = blockIdx.x, q = lin >> 3, x = lin & 7;
        const int kk = q / nct;
        ctile = q - kk * nct;
        tile = 8 * kk + x;
        if (tile >= *g.n_tiles) return;
    }
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int l32 = lane & 31, g2 = lane >> 5;
    const G4Tile t = g4_tile(g, tile, s_p, s_arow);
    const int nrt = __builtin_amdgcn_readfirstlane(t.nrt);
    const uint32_t Kin = (uint32_t)g.a.K;
    const int nb = (int)(Kin / QK);
    const rsrc_t rx = g4_rsrc(g.xh, g.xrows * (int64_t)Kin * 2);
    // weight rows n0 + r of the expert matrix; rows past ncols read zeros
    // (past the matrix's resource) or unused bytes, and are not stored
    rsrc_t rw[4];
    uint32_t woff[4];
    {
        const uint8_t *mat = g.a.data + (int64_t)t.e * g.a.mat_bytes;
        const uint32_t mis = WT == 14 ? (uint32_t)((uintptr_t)mat & 3u) : 0u;
        const rsrc_t r = g4_rsrc(mat - mis, g.a.mat_bytes + mis);
        const uint32_t rb = (uint32_t)g.a.row_bytes;
        const int n0 = ctile * G4_NWG + 128 * wave;
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
            rw[ct] = r;
            woff[ct] = mis + (uint32_t)(n0 + 32 * ct + l32) * rb;
        }
    }
    const G4WDma<WT> dm = [&]() {
        const uint8_t *mat = g.a.data + (int64_t)t.e * g.a.mat_bytes;
        const uint32_t mis = WT == 14 ? (uint32_t)((uintptr_t)mat & 3u) : 0u;
        const int n0 = ctile * G4_NWG + 128 * wave;
        return g4_wdma<WT>(rw[0], rw[0], n0, n0 + 64, (uint32_t)g.a.row_bytes, mis, lane);
    }();
    f32x16 acc[4][4];
    g4_kloop<WT>(rx, s_arow, 2u * Kin, rw, woff, dm, Ws[wave], nb, wave, lane, nrt, As0, As1, acc);
    // rows 32 rt + 8 (i / 4) + 4 g2 + i % 4, columns nb0 + 32 ct
    const int nb0 = ctile * G4_NWG + 128 * wave + l32;
    const int ncv = imin(4, (int)((g.ncols - nb0 + 31) / 32));   // column tiles of this lane inside ncols
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
        if (rt >= nrt) break;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int m = 32 * rt + 8 * (i >> 2) + 4 * g2 + (i & 3);
            if (m < t.mrows) {
                float *yr = g.y + (int64_t)s_p[m] * g.ldy + nb0;
#pragma unroll
                for (int ct = 0; ct < 4; ++ct)
                    if (ct < ncv) yr[32 * ct] = acc[rt][ct][i];
            }
        }
    }
}

// ------------------------------------------------------------------ launch
int launch_gemm4(const G2Args &g, hipStream_t st) {
    if (g.max_tiles <= 0) return 0;
    if (g.a.K % QK) return -6;
    const int64_t lim = 0x7fffffff;
    // byte offsets of the buffer loads are 32-bit
    if (g.xrows <= 0 || g.xrows * g.a.K * 2 > lim || g.a.mat_bytes + 4 > lim) return -6;
    const int ntile8 = (g.max_tiles + 7) / 8;
    if (g.glu) {
        if (g.a.type != 12 || (g.I % QK)) return -6;
        if (!g.fused && (g.b.mat_bytes > lim || g.b.type != 12)) return -6;
        // dword loads of the blocks
        if ((uintptr_t)g.a.data % 4 || g.a.mat_bytes % 4 || g.a.row_bytes % 4) return -6;
        if (!g.fused && ((uintptr_t)g.b.data % 4 || g.b.mat_bytes % 4 || g.b.row_bytes % 4)) return -6;
        const int nct = (int)(g.I / QK);
        const dim3 grid((unsigned)(8 * nct * ntile8));
        if (g.next_type == 14) hipLaunchKernelGGL(k_g4_glu<14>, grid, dim3(G4_THREADS), 0, st, g);
        else hipLaunchKernelGGL(k_g4_glu<12>, grid, dim3(G4_THREADS), 0, st, g);
    } else {
        const int nct = (int)((g.ncols + G4_NWG - 1) / G4_NWG);
        const dim3 grid((unsigned)(8 * nct * ntile8));
        if (g.a.type == 12) {
            if ((uintptr_t)g.a.data % 4 || g.a.mat_bytes % 4) return -6;
            hipLaunchKernelGGL(k_g4_store<12>, grid, dim3(G4_THREADS), 0, st, g);
        } else if (g.a.type == 14) {
            hipLaunchKernelGGL(k_g4_store<14>, grid, dim3(G4_THREADS), 0, st, g);
        } else {
            return -3;
        }
    }
    return hip_check_launch();
}

}  // namespace mimoe
