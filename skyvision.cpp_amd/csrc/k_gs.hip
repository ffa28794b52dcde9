// k_gs.hip - grouped Q4_K products for calls that dispatch few rows per
// expert: tiles of at most GS_BM = 16 rows from a balanced dispatch.  Every
// weight byte then feeds at most 16 rows, so the products are bound by the
// weight stream, and these kernels are built to keep that stream full:
// gate/up with the GLU fused in (k_gs_glu) and the plain product (k_gs_store,
// the down product).
//
// Work: an item is (tile, column split).  The item's activation rows (fp16
// d*q of their Q8_K, in the 32x32x16 MFMA K order of Q4_K that the 4-wave
// GEMMs read too) are staged in LDS once; each of the 4 waves then walks its
// share of the split's 16-column groups block by block.  A step is one
// 256-value super-block of 16 weight rows (GLU: 16 gate rows and the 16
// matching up rows).  The lane's weight bytes go straight into registers
// (16-byte loads of the block's header - d, dmin, scales - and of the 32
// bytes of its qs chunk) in groups of consecutive steps, across column-group
// boundaries.
//
// MFMA: v_mfma_f32_16x16x32_f16, weights as A (16 rows), the tile's rows as
// B (16 columns).  Lane (i = lane % 16, G = lane / 16) supplies 8 weights of
// weight row i and 8 activations of tile row i, both of K group G.  Step S
// (0..7) of a super-block takes, for group G, qs dword S of chunk G (low
// nibbles: sub-block 2 G, high nibbles: 2 G + 1), whose 8 values the
// 32x32x16 order keeps at step s = 8 (G / 2) + S, group g = G % 2: halfs
// 16 s + 8 g .. + 7 of the block's activations.  The accumulator lane holds
// weight rows 4 G .. 4 G + 3 of tile row i: four consecutive outputs of one
// row, stored as one 8-byte (fp16) or 16-byte (fp32) piece.
//
// LDS: the tile's rows at a stride of 2 K + 16 bytes (the 16-byte pad puts
// the 16 rows an operand read touches on distinct banks), filled by buffer
// loads that write LDS directly, 1 KB per instruction (pad slots and slots
// past the tile's rows fetch a valid dummy piece).
#include "act.hpp"
#include "common.hpp"
#include "launch.hpp"

namespace mimoe {

// waves per work-group: one work-group per CU (GLU: 2 waves per SIMD; the
// store, with fewer weight registers per step: 4), so that no work-group of
// a CU outlasts another (the older work-group's waves win the issue
// arbitration)
constexpr int GS_WAVES_GLU = 8, GS_WAVES_ST = 16;   // waves per work-group
constexpr int GS_WGS_GLU = 1, GS_WGS_ST = 1;         // work-groups per CU
template <bool GLU> constexpr int gs_waves() { return GLU ? GS_WAVES_GLU : GS_WAVES_ST; }
template <bool GLU> constexpr int gs_waves_per_simd() { return gs_waves<GLU>() * (GLU ? GS_WGS_GLU : GS_WGS_ST) / 4; }
constexpr int GS_GROUP_GLU = 3;   // weight steps per load group (GLU: 2 matrices per step)
constexpr int GS_GROUP_ST = 6;    // (store: 1 matrix per step)

typedef __attribute__((address_space(3))) void gs_lds_t;
typedef __amdgpu_buffer_rsrc_t gs_rsrc_t;

__device__ inline gs_rsrc_t gs_rsrc(const void *p, int64_t nbytes) {
    const int n = nbytes > 0x7fffffff ? 0x7fffffff : (int)nbytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, n, 0x00020000);
}

// (v & mask) | orv in one v_and_or_b32 (mask in an SGPR)
__device__ __forceinline__ uint32_t gs_and_or(uint32_t v, uint32_t mask, uint32_t orv) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(mask), "v"(orv));
    return r;
}
__device__ inline half2_t gs_u2h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ inline uint32_t gs_h22u(half2_t h) { return __builtin_bit_cast(uint32_t, h); }
__device__ inline half2_t gs_splat(float f) {
    const _Float16 h = (_Float16)f;
    half2_t r = {h, h};
    return r;
}

// one step's weight bytes of the lane, NM matrices (GLU: gate, up)
template <int NM> struct GsW {
    u32x4 h[NM];    // block header: d, dmin, scales[12]
    u32x4 q0[NM];   // qs chunk G, dwords 0..3
    u32x4 q1[NM];   // dwords 4..7
};

// scales of the lane's sub-blocks 2 G (A, low nibbles) and 2 G + 1 (B):
// s = d * sc, nm = 8 d * sc - dmin * m (centred codes, q4k_center)
struct GsSc {
    half2_t sA, nmA, sB, nmB;
};
__device__ __forceinline__ GsSc gs_scales(u32x4 h, int G) {
    const uint32_t hx = h.x;
    const float d = h2f((uint16_t)(hx & 0xffffu)), dmin = h2f((uint16_t)(hx >> 16));
    GsSc s;
    int sc, m;
    scale_min_k4_reg(2 * G, h.y, h.z, h.w, sc, m);
    s.sA = gs_splat(d * (float)sc);
    s.nmA = gs_splat(q4k_center(d, sc, dmin, m));
    scale_min_k4_reg(2 * G + 1, h.y, h.z, h.w, sc, m);
    s.sB = gs_splat(d * (float)sc);
    s.nmB = gs_splat(q4k_center(d, sc, dmin, m));
    return s;
}

// dword v of qs (nibbles a0 b0 a1 b1 a2 b2 a3 b3, a = sub-block 2 G, b =
// 2 G + 1) -> the operand (a0, a2, b0, b2, a1, a3, b1, b3): codes as exact
// fp16 integers q - 8 (1024 + q - 1032, 64 + q - 72), one packed fma per
// pair: w = (q - 8) s + nm
__device__ __forceinline__ half8_t gs_dq(uint32_t v, const GsSc &s) {
    const half2_t c1032 = {(_Float16)1032.f, (_Float16)1032.f};
    const half2_t c72 = {(_Float16)72.f, (_Float16)72.f};
    const uint32_t v8 = v >> 8;
    const half2_t t0 = gs_u2h2(gs_and_or(v, 0x000F000Fu, 0x64006400u)) - c1032;
    const half2_t t1 = gs_u2h2(gs_and_or(v, 0x00F000F0u, 0x54005400u)) - c72;
    const half2_t t2 = gs_u2h2(gs_and_or(v8, 0x000F000Fu, 0x64006400u)) - c1032;
    const half2_t t3 = gs_u2h2(gs_and_or(v8, 0x00F000F0u, 0x54005400u)) - c72;
    const u32x4 r = {gs_h22u(__builtin_elementwise_fma(t0, s.sA, s.nmA)),
                     gs_h22u(__builtin_elementwise_fma(t1, s.sB, s.nmB)),
                     gs_h22u(__builtin_elementwise_fma(t2, s.sA, s.nmA)),
                     gs_h22u(__builtin_elementwise_fma(t3, s.sB, s.nmB))};
    return __builtin_bit_cast(half8_t, r);
}

// dword S of a step's qs chunk (S compile-time after unrolling)
template <int NM>
__device__ __forceinline__ uint32_t gs_qdw(const GsW<NM> &w, int m, int S) {
    const u32x4 q = S < 4 ? w.q0[m] : w.q1[m];
    const int k = S & 3;
    return k == 0 ? q.x : k == 1 ? q.y : k == 2 ? q.z : q.w;
}

// The weight stream's loads are issued by asm statements, in program order,
// and waited for by explicit counts (gs_wait: at most N of this wave's
// vector-memory operations outstanding, which they leave in issue order)
// followed by gs_pin on the registers the wait covers, so that nothing reads
// them earlier.  (The compiler's own wait placement cannot follow a ring of
// registers loaded several steps ahead through a loop: it waited for the
// whole ring at every turn.)  Loads and waits the compiler places itself
// only ever wait longer with these outstanding, never shorter.  Global loads
// with 64-bit lane addresses: no scalar operand, so no uniformity the
// compiler would have to prove; every address they are given lies inside
// its table.
template <int OFF>
__device__ __forceinline__ u32x4 gs_ld16(const uint8_t *p) {
    u32x4 r;
    asm volatile("global_load_dwordx4 %0, %1, off offset:%2" : "=v"(r) : "v"(p), "n"(OFF));
    return r;
}
__device__ __forceinline__ int gs_ld4(const int32_t *p) {
    int r;
    asm volatile("global_load_dword %0, %1, off" : "=v"(r) : "v"(p));
    return r;
}
template <int N>
__device__ __forceinline__ void gs_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N));
}

// the weight stream of a wave: the lane's pointer to its row's block 0 in
// each matrix (header; the qs chunk is 16 + 32 G further), and the position
// (column group, block) of the next step to load
template <int NM> struct GsStream {
    const uint8_t *ptr[NM];   // lane's row, block 0
    uint32_t qoff;            // 16 + 32 G
    uint32_t cg_stride;       // bytes from a column group of the wave to its next (4 groups of 16 rows)
    uint32_t bstride;         // bytes from a block of the row to its next: 144 (rows), 4608 (tiled)
    int kb, nb;               // next block, blocks per row
    int left;                 // steps still to load after the next (the last one repeats)
};

// issue the next step's 3 NM loads into w and advance (selects, no branch)
template <int NM>
__device__ __forceinline__ void gs_load(GsStream<NM> &st, GsW<NM> &w) {
    const uint32_t boff = (uint32_t)st.kb * st.bstride;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        const uint8_t *b = st.ptr[m] + boff;
        w.h[m] = gs_ld16<0>(b);
        w.q0[m] = gs_ld16<0>(b + st.qoff);
        w.q1[m] = gs_ld16<16>(b + st.qoff);
    }
    const bool adv = st.left > 0;
    const bool wrap = adv && st.kb + 1 == st.nb;
    st.left -= adv ? 1 : 0;
    st.kb = wrap ? 0 : st.kb + (adv ? 1 : 0);
#pragma unroll
    for (int m = 0; m < NM; ++m) st.ptr[m] += wrap ? st.cg_stride : 0u;
}

template <int NM>
__device__ __forceinline__ void gs_pin(GsW<NM> &w) {
#pragma unroll
    for (int m = 0; m < NM; ++m) asm volatile("" : "+v"(w.h[m]), "+v"(w.q0[m]), "+v"(w.q1[m]));
}

// one step: 8 MFMAs per matrix on the block's activations at lds_a (the
// lane's B operand base for this block)
template <int NM>
__device__ __forceinline__ void gs_step(const GsW<NM> &w, const char *lds_a, int G, float4_t (&acc)[NM]) {
    GsSc sc[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) sc[m] = gs_scales(w.h[m], G);
#pragma unroll
    for (int S = 0; S < 8; ++S) {
        const half8_t b = *(const half8_t *)(lds_a + 32 * S);
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            const half8_t a = gs_dq(gs_qdw<NM>(w, m, S), sc[m]);
            acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[m], 0, 0, 0);
        }
    }
}

struct GsItem {
    int e, mrows, split, tile;
};
// the item's tile and split, its rows' slot indices (the dispatch's per-tile
// copy of the perm entries: lane i holds tile row i % 16's; rows past the
// tile's hold stale values) issued first, then the tile's expert and row
// count and n_tiles by scalar loads: one round trip.  False for an item past
// the dispatch's tiles (its slot-index load is waited for first).
__device__ __forceinline__ bool gs_item(const G2Args &g, int splits, int lane, GsItem &it, int &p_row) {
    const int item = blockIdx.x, tile = item / splits;
    const int tt = tile < g.max_tiles ? tile : g.max_tiles - 1;
    p_row = gs_ld4(g.tile_perm + (int64_t)tt * GS_BM + (lane & 15));
    const int nt = *g.n_tiles;
    it.e = g.tile_e[tt];
    it.mrows = g.tile_rows[tt];
    it.split = item - tile * splits;
    it.tile = tile;
    if (tile < nt) return true;
    gs_wait<0>();
    return false;
}

// the tile's rows (arow: the activation row of tile row lane % 16, valid in
// every lane) into LDS: slot f (16 bytes) of the row-major image with rows
// of P + 1 slots holds piece f % (P + 1) of row f / (P + 1); pad slots and
// rows past mrows fetch piece 0 of row arow(0)
__device__ __forceinline__ void gs_stage_rows(gs_rsrc_t rx, char *As, int arow, int mrows, int P, uint32_t rowbytes,
                                              int wave, int nwaves, int lane) {
    const int nslot = mrows * (P + 1), nch = (nslot + 63) >> 6;
    const int a0 = __builtin_amdgcn_readlane(arow, 0);
    for (int c = wave; c < nch; c += nwaves) {
        const int f = 64 * c + lane;
        const int r = f / (P + 1), k = f - r * (P + 1);
        const int ar = __shfl(arow, r & 15, 64);
        const bool live = r < mrows && k < P;
        const uint32_t off = live ? (uint32_t)ar * rowbytes + 16u * (uint32_t)k : (uint32_t)a0 * rowbytes;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (gs_lds_t *)(As + 1024 * c), 16, (int)off, 0, 0, 0);
    }
}

// One kernel for both products.  GLU: column groups of 16 act columns (h
// rows n, g rows I + n of the fused matrix or n of the up matrix), act(h, g)
// rows out; else column groups of 16 output columns n.  Rows out as fp16
// (yh, saturated and counted) or fp32 (y), [p][ldy].  KMAX: the longest
// activation row the LDS holds.
template <bool GLU, int ACT, int KMAX>
__global__ void __launch_bounds__(64 * gs_waves<GLU>()) __attribute__((amdgpu_waves_per_eu(gs_waves_per_simd<GLU>(), gs_waves_per_simd<GLU>())))
k_gs(G2Args g, int splits) {
    constexpr int NW = gs_waves<GLU>();
    constexpr int NM = GLU ? 2 : 1, LPS = 3 * NM;
    constexpr int D = GLU ? GS_GROUP_GLU : GS_GROUP_ST;
    constexpr int LDSB = ((GS_BM * (2 * KMAX + 16) + 1023) / 1024) * 1024;
    __shared__ __attribute__((aligned(1024))) char As[LDSB];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    GsItem it;
    int p_row;   // slot index of tile row lane % 16
    if (!gs_item(g, splits, lane, it, p_row)) return;
    const int G = lane >> 4, i16 = lane & 15;
    const int Kin = (int)g.a.K, nb = Kin / QK;
    const int ncg = (int)((GLU ? g.I : g.ncols) / 16);
    const int c_lo = (int)((int64_t)it.split * ncg / splits), c_hi = (int)((int64_t)(it.split + 1) * ncg / splits);
    const int ncw = c_hi - c_lo > wave ? (c_hi - c_lo - wave + NW - 1) / NW : 0;
    const int nsteps = ncw * nb;
    const int64_t rb = g.a.row_bytes;
    GsStream<NM> st;
    const int64_t n0 = ncw > 0 ? 16 * (c_lo + wave) + i16 : 0;   // (a wave without steps loads row 0 and never uses it)
    // tiled tables: row n's block b at (n / 32) 32 rb + 4608 b + 144 (n % 32);
    // 16 NW rows on (a whole number of 32-row groups) stays cg_stride
    const int64_t roff = g.tiled ? (n0 >> 5) * 32 * rb + (n0 & 31) * Q4K_BYTES : n0 * rb;
    st.ptr[0] = g.a.data + (int64_t)it.e * g.a.mat_bytes + roff;
    if constexpr (GLU) {
        st.ptr[1] = g.fused ? st.ptr[0] + g.I * rb : g.b.data + (int64_t)it.e * g.b.mat_bytes + roff;
    }
    st.bstride = g.tiled ? 32u * Q4K_BYTES : (uint32_t)Q4K_BYTES;
    st.qoff = 16u + 32u * (uint32_t)G;
    st.cg_stride = (uint32_t)(16 * NW * rb);
    st.kb = 0;
    st.nb = nb;
    st.left = nsteps - 1;
    // Prologue, in issue order: once the slot indices are in, the activation
    // rows into LDS and the first group of weight steps; the K loop starts
    // when the work-group's rows are in.
    gs_wait<0>();
    asm volatile("" : "+v"(p_row));
    const int arow = g.ne11 == 1 ? p_row / g.K : p_row;
    const gs_rsrc_t rx = gs_rsrc(g.xh, g.xrows * (int64_t)Kin * 2);
    gs_stage_rows(rx, As, arow, it.mrows, Kin / 8, 2u * (uint32_t)Kin, wave, NW, lane);
    // weights in groups of D steps: a group is loaded, waited for and
    // computed (the other waves of the CU keep the memory busy meanwhile).
    // Consecutive blocks of a row leave together, which the memory serves
    // faster than the same loads spread one step apart: a rolling ring that
    // kept D steps in flight measured 1-3 % slower per layer.
    GsW<NM> w[D];
#pragma unroll
    for (int j = 0; j < D; ++j) gs_load<NM>(st, w[j]);
    gs_wait<D * LPS>();   // the wave's LDS loads landed
    lds_barrier();        // (a barrier without the memory fence: the weight steps stay in flight)
    const uint32_t rs = 2u * (uint32_t)Kin + 16u;
    const char *lds_lane = As + i16 * rs + 16 * (G & 1) + 256 * (G >> 1);
    float4_t acc[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) acc[m] = float4_t{0.f, 0.f, 0.f, 0.f};
    bool over = false;
    int ckb = 0, ccg = c_lo + wave;
    const bool row_live = i16 < it.mrows;
    // one step on the weights in w[j]; at a column group's last block its
    // 16 x 16 outputs leave
    auto step = [&](GsW<NM> &wj) __attribute__((always_inline)) {
        gs_pin<NM>(wj);
        gs_step<NM>(wj, lds_lane + 512 * ckb, G, acc);
        if (++ckb == nb) {
            ckb = 0;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if constexpr (GLU) v[r] = act_pair_fast<ACT>(acc[0][r], acc[1][r]);
                else v[r] = acc[0][r];
            }
            const int64_t col = (int64_t)ccg * 16 + 4 * G;
            if (g.yh) {
                // (rows past the tile's hold stale LDS bytes: not counted, not stored)
#pragma unroll
                for (int r = 0; r < 4; ++r) over = over || (row_live && !(fabsf(v[r]) <= kF16Max));
                const uint32_t h01 = (uint32_t)__builtin_bit_cast(uint16_t, f16_sat(v[0])) |
                                     ((uint32_t)__builtin_bit_cast(uint16_t, f16_sat(v[1])) << 16);
                const uint32_t h23 = (uint32_t)__builtin_bit_cast(uint16_t, f16_sat(v[2])) |
                                     ((uint32_t)__builtin_bit_cast(uint16_t, f16_sat(v[3])) << 16);
                if (row_live) *(uint2 *)(g.yh + (int64_t)p_row * g.ldy + col) = make_uint2(h01, h23);
            } else if (row_live) {
                *(float4 *)(g.y + (int64_t)p_row * g.ldy + col) = make_float4(v[0], v[1], v[2], v[3]);
            }
#pragma unroll
            for (int m = 0; m < NM; ++m) acc[m] = float4_t{0.f, 0.f, 0.f, 0.f};
            ccg += NW;
        }
    };
    // the exit test before every step leaves a group only forwards
    for (int s0 = 0;; s0 += D) {
        gs_wait<0>();
#pragma unroll
        for (int j = 0; j < D; ++j) {
            if (s0 + j >= nsteps) goto done;
            step(w[j]);
        }
#pragma unroll
        for (int j = 0; j < D; ++j) gs_load<NM>(st, w[j]);
    }
done:
    gs_wait<0>();   // the last group's unused loads land before the wave ends
    if (__ballot(over) != 0 && lane == 0 && g.range_total) atomicAdd(g.range_total, 1);
}

// ------------------------------------------------------------------ launch
int gemm_gs_waves(int glu) { return glu ? GS_WAVES_GLU : GS_WAVES_ST; }
int gemm_gs_wgs_per_cu(int glu) { return glu ? GS_WGS_GLU : GS_WGS_ST; }

int launch_gemm_gs(const G2Args &g, int splits, hipStream_t st) {
    if (g.max_tiles <= 0) return 0;
    if (g.bm != GS_BM || !g.tile_perm || splits < 1 || splits > 64) return -6;
    if (g.a.type != 12 || g.a.K % QK || g.a.K > GS_KMAX) return -6;
    const int64_t lim = 0x7fffffff;
    if (g.xrows <= 0 || g.xrows * g.a.K * 2 > lim || g.a.mat_bytes + 64 > lim) return -6;
    if ((uintptr_t)g.a.data % 4 || g.a.mat_bytes % 4 || g.a.row_bytes % 4 || (uintptr_t)g.xh % 16) return -6;
    const int64_t ncols = g.glu ? g.I : g.ncols;
    if (ncols <= 0 || ncols % 16 || (int64_t)g.max_tiles * splits > lim) return -6;
    if (g.yh ? (g.ldy % 4 || (uintptr_t)g.yh % 8) : (g.ldy % 4 || (uintptr_t)g.y % 16)) return -6;
    // tiled: whole 32-row groups, no padding between matrices, the fused
    // matrix's g half starting on a group
    static_assert(GS_WAVES_GLU % 2 == 0 && GS_WAVES_ST % 2 == 0, "a wave's column groups step whole 32-row groups");
    if (g.tiled && (g.a.N % 32 || g.a.mat_bytes != g.a.N * g.a.row_bytes || (g.glu && g.fused && g.I % 32) ||
                    (g.glu && !g.fused && (g.b.N % 32 || g.b.mat_bytes != g.b.N * g.b.row_bytes))))
        return -6;
    const dim3 grid((unsigned)(g.max_tiles * splits));
    if (g.glu) {
        if (!g.fused && (g.b.type != 12 || g.b.row_bytes != g.a.row_bytes || g.b.mat_bytes + 64 > lim ||
                         (uintptr_t)g.b.data % 4 || g.b.mat_bytes % 4))
            return -6;
        switch (g.act) {
        case 0: hipLaunchKernelGGL((k_gs<true, 0, GS_KMAX>), grid, dim3(64 * gs_waves<true>()), 0, st, g, splits); break;
        case 1: hipLaunchKernelGGL((k_gs<true, 1, GS_KMAX>), grid, dim3(64 * gs_waves<true>()), 0, st, g, splits); break;
        case 2: hipLaunchKernelGGL((k_gs<true, 2, GS_KMAX>), grid, dim3(64 * gs_waves<true>()), 0, st, g, splits); break;
        case 3: hipLaunchKernelGGL((k_gs<true, 3, GS_KMAX>), grid, dim3(64 * gs_waves<true>()), 0, st, g, splits); break;
        default: return -6;
        }
    } else if (g.a.K <= GS_KMAX / 2) {
        hipLaunchKernelGGL((k_gs<false, 0, GS_KMAX / 2>), grid, dim3(64 * gs_waves<false>()), 0, st, g, splits);
    } else {
        hipLaunchKernelGGL((k_gs<false, 0, GS_KMAX>), grid, dim3(64 * gs_waves<false>()), 0, st, g, splits);
    }
    return hip_check_launch();
}

}  // namespace mimoe
