// k_gemm4.hip - grouped k-quant GEMMs of the prefill on v_mfma_f32_32x32x16_f16:
// gate/up with the GLU fused in (k_g4_glu, fp32 activations out) and the
// plain product (k_g4_store: the down product, mul_mat_id).
//
// One work-group of 4 waves per CU, one wave per SIMD.  A work-group owns a
// tile of up to G4_BM = 192 dispatched rows of one expert (tokens gathered
// through the permutation; an expert's rows are split into equal tiles of at
// most 192, so nearly every expert is one tile and its weights are streamed
// once per column tile) and 256 weight rows; each wave owns all of the tile's
// rows and 64 weight rows: up to 6 x 2 MFMA tiles of 32 x 32 (192 fp32
// accumulators per lane).  Every dequantized weight operand feeds one MFMA per row tile
// and every activation operand two.  Row tiles past the tile's rows are
// skipped (one specialization of the K loop per row-tile count).
//
// The K loop runs in stages of half a super-block (128 K values = 8 MFMA
// steps of K 16):
//  * activations (fp16 d*q of the Q8_K rows, in the weight type's MFMA K
//    order, common.hpp) reach LDS by buffer loads that write LDS directly,
//    double buffered; row r of a stage is 16 chunks of 16 B with K chunk c in
//    slot c ^ (r & 15), so the rows an operand read touches spread over all
//    banks.
//  * weights: each wave stages the whole block of its 64 rows in a private
//    LDS region (coalesced loads that write LDS directly, every byte fetched
//    once), copies its lanes' operand bytes for both stages into registers at
//    the block start and loads the next block over the region, one block
//    ahead; operands are dequantized to fp16 in-register (Q4_K d*sc*q -
//    dmin*m, Q6_K d*sc*(q - 32)).
// LDS: two activation stages of 48 KB and the waves' weight regions (4 x 9
// KB Q4_K, 4 x 16 KB Q6_K: 160 KB in all); the tile's activation rows sit in
// the second stage until the K loop has taken its load offsets, the rows'
// slot indices in the first after the K loop.
// Between its MFMAs a stage dequantizes the next weight operand a quarter at
// a time, reads the next step's activation operands and issues the next
// loads, in a fixed interleave (one wave per SIMD hides ~4 VALU instructions
// behind an MFMA, but only between MFMAs).
//
// Work-group 8 q + x (x = XCD) runs tile 8 (q / nct) + x, column tile q % nct:
// the column tiles of one row tile share that XCD's L2 for the activations.
#include "act.hpp"
#include "common.hpp"
#include "launch.hpp"
#include "q8h.hpp"
#include "wave_ops.hpp"

namespace mimoe {

constexpr int G4_WAVES = 4;
constexpr int G4_THREADS = G4_WAVES * 64;
constexpr int G4_NWG = 256;            // weight rows per work-group
constexpr int G4_SK = 128;             // K values per stage

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

// buffer resource of a byte range (reads past nbytes return 0)
__device__ inline rsrc_t g4_rsrc(const void *p, int64_t nbytes) {
    const int n = nbytes > 0x7fffffff ? 0x7fffffff : (int)nbytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, n, 0x00020000);
}

// ------------------------------------------------------------------ tiles
// Prologue order (each step one memory round trip): the tile's descriptor
// (expert, first row in perm, rows) and n_tiles together; then the rows'
// slot indices (perm) with the block-0 weight loads issued right behind
// them (they need only the expert); then, once the slot indices are in, the
// block-0 activation loads, while the weight loads are still landing.
struct G4Tile {
    int e, start, mrows, nrt;
    bool live;   // tile < n_tiles (the grid is rounded up to whole XCD rounds)
};

__device__ __forceinline__ G4Tile g4_desc(const G2Args &g, int tile) {
    const int tt = tile < g.max_tiles ? tile : g.max_tiles - 1;   // padding tiles read a valid entry
    G4Tile t;
    int nt = *g.n_tiles;
    t.e = g.tile_e[tt];
    t.start = g.tile_start[tt];
    t.mrows = g.tile_rows[tt];
    // all four values before the n_tiles test: one round trip, not two (the
    // compiler would not hoist the tile loads above the exit)
    asm volatile("" : "+s"(t.e), "+s"(t.start), "+s"(t.mrows), "+s"(nt));
    t.nrt = (t.mrows + 31) >> 5;
    t.live = tile < nt;
    return t;
}

// Small calls without a dispatch launch (G2Args::ids set, at most
// G4_SD_IDS ids, bm = G4_BM_SMALL or G4_BM_TINY): every work-group derives its own tile
// from the call's flat ids in LDS (scratch: the first activation buffer,
// free until the K loop) - the counts per expert, ceil(count / BM) equal
// tiles per expert in expert order (the dispatch's balanced tiles: the
// first count % tiles tiles one row longer), the expert holding tile
// `tile`, and that tile's rows: the expert's flat slot indices in ascending
// order (ballots per wave, wave totals in LDS), rows r0 .. r0 + rows of
// them.  Thread m < rows returns row m's slot index in p, else -1.
constexpr int G4_SD_NPT = G4_SD_IDS / G4_THREADS;   // ids per thread
static_assert(G4_SD_IDS == G4_SD_NPT * G4_THREADS && G4_SD_NPT <= 4, "whole ids per thread");
template <int BM>
__device__ __forceinline__ G4Tile g4_self_tile(const G2Args &g, int tile, int *s, int &p) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int E = g.n_expert, n = g.nids;
    int *s_cnt = s;              // [256] rows per expert
    int *s_wt = s + 256;         // [4] wave totals of the tile scan; [4 + 4 j, 8 + 4 j): ballot counts of id j
    int *s_sel = s + 280;        // [0] expert of the tile (-1: none), [1] its tile index within the expert
    int *s_rows = s + 288;       // [BM] the tile's slot indices
    int id[G4_SD_NPT];           // thread i holds ids i + j * G4_THREADS
#pragma unroll
    for (int j = 0; j < G4_SD_NPT; ++j) id[j] = tid + j * G4_THREADS < n ? g.ids[tid + j * G4_THREADS] : -1;
    s_cnt[tid] = 0;
    if (tid == 0) s_sel[0] = -1;
    if (tid < BM) s_rows[tid] = 0;   // (every entry a valid row, whatever follows)
    __syncthreads();
#pragma unroll
    for (int j = 0; j < G4_SD_NPT; ++j)
        if (id[j] >= 0 && id[j] < E) atomicAdd(&s_cnt[id[j]], 1);
    __syncthreads();
    // tiles per expert (thread e), inclusive scan over the 256 experts
    const int cnt_e = tid < E ? s_cnt[tid] : 0;
    const int nt_e = (cnt_e + BM - 1) / BM;
    const int inc = wave_incl_scan(nt_e);
    if (lane == 63) s_wt[wave] = inc;
    __syncthreads();
    int before = 0;
#pragma unroll
    for (int w = 0; w < G4_WAVES; ++w) before += w < wave ? s_wt[w] : 0;
    const int ts = before + inc - nt_e;   // the expert's first tile
    if (nt_e > 0 && tile >= ts && tile < ts + nt_e) {
        s_sel[0] = tid;
        s_sel[1] = tile - ts;
    }
    __syncthreads();
    G4Tile t;
    t.e = s_sel[0];
    const int sub = s_sel[1];
    p = -1;
    t.start = 0;
    t.live = t.e >= 0;
    if (!t.live) {
        t.mrows = 0;
        t.nrt = 0;
        return t;
    }
    const int cnt = s_cnt[t.e], nt = (cnt + BM - 1) / BM, base = cnt / nt, extra = cnt % nt;
    const int r0 = sub * base + (sub < extra ? sub : extra);
    t.mrows = base + (sub < extra ? 1 : 0);
    t.nrt = (t.mrows + 31) >> 5;
    // ranks in flat order: ids 0 .. G4_THREADS - 1 (id[0]), then the next
    // G4_THREADS (id[1]), ...
    const uint64_t below = (1ull << lane) - 1ull;
    uint64_t bal[G4_SD_NPT];
#pragma unroll
    for (int j = 0; j < G4_SD_NPT; ++j) {
        bal[j] = __ballot(id[j] == t.e);
        if (lane == 0) s_wt[4 + 4 * j + wave] = __builtin_popcountll(bal[j]);
    }
    __syncthreads();
    int done = 0;   // the expert's ids among the earlier groups
#pragma unroll
    for (int j = 0; j < G4_SD_NPT; ++j) {
        int pre = 0, tot = 0;
#pragma unroll
        for (int w = 0; w < G4_WAVES; ++w) {
            tot += s_wt[4 + 4 * j + w];
            pre += w < wave ? s_wt[4 + 4 * j + w] : 0;
        }
        const int rk = done + pre + __builtin_popcountll(bal[j] & below);
        if (id[j] == t.e && rk >= r0 && rk < r0 + t.mrows) s_rows[rk - r0] = tid + j * G4_THREADS;
        done += tot;
    }
    __syncthreads();
    p = tid < t.mrows ? s_rows[tid] : -1;
    return t;
}

// thread m < mrows: row m's flat slot index p (t*K + k), else -1
__device__ __forceinline__ int g4_rows_load(const G2Args &g, const G4Tile &t) {
    return (int)threadIdx.x < t.mrows ? g.perm[t.start + threadIdx.x] : -1;
}

// the rows' activation row indices to s_arow (row 0 past the tile), then a
// barrier that waits only for LDS: the block-0 weight loads issued before
// stay in flight, so the K loop's first activation loads go out while they
// land (__syncthreads would wait for them: one more round trip before the
// first MFMA)
template <int BM>
__device__ __forceinline__ void g4_rows_publish(const G2Args &g, int p, int *s_arow) {
    if (threadIdx.x < BM) s_arow[threadIdx.x] = p < 0 ? 0 : (g.ne11 == 1 ? p / g.K : p);
    lds_barrier();
}

// after the K loop (every load of this wave landed): the rows' slot indices
// to LDS, in the first activation buffer once no wave has a load in flight
template <int BM>
__device__ __forceinline__ const int *g4_publish_rows(_Float16 *As0, int p) {
    int *s_p = (int *)As0;
    __syncthreads();
    if (threadIdx.x < BM) s_p[threadIdx.x] = p;
    __syncthreads();
    return s_p;
}

// ------------------------------------------------------------------ weights
// The wave's 64 rows are two column tiles of 32 (ct 0, 1), each staged in its
// own part of the wave's region, row r of a part at r * SLOTS * 16 bytes.
//  Q4_K (dword-aligned 144-byte blocks): a row is its whole block, 9 slots
//   (stride 9 slots spreads 8 rows over all bank groups); 32 rows = 4.5 KB,
//   loaded by 4 loads of 1 KB and one of 512 B (its lanes 32-63 idle), so
//   that a column tile takes exactly its 4608 bytes of LDS.
//  Q6_K (210-byte blocks at any even byte): a row is 16 slots: 9 slots of ql
//   from the dword at or below the block start (sh = bs & 3 bytes before it),
//   5 slots of qh from the dword at or below bs + 128, 2 slots of scales and
//   d from the dword at or below bs + 192; slot k of row r sits at position
//   k ^ (r & 7).  32 rows = 8 KB = 8 loads.
template <int WT> struct G4Fmt;
template <> struct G4Fmt<12> {
    static constexpr int SLOTS = 9, PART = 32 * 9 * 16, NLD = 5;   // slots per row, bytes per column tile, loads per column tile
};
template <> struct G4Fmt<14> {
    static constexpr int SLOTS = 16, PART = 8 * 1024, NLD = 8;
};
// Q6_K in the tiled order (launch_tile_q6k): a column tile's block is 8 KB of
// merged codes, chunk c of 1 KB holding lane i's 16 bytes at 16 i (the LDS
// image is the copy's bytes), and 1 KB of fp16 scales loaded to registers
template <> struct G4Fmt<15> {
    static constexpr int SLOTS = 16, PART = 8 * 1024, NLD = 8;
};
template <int WT> constexpr int g4_wregion() { return 2 * G4Fmt<WT>::PART; }

// the whole block's operand bytes of the lane, both stages, per column tile
template <int WT> struct G4W;
template <> struct G4W<12> {
    u32x4 hdr[2];       // d, dmin, scales
    u32x4 q[2][2][2];   // [ct][h][half]: qs chunk 2 h + g2 (stage h, steps 0-3 / 4-7)
};
template <> struct G4W<15> {
    u32x4 q[2][2][4];   // [ct][h][m]: codes of stage h, dword m of the runs: a lo, a hi, b lo, b hi
    u32x4 s[2];         // [ct]: fp16 d * scale of the lane's sub-blocks, half 4 h + j
};
template <> struct G4W<14> {
    // [ct][h]: 16 bytes each of ql 64 h + 16 g2 .., ql 64 h + 32 + 16 g2 ..,
    // qh 32 h + 16 g2 .. (shifted into place at the copy)
    uint32_t a[2][2][4], b[2][2][4], c[2][2][4];
    uint32_t sc[2][5];  // scales (sh bytes early) and d (bytes 16 + sh ..)
};

// per-lane weight-load descriptors of the wave's two column tiles
template <int WT> struct G4WDma;
template <> struct G4WDma<12> {
    rsrc_t r[2];
    uint32_t off[2][5];   // [ct][j]: byte offset at block 0 of the lane's 16 bytes
    uint32_t bstride;     // bytes from one block to the next: 144 (rows), 4608 (tiled)
};
template <> struct G4WDma<15> {
    rsrc_t r[2];
    uint32_t base[2];     // [ct]: byte offset of the column tile's block 0 plus 16 lane
};
template <> struct G4WDma<14> {
    rsrc_t r[2];
    uint32_t x[2][2];     // [ct][j & 1]: run start of the lane's slot at block 0, before the dword rounding
    uint32_t kk[2];       // [j & 1]: 16 * slot index within its run
    uint32_t rstride;     // 4 rows
};

// rowbase[ct]: weight row of row 0 of column tile ct in r[ct]; mis: the
// matrix's misalignment below a dword (Q6_K; the resource starts at the
// dword at or below the matrix); tiled: Q4_K in the tiled order (rowbase a
// multiple of 32: the tile's block b is the 4608 bytes at rowbase rb + 4608 b,
// in the order of the LDS image)
template <int WT>
__device__ __forceinline__ G4WDma<WT> g4_wdma(rsrc_t r0, rsrc_t r1, const int64_t (&rowbase)[2], uint32_t rb,
                                              uint32_t mis, int lane, bool tiled = false) {
    G4WDma<WT> dm;
    dm.r[0] = r0;
    dm.r[1] = r1;
    if constexpr (WT == 12) {
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int j = 0; j < 5; ++j) {
                const int q = 64 * j + lane, r = imin(q / 9, 31), k = q - 9 * (q / 9);
                dm.off[ct][j] = tiled ? (uint32_t)(rowbase[ct] * rb) + 16u * (uint32_t)q
                                      : (uint32_t)((rowbase[ct] + r) * rb) + 16u * (uint32_t)k;
            }
        dm.bstride = tiled ? 32u * Q4K_BYTES : (uint32_t)Q4K_BYTES;
    } else if constexpr (WT == 15) {
        (void)mis;
        (void)tiled;
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) dm.base[ct] = (uint32_t)(rowbase[ct] * rb) + 16u * (uint32_t)lane;
    } else {
#pragma unroll
        for (int par = 0; par < 2; ++par) {
            const int rl = lane >> 4, k = (lane & 15) ^ (4 * par + rl);
            const uint32_t R = k < 9 ? 0u : (k < 14 ? 128u : 192u);
            dm.kk[par] = 16u * (uint32_t)(k < 9 ? k : (k < 14 ? k - 9 : k - 14));
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) dm.x[ct][par] = mis + (uint32_t)((rowbase[ct] + rl) * rb) + R;
        }
        dm.rstride = 4u * rb;
    }
    return dm;
}

// block 0's weight loads (issued before the K loop, right after the tile's
// descriptor is known)
template <int WT>
__device__ __forceinline__ void g4_issue_w0(const G4WDma<WT> &dm, uint8_t *W);

// load j (0 .. 2 NLD - 1: column tile j / NLD) of block b into the region W
template <int WT>
__device__ __forceinline__ void g4_issue_w(const G4WDma<WT> &dm, uint8_t *W, int j, int b) {
    using F = G4Fmt<WT>;
    const int ct = j / F::NLD, jj = j % F::NLD;
    uint8_t *dst = W + ct * F::PART + 1024 * jj;
    rsrc_t r = dm.r[ct];   // the builtin takes no const-qualified resource
    if constexpr (WT == 12) {
        // (the last load's lanes past the tile's 288 slots write nothing)
        if (jj + 1 < F::NLD || (int)(threadIdx.x & 63) < F::PART / 16 - 64 * (F::NLD - 1))
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t *)dst, 16, (int)dm.off[ct][jj],
                                                     b * (int)dm.bstride, 0, 0);
    } else if constexpr (WT == 15) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t *)dst, 16, (int)(dm.base[ct] + 1024u * (uint32_t)jj),
                                                 b * (32 * Q6X_ROW_BYTES), 0, 0);
    } else {
        const uint32_t x = dm.x[ct][jj & 1] + (uint32_t)jj * dm.rstride + (uint32_t)(b * Q6K_BYTES);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t *)dst, 16, (int)((x & ~3u) + dm.kk[jj & 1]), 0, 0,
                                                 0);
    }
}

template <int WT>
__device__ __forceinline__ void g4_issue_w0(const G4WDma<WT> &dm, uint8_t *W) {
#pragma unroll
    for (int j = 0; j < 2 * G4Fmt<WT>::NLD; ++j) g4_issue_w<WT>(dm, W, j, 0);
}

// Q6_K tiled: the scales of column tile ct, block b, into registers
__device__ __forceinline__ u32x4 g4_load_s15(const G4WDma<15> &dm, int ct, int b) {
    rsrc_t r = dm.r[ct];
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)(dm.base[ct] + 8192u), b * (32 * Q6X_ROW_BYTES), 0);
}

// the lane's operand bytes of the whole block from the region
template <int WT>
__device__ __forceinline__ void g4_copy_w(const uint8_t *W, int l32, int g2, uint32_t sh, G4W<WT> &w) {
    using F = G4Fmt<WT>;
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
        const uint8_t *row = W + ct * F::PART + l32 * (F::SLOTS * 16);
        if constexpr (WT == 15) {
            (void)row;
            const uint8_t *img = W + ct * F::PART + 16 * (l32 + 32 * g2);
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int m = 0; m < 4; ++m) w.q[ct][h][m] = *(const u32x4 *)(img + 1024 * (4 * h + m));
        } else if constexpr (WT == 12) {
            w.hdr[ct] = *(const u32x4 *)row;
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int c = 0; c < 2; ++c) w.q[ct][h][c] = *(const u32x4 *)(row + 16 * (1 + 2 * (2 * h + g2) + c));
        } else {
            const int z = l32 & 7;
            // 16 bytes from sh bytes into slot k (the run's data starts sh
            // bytes past the dword it was loaded from)
            auto rd = [&](int k, uint32_t (&d)[4]) __attribute__((always_inline)) {
                const u32x4 v = *(const u32x4 *)(row + 16 * (k ^ z));
                const uint32_t v4 = *(const uint32_t *)(row + 16 * ((k + 1) ^ z));
                d[0] = __builtin_amdgcn_alignbyte(v.y, v.x, sh);
                d[1] = __builtin_amdgcn_alignbyte(v.z, v.y, sh);
                d[2] = __builtin_amdgcn_alignbyte(v.w, v.z, sh);
                d[3] = __builtin_amdgcn_alignbyte(v4, v.w, sh);
            };
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                rd(4 * h + g2, w.a[ct][h]);
                rd(4 * h + 2 + g2, w.b[ct][h]);
                rd(9 + 2 * h + g2, w.c[ct][h]);
            }
            {
                const u32x4 v = *(const u32x4 *)(row + 16 * (14 ^ z));
                w.sc[ct][0] = v.x; w.sc[ct][1] = v.y; w.sc[ct][2] = v.z; w.sc[ct][3] = v.w;
                w.sc[ct][4] = *(const uint32_t *)(row + 16 * (15 ^ z));
            }
        }
    }
}

// ------------------------------------------------------------------ scales
// Per column tile and stage h: Q4_K s = d*sc and nm = 8 d*sc - dmin*m of the lane's
// sub-blocks 4 h + 2 g2 (low nibbles) and + 1 (high); Q6_K d*scale of the
// scales 8 h + g2 + {0, 2, 4, 6} of the lane's quarter-rows (steps with w = 0
// use the first two, w = 1 the last two).
template <int WT> struct G4Sc;
template <> struct G4Sc<12> {
    half2_t s_lo[2], nm_lo[2], s_hi[2], nm_hi[2];
};
template <> struct G4Sc<14> {
    half2_t sq[2][4];
};
template <> struct G4Sc<15> {
    half2_t sq[2][4];
};

template <int WT>
__device__ __forceinline__ void g4_scales(const G4W<WT> &w, int ct, int g2, int h, uint32_t sh, G4Sc<WT> &s) {
    if constexpr (WT == 12) {
        const u32x4 hv = w.hdr[ct];
        const float d = h2f((uint16_t)(hv.x & 0xffffu)), dmin = h2f((uint16_t)(hv.x >> 16));
        int sc, m;
        scale_min_k4_reg(4 * h + 2 * g2, hv.y, hv.z, hv.w, sc, m);
        s.s_lo[ct] = g4_splat(d * (float)sc);
        s.nm_lo[ct] = g4_splat(q4k_center(d, sc, dmin, m));
        scale_min_k4_reg(4 * h + 2 * g2 + 1, hv.y, hv.z, hv.w, sc, m);
        s.s_hi[ct] = g4_splat(d * (float)sc);
        s.nm_hi[ct] = g4_splat(q4k_center(d, sc, dmin, m));
    } else if constexpr (WT == 15) {
        (void)g2;
        (void)sh;
        const u32x4 v = w.s[ct];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t dw = v[2 * h + (j >> 1)];
            const _Float16 x = __builtin_bit_cast(_Float16, (uint16_t)((j & 1) ? dw >> 16 : dw & 0xffffu));
            s.sq[ct][j] = half2_t{x, x};
        }
    } else {
        const uint32_t dw = __builtin_amdgcn_alignbyte(w.sc[ct][4], w.sc[ct][4], sh);   // bytes 16 + sh .. : d
        const float d = h2f((uint16_t)(dw & 0xffffu));
        const uint32_t w0 = __builtin_amdgcn_alignbyte(w.sc[ct][2 * h + 1], w.sc[ct][2 * h], sh);
        const uint32_t w1 = __builtin_amdgcn_alignbyte(w.sc[ct][2 * h + 2], w.sc[ct][2 * h + 1], sh);
        const uint32_t sg = 8u * (uint32_t)g2;
        s.sq[ct][0] = g4_splat(d * (float)(int)(int8_t)(w0 >> sg));
        s.sq[ct][1] = g4_splat(d * (float)(int)(int8_t)(w0 >> (sg + 16u)));
        s.sq[ct][2] = g4_splat(d * (float)(int)(int8_t)(w1 >> sg));
        s.sq[ct][3] = g4_splat(d * (float)(int)(int8_t)(w1 >> (sg + 16u)));
    }
}

// ------------------------------------------------------------------ operands
// dword p of the weight operand of step sp of stage h, column tile ct: one
// quarter of a dequantization, so that it can sit between two MFMAs
template <int WT>
__device__ __forceinline__ uint32_t g4_piece(const G4W<WT> &w, const G4Sc<WT> &s, uint32_t sh, int h, int sp, int ct,
                                             int p) {
    if constexpr (WT == 12) {
        // centred codes q - 8 (see dq_q4k): 1024 + q - 1032, 64 + q - 72
        const half2_t c1032 = {(_Float16)1032.f, (_Float16)1032.f};
        const half2_t c72 = {(_Float16)72.f, (_Float16)72.f};
        const uint32_t v = w.q[ct][h][sp >> 2][sp & 3];
        const uint32_t x = p < 2 ? v : v >> 8;
        half2_t t;
        if (p & 1) t = g4_u2h2(g4_and_or(x, 0x00F000F0u, 0x54005400u)) - c72;
        else t = g4_u2h2(g4_and_or(x, 0x000F000Fu, 0x64006400u)) - c1032;
        return g4_h22u((p & 1) ? __builtin_elementwise_fma(t, s.s_hi[ct], s.nm_hi[ct])
                               : __builtin_elementwise_fma(t, s.s_lo[ct], s.nm_lo[ct]));
    } else if constexpr (WT == 15) {
        // the codes merged at the copy: the Q6_K form below without the merge
        (void)sh;
        const half2_t c1056 = {(_Float16)1056.f, (_Float16)1056.f};
        const int ww = sp & 1;
        const uint32_t q = w.q[ct][h][sp >> 1][ww + 2 * (p >> 1)];
        const uint32_t sel = (p & 1) ? 0x04030402u : 0x04010400u;
        const half2_t sc = s.sq[ct][2 * ww + (p >> 1)];
        return g4_h22u((g4_u2h2(__builtin_amdgcn_perm(0x64646464u, q, sel)) - c1056) * sc);
    } else {
        const half2_t c1056 = {(_Float16)1056.f, (_Float16)1056.f};
        const int m = sp >> 1, ww = sp & 1;
        const uint32_t qh = w.c[ct][h][m];
        uint32_t q;
        if (p < 2) {
            const uint32_t ql = w.a[ct][h][m];
            q = ww == 0 ? (ql & 0x0F0F0F0Fu) | ((qh << 4) & 0x30303030u) : ((ql >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u);
        } else {
            const uint32_t ql = w.b[ct][h][m];
            q = ww == 0 ? (ql & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u)
                        : ((ql >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u);
        }
        const uint32_t sel = (p & 1) ? 0x04030402u : 0x04010400u;
        const half2_t sc = s.sq[ct][2 * ww + (p >> 1)];
        return g4_h22u((g4_u2h2(__builtin_amdgcn_perm(0x64646464u, q, sel)) - c1056) * sc);
    }
}

// ------------------------------------------------------------------ activations
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

// tiles of TR < 32 rows (G4_BM_TINY): rows 4 w .. 4 w + 3 by wave w < TR / 4,
// one load per stage; the operands of rows TR .. 31 read rows r % TR (their
// products are not stored)
template <int TR>
__device__ __forceinline__ uint32_t g4_aoff_tiny(const int *s_arow, int wave, int lane, uint32_t rowbytes) {
    const int r = imin(4 * wave + (lane >> 4), TR - 1);
    return (uint32_t)s_arow[r] * rowbytes + 16u * (uint32_t)((lane & 15) ^ (r & 15));
}
template <int TR>
__device__ __forceinline__ void g4_issue_a_tiny(rsrc_t rx, uint32_t off, int wave, _Float16 *st, int b, int h) {
    if (wave < TR / 4)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void_t *)(st + 4 * wave * G4_SK), 16, (int)off,
                                                 512 * b + 256 * h, 0, 0);
}

// activation operand of step sp, row tile rt: lane (l32, g2) reads row
// 32 rt + l32, K chunk 2 sp + g2, at slot chunk ^ (l32 % 16); abase =
// 256 l32 + 16 (g2 ^ (l32 % 16)) bytes, so the step's offset is abase ^ 32 sp
__device__ __forceinline__ half8_t g4_read_a(const char *stb, uint32_t abase, int sp, int rt) {
    return *(const half8_t *)(stb + (abase ^ (uint32_t)(32 * sp)) + rt * 32 * 256);
}

// wait until at most N vector-memory loads of this wave are outstanding (and
// no LDS access), then for every wave (raw barrier: the asm memory clobber
// keeps the compiler from moving memory accesses across it)
template <int N>
__device__ __forceinline__ void g4_stage_sync() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
    asm volatile("s_barrier" ::: "memory");
}

// ------------------------------------------------------------------ one stage
// 8 steps x 2 column tiles x NRT row tiles = 16 NRT MFMA slots in a fixed
// interleave: slot (sp, ct, rt) issues the MFMA of row tile rt on the current
// weight operand, its share of the dequantization of the next operand, during
// column tile 0 the activation operand of row tile rt for the next step, and
// extra(slot) (loads and scales for what comes next).
template <int WT, int NRT, int NA, typename Extra>
__device__ __forceinline__ void g4_stage(const _Float16 *st, uint32_t abase, const G4W<WT> &w, const G4Sc<WT> &sc,
                                         uint32_t sh, int h, f32x16 (&acc)[NA][2], Extra &&extra) {
    const char *stb = (const char *)st;
    half8_t A[2][NRT];
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) A[0][rt] = g4_read_a(stb, abase, 0, rt);
    u32x4 Bc;
#pragma unroll
    for (int p = 0; p < 4; ++p) Bc[p] = g4_piece<WT>(w, sc, sh, h, 0, 0, p);
    int slot = 0;
#pragma unroll
    for (int sp = 0; sp < 8; ++sp) {
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            const int nsp = ct == 1 ? sp + 1 : sp, nct = ct ^ 1;
            u32x4 Bn = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt) {
                acc[rt][ct] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[sp & 1][rt], __builtin_bit_cast(half8_t, Bc),
                                                                     acc[rt][ct], 0, 0, 0);
                if (nsp < 8) {
#pragma unroll
                    for (int p = 0; p < 4; ++p)
                        if (p * NRT / 4 == rt) Bn[p] = g4_piece<WT>(w, sc, sh, h, nsp, nct, p);
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

// the whole K loop for NRT row tiles: nb blocks = 2 nb stages.
//  stage (b, 0): copy block b's weight operands out of the region, scales of
//    stage 0; between the MFMAs: the activation loads of (b, 1), then (after
//    the copy has landed) the weight loads of block b + 1 into the region,
//    and the scales of stage 1.
//  stage (b, 1): the activation loads of (b + 1, 0).
// The sync before (b, 1) waits only for the activations (issued before the
// weight loads, which stay in flight); the one before (b + 1, 0) for all.
// The last block's loads for a next one repeat it (valid addresses, unused
// data; the epilogue waits for them): measured faster than skipping them
// behind a uniform test per block, which costs the stage code more than the
// loads cost.
// Q6_K tiled (WT 15): sn holds the next block's scales (block 0's loaded
// with its weights); block b + 1's two scale loads follow its weight loads.
template <int WT, int NRT, int NA, int TR = 0>
__device__ __forceinline__ void g4_kloop_n(rsrc_t rx, const int *s_arow, uint32_t arowbytes, const G4WDma<WT> &dm,
                                           const uint32_t (&wsh)[2], uint8_t *W, int nb, int wave, int lane,
                                           _Float16 *As0, _Float16 *As1, f32x16 (&acc)[NA][2], u32x4 (&sn)[2]) {
    using F = G4Fmt<WT>;
    static_assert(TR == 0 || NRT == 1, "tiny tiles: one row tile");
    constexpr int NW = 2 * F::NLD, NSL = WT == 15 ? 2 : 0;   // weight loads, scale loads per block
    const int l32 = lane & 31, g2 = lane >> 5;
    const int ar = TR ? (l32 & (TR - 1)) : l32;   // the activation row the lane's operand reads
    const uint32_t abase = 256u * (uint32_t)ar + 16u * (uint32_t)(g2 ^ (ar & 15));
    uint32_t aoff[2 * NRT];
    if constexpr (TR > 0) {
        aoff[0] = aoff[1] = g4_aoff_tiny<TR>(s_arow, wave, lane, arowbytes);
    } else {
        g4_aoffsets<NRT>(s_arow, wave, lane, arowbytes, aoff);
    }
    auto issue_a = [&](int j, _Float16 *st, int bb, int h) __attribute__((always_inline)) {
        if constexpr (TR > 0) g4_issue_a_tiny<TR>(rx, aoff[0], wave, st, bb, h);
        else g4_issue_a<NRT>(rx, aoff, wave, j, st, bb, h);
    };
    constexpr int NAL = TR > 0 ? 1 : 2 * NRT;   // activation loads per stage (per wave)
#pragma unroll
    for (int rt = 0; rt < NA; ++rt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[rt][ct][i] = 0.f;
    G4W<WT> w;
    G4Sc<WT> s0, s1;
    // (block 0's weight loads are out already: g4_issue_w0)
#pragma unroll
    for (int j = 0; j < NAL; ++j) issue_a(j, As0, 0, 0);
    // extra work of stage 0 spread over its 16 NRT slots: the activation
    // loads at slots 4 i (i < 2 NRT), then, all after the last of them (the
    // sync before stage 1 counts on that order) and after the copy has
    // landed, the NW weight loads and the 2 column tiles' stage-1 scales
    constexpr int NS = 16 * NRT, S0 = 8 * NRT - 3, NI = NW + NSL + 2;
    for (int b = 0; b < nb; ++b) {
        // block b + 1's loads go out during block b; the last block reloads
        // itself (valid addresses, data unused) so that no stage branches
        const int bn = b + 1 < nb ? b + 1 : b;
        // Q6_K: bytes the block starts past a dword (same for all the lane's rows)
        const uint32_t sh = WT == 14 ? ((wsh[0] + (uint32_t)(b * Q6K_BYTES)) & 3u) : 0u;
        g4_stage_sync<0>();
        g4_copy_w<WT>(W, l32, g2, sh, w);
        if constexpr (WT == 15) {
            w.s[0] = sn[0];
            w.s[1] = sn[1];
        }
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) g4_scales<WT>(w, ct, g2, 0, sh, s0);
        g4_stage<WT, NRT>(As0, abase, w, s0, sh, 0, acc, [&](int slot) __attribute__((always_inline)) {
            if ((slot & 3) == 0 && (slot >> 2) < NAL) issue_a(slot >> 2, As1, b, 1);
            if (slot == S0) __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): the copy is in registers
#pragma unroll
            for (int it = 0; it < NI; ++it) {
                if (S0 + it * (NS - S0) / NI != slot) continue;
                if (it < NW) {
                    g4_issue_w<WT>(dm, W, it, bn);
                } else if (it < NW + NSL) {
                    if constexpr (WT == 15) sn[it - NW] = g4_load_s15(dm, it - NW, bn);
                } else {
                    g4_scales<WT>(w, it - NW - NSL, g2, 1, sh, s1);
                }
            }
        });
        g4_stage_sync<NW + NSL>();
        g4_stage<WT, NRT>(As1, abase, w, s1, sh, 1, acc, [&](int slot) __attribute__((always_inline)) {
            if (slot < NAL) issue_a(slot, As0, bn, 0);
        });
    }
}

// one specialization per row-tile count (branch once per work-group); NA
// row tiles of accumulators (the tile size's)
template <int WT, int NA, int TR = 0>
__device__ __forceinline__ void g4_kloop(rsrc_t rx, const int *s_arow, uint32_t arowbytes, const G4WDma<WT> &dm,
                                         const uint32_t (&wsh)[2], uint8_t *W, int nb, int wave, int lane, int nrt,
                                         _Float16 *As0, _Float16 *As1, f32x16 (&acc)[NA][2], u32x4 (&sn)[2]) {
    if constexpr (NA == 1) {
        g4_kloop_n<WT, 1, 1, TR>(rx, s_arow, arowbytes, dm, wsh, W, nb, wave, lane, As0, As1, acc, sn);
    } else {
        switch (nrt) {
        case 1: g4_kloop_n<WT, 1>(rx, s_arow, arowbytes, dm, wsh, W, nb, wave, lane, As0, As1, acc, sn); break;
        case 2: g4_kloop_n<WT, 2>(rx, s_arow, arowbytes, dm, wsh, W, nb, wave, lane, As0, As1, acc, sn); break;
        case 3: g4_kloop_n<WT, 3>(rx, s_arow, arowbytes, dm, wsh, W, nb, wave, lane, As0, As1, acc, sn); break;
        case 4: g4_kloop_n<WT, 4>(rx, s_arow, arowbytes, dm, wsh, W, nb, wave, lane, As0, As1, acc, sn); break;
        case 5: g4_kloop_n<WT, 5>(rx, s_arow, arowbytes, dm, wsh, W, nb, wave, lane, As0, As1, acc, sn); break;
        default: g4_kloop_n<WT, 6>(rx, s_arow, arowbytes, dm, wsh, W, nb, wave, lane, As0, As1, acc, sn); break;
        }
    }
}

// work-group -> (tile, column tile)
__device__ __forceinline__ void g4_coords(int nct, int &tile, int &ctile) {
    const int lin = blockIdx.x, q = lin >> 3, x = lin & 7;
    const int kk = q / nct;
    ctile = q - kk * nct;
    tile = 8 * kk + x;
}

// ------------------------------------------------------------------ GLU
// Wave w owns act columns 32 w .. 32 w + 31 of the work-group's 128: column
// tile 0 holds their h (gate) rows, column tile 1 their g (up) rows; the GLU
// values go out as rows (fp32 to y, or fp16 to yh), whose Q8_K for the down
// product needs whole 256-column blocks, which span two work-groups.
template <int ACT, int NA, int BM>
__device__ __forceinline__ void g4_glu_store(const G2Args &g, const f32x16 (&acc)[NA][2], const G4Tile &t,
                                             int ctile, int wave, int lane, const int *s_p, _Float16 *As0,
                                             _Float16 *As1) {
    // through LDS: the wave's 32 GLU columns of every row into the activation
    // buffers (rows 0-95 in As0, 96-191 in As1, 512 bytes per row), then
    // whole rows (512 bytes fp32, 256 bytes fp16) out in 16-byte pieces
    const int l32 = lane & 31, g2 = lane >> 5;
    if (g.yh) {
        bool over = false;
#pragma unroll
        for (int rt = 0; rt < NA; ++rt) {
            if (rt >= t.nrt) break;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                if (BM < 32 && 8 * (i >> 2) >= BM) continue;   // (rows past a tiny tile's)
                const int m = 32 * rt + 8 * (i >> 2) + 4 * g2 + (i & 3);
                _Float16 *row = m < (BM / 2) ? As0 + m * 256 : As1 + (m - (BM / 2)) * 256;
                const float v = act_pair_fast<ACT>(acc[rt][0][i], acc[rt][1][i]);
                over = over || !(fabsf(v) <= kF16Max);
                row[32 * wave + l32] = f16_sat(v);
            }
        }
        if (__ballot(over) != 0 && lane == 0 && g.range_total) atomicAdd(g.range_total, 1);
        __syncthreads();
        for (int idx = threadIdx.x; idx < t.mrows * 16; idx += G4_THREADS) {
            const int r = idx >> 4, c = idx & 15;
            const _Float16 *row = r < (BM / 2) ? As0 + r * 256 : As1 + (r - (BM / 2)) * 256;
            *(uint4 *)(g.yh + (int64_t)s_p[r] * g.ldy + (int64_t)ctile * 128 + 8 * c) = *(const uint4 *)(row + 8 * c);
        }
        return;
    }
#pragma unroll
    for (int rt = 0; rt < NA; ++rt) {
        if (rt >= t.nrt) break;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            if (BM < 32 && 8 * (i >> 2) >= BM) continue;
            const int m = 32 * rt + 8 * (i >> 2) + 4 * g2 + (i & 3);
            float *row = (float *)(m < (BM / 2) ? As0 + m * 256 : As1 + (m - (BM / 2)) * 256);
            row[32 * wave + l32] = act_pair_fast<ACT>(acc[rt][0][i], acc[rt][1][i]);
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < t.mrows * 32; idx += G4_THREADS) {
        const int r = idx >> 5, c = idx & 31;
        const float *row = (const float *)(r < (BM / 2) ? As0 + r * 256 : As1 + (r - (BM / 2)) * 256);
        *(float4 *)(g.y + (int64_t)s_p[r] * g.ldy + (int64_t)ctile * 128 + 4 * c) = *(const float4 *)(row + 4 * c);
    }
}

// Profiling only: the work-group's shader-clock and wall-clock counters
// (s_memtime, s_memrealtime) at its start (slot 0) and end (slot 1), from
// which the host measures the clock the CUs ran at under this kernel; a
// work-group with no tile writes zeros.
__device__ __forceinline__ void g4_clock(const G2Args &g, int slot, bool live) {
    if (g.clk != nullptr && threadIdx.x == 0 && blockIdx.x < (unsigned)g.clk_n) {
        uint64_t *p = g.clk + 4 * (size_t)blockIdx.x + 2 * slot;
        p[0] = live ? (uint64_t)clock64() : 0ull;
        p[1] = live ? (uint64_t)wall_clock64() : 0ull;
    }
}

// BM: tile rows (G4_BM; G4_BM_SMALL for few rows per expert: 52 KB of LDS
// with Q4_K weights, so that three work-groups share a CU and keep three
// times the weight stream in flight; G4_BM_TINY, calls without a dispatch
// launch and at most 4 rows per expert: 40 KB, four work-groups per CU)
template <int BM>
__global__ void __launch_bounds__(G4_THREADS)
    __attribute__((amdgpu_waves_per_eu(BM == G4_BM_TINY ? 4 : BM == G4_BM_MID ? 2 : 1, BM == G4_BM ? 1 : BM == G4_BM_TINY ? 4 : BM == G4_BM_MID ? 2 : 3)))
    k_g4_glu(G2Args g) {
    constexpr int NA = BM >= 32 ? BM / 32 : 1, TR = BM < 32 ? BM : 0;
    __shared__ __attribute__((aligned(1024))) _Float16 As0[BM * G4_SK];
    __shared__ __attribute__((aligned(1024))) _Float16 As1[BM * G4_SK];
    __shared__ __attribute__((aligned(1024))) uint8_t Ws[G4_WAVES][g4_wregion<12>()];
    int tile, ctile;
    g4_coords((int)(g.I / 128), tile, ctile);
    const bool self = BM <= G4_BM_SMALL && g.ids != nullptr;
    int my_p = -1;
    const G4Tile t = self ? g4_self_tile<BM>(g, tile, (int *)As0, my_p) : g4_desc(g, tile);
    g4_clock(g, 0, t.live);
    if (!t.live) {
        g4_clock(g, 1, false);
        return;
    }
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (!self) my_p = g4_rows_load(g, t);
    const int nrt = __builtin_amdgcn_readfirstlane(t.nrt);
    const uint32_t Kin = (uint32_t)g.a.K;
    const rsrc_t rx = g4_rsrc(g.xh, g.xrows * (int64_t)Kin * 2);
    // weight rows: h rows n0 .. n0 + 31 (column tile 0), g rows at I + n0 of
    // the fused matrix or n0 of the up matrix (column tile 1)
    const int64_t n0 = (int64_t)ctile * 128 + 32 * wave;
    const rsrc_t ra = g4_rsrc(g.a.data + (int64_t)t.e * g.a.mat_bytes, g.a.mat_bytes);
    const rsrc_t rg = g.fused ? ra : g4_rsrc(g.b.data + (int64_t)t.e * g.b.mat_bytes, g.b.mat_bytes);
    const int64_t rowbase[2] = {n0, g.fused ? g.I + n0 : n0};
    const G4WDma<12> dm = g4_wdma<12>(ra, rg, rowbase, (uint32_t)g.a.row_bytes, 0u, lane, g.tiled != 0);
    g4_issue_w0<12>(dm, Ws[wave]);
    // the activation rows live in the second activation buffer until the K
    // loop has computed its load offsets (its first write comes later)
    int *s_arow = (int *)As1;
    g4_rows_publish<BM>(g, my_p, s_arow);
    const uint32_t wsh[2] = {0u, 0u};
    f32x16 acc[NA][2];
    u32x4 sn[2];   // (Q6_K tiled only)
    g4_kloop<12, NA, TR>(rx, s_arow, 2u * Kin, dm, wsh, Ws[wave], (int)(Kin / QK), wave, lane, nrt, As0, As1, acc, sn);
    __builtin_amdgcn_s_waitcnt(0);   // no load may land in LDS after the work-group ends
    const int *s_p = g4_publish_rows<BM>((_Float16 *)&Ws[0][0], my_p);   // the row table in the weight region
    switch (g.act) {
    case 0: g4_glu_store<0, NA, BM>(g, acc, t, ctile, wave, lane, s_p, As0, As1); break;
    case 1: g4_glu_store<1, NA, BM>(g, acc, t, ctile, wave, lane, s_p, As0, As1); break;
    case 2: g4_glu_store<2, NA, BM>(g, acc, t, ctile, wave, lane, s_p, As0, As1); break;
    default: g4_glu_store<3, NA, BM>(g, acc, t, ctile, wave, lane, s_p, As0, As1); break;
    }
    g4_clock(g, 1, true);
}

// The Q8_K of the tile's activation rows (G2Args::q8src), made by the
// work-group before its K loop: one wave per (row, 4 blocks), 16 lanes per
// block (q8h.hpp, the code of the separate pass), written to xh, then every
// wave's stores out before the first activation loads.  Every column tile of
// the row tile writes the same bits.
template <int XO>
__device__ __forceinline__ void g4_q8_rows(const G2Args &g, int mrows, const int *s_arow, bool count, int wave,
                                           int lane) {
    const int nb = (int)(g.a.K / QK), ngrp = (nb + 3) >> 2;
    const int bl = lane >> 4, s = lane & 15;
    _Float16 *xh = const_cast<_Float16 *>(g.xh);
    for (int item = wave; item < mrows * ngrp; item += G4_WAVES) {   // (uniform per wave: DPP inside)
        const int r = item / ngrp, grp = item - r * ngrp;
        const int b = 4 * grp + bl;
        const bool bok = b < nb;
        const int64_t p = s_arow[r];
        float v[16];
        if (bok) {
            q8h_gather<XO>(g.q8src + p * g.q8ld + (int64_t)b * QK, s, v);
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = 0.f;
        }
        q8h_quant_store(v, bok, xh + p * (int64_t)nb * QK + (int64_t)b * QK, s, count ? g.range_total : nullptr);
    }
    vm_drain();       // this wave's rows are out (block 0's weight loads are in too)
    __syncthreads();  // every wave's rows before any activation load
}

// ------------------------------------------------------------------ STORE
// y[p][n] = sum_k x[p][k] w[n][k] for the tile's rows p; wave w owns weight
// rows 256 ctile + 64 w + 32 ct + l32 (rows past ncols read zeros past the
// matrix's resource or unused bytes, and are not stored).
template <int WT, int BM>
__global__ void __launch_bounds__(G4_THREADS)
    __attribute__((amdgpu_waves_per_eu(BM == G4_BM_TINY ? 4 : BM == G4_BM_MID ? 2 : 1, BM == G4_BM ? 1 : BM == G4_BM_TINY ? 4 : BM == G4_BM_MID ? 2 : 3)))
    k_g4_store(G2Args g) {
    constexpr int NA = BM >= 32 ? BM / 32 : 1, TR = BM < 32 ? BM : 0;
    __shared__ __attribute__((aligned(1024))) _Float16 As0[BM * G4_SK];
    __shared__ __attribute__((aligned(1024))) _Float16 As1[BM * G4_SK];
    __shared__ __attribute__((aligned(1024))) uint8_t Ws[G4_WAVES][g4_wregion<WT>()];
    int tile, ctile;
    g4_coords((int)((g.ncols + G4_NWG - 1) / G4_NWG), tile, ctile);
    const bool self = BM <= G4_BM_SMALL && g.ids != nullptr;
    int my_p = -1;
    const G4Tile t = self ? g4_self_tile<BM>(g, tile, (int *)As0, my_p) : g4_desc(g, tile);
    g4_clock(g, 0, t.live);
    if (!t.live) {
        g4_clock(g, 1, false);
        return;
    }
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int l32 = lane & 31, g2 = lane >> 5;
    if (!self) my_p = g4_rows_load(g, t);
    const int nrt = __builtin_amdgcn_readfirstlane(t.nrt);
    const uint32_t Kin = (uint32_t)g.a.K;
    const rsrc_t rx = g4_rsrc(g.xh, g.xrows * (int64_t)Kin * 2);
    const uint8_t *mat = g.a.data + (int64_t)t.e * g.a.mat_bytes;
    const uint32_t mis = WT == 14 ? (uint32_t)((uintptr_t)mat & 3u) : 0u;   // (WT 15: the tiled Q6_K copy)
    const rsrc_t r = g4_rsrc(mat - mis, g.a.mat_bytes + mis);
    const uint32_t rb = (uint32_t)g.a.row_bytes;
    const int n0 = ctile * G4_NWG + 64 * wave;
    const int64_t rowbase[2] = {n0, n0 + 32};
    const G4WDma<WT> dm = g4_wdma<WT>(r, r, rowbase, rb, mis, lane, WT == 12 && g.tiled != 0);
    g4_issue_w0<WT>(dm, Ws[wave]);
    u32x4 sn[2];
    if constexpr (WT == 15) {
        sn[0] = g4_load_s15(dm, 0, 0);
        sn[1] = g4_load_s15(dm, 1, 0);
    }
    int *s_arow = (int *)As1;   // as in k_g4_glu
    g4_rows_publish<BM>(g, my_p, s_arow);
    if constexpr (BM <= G4_BM_SMALL) {
        if (g.q8src) g4_q8_rows<WT == 12 ? XO_Q4 : XO_Q6>(g, t.mrows, s_arow, ctile == 0, wave, lane);
    }
    // byte offset of the lane's own rows (Q6_K block alignment)
    const uint32_t wsh[2] = {mis + (uint32_t)(n0 + l32) * rb, mis + (uint32_t)(n0 + 32 + l32) * rb};
    f32x16 acc[NA][2];
    g4_kloop<WT, NA, TR>(rx, s_arow, 2u * Kin, dm, wsh, Ws[wave], (int)(Kin / QK), wave, lane, nrt, As0, As1, acc, sn);
    __builtin_amdgcn_s_waitcnt(0);   // no load may land in LDS after the work-group ends
    // rows 32 rt + 8 (i / 4) + 4 g2 + i % 4, columns n0 + 32 ct + l32
    if (g.yh) {
        // fp16 out through LDS: the wave's columns of every row into the
        // activation buffers (rows 0-95 in As0, 96-191 in As1, 512 bytes per
        // row), then whole 512-byte rows out in 16-byte pieces (full lines
        // instead of 64-byte runs); the row table lives in the weight region
        const int *s_p = g4_publish_rows<BM>((_Float16 *)&Ws[0][0], my_p);
        bool over = false;
#pragma unroll
        for (int rt = 0; rt < NA; ++rt) {
            if (rt >= nrt) break;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                if (BM < 32 && 8 * (i >> 2) >= BM) continue;   // (rows past a tiny tile's)
                const int m = 32 * rt + 8 * (i >> 2) + 4 * g2 + (i & 3);
                _Float16 *row = m < (BM / 2) ? As0 + m * G4_NWG : As1 + (m - (BM / 2)) * G4_NWG;
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) {
                    const float v = acc[rt][ct][i];
                    over = over || fabsf(v) > kF16Max;
                    row[64 * wave + 32 * ct + l32] = f16_sat(v);
                }
            }
        }
        if (__ballot(over) != 0 && lane == 0 && g.range_total) atomicAdd(g.range_total, 1);
        __syncthreads();
        for (int idx = threadIdx.x; idx < t.mrows * (G4_NWG / 8); idx += G4_THREADS) {
            const int r = idx / (G4_NWG / 8), c = idx % (G4_NWG / 8);
            const _Float16 *row = r < (BM / 2) ? As0 + r * G4_NWG : As1 + (r - (BM / 2)) * G4_NWG;
            *(uint4 *)(g.yh + (int64_t)s_p[r] * g.ldy + (int64_t)ctile * G4_NWG + 8 * c) = *(const uint4 *)(row + 8 * c);
        }
    } else {
        const int *s_p = g4_publish_rows<BM>(As0, my_p);
#pragma unroll
        for (int rt = 0; rt < NA; ++rt) {
            if (rt >= nrt) break;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int m = 32 * rt + 8 * (i >> 2) + 4 * g2 + (i & 3);
                if (m < t.mrows) {
                    float *yr = g.y + (int64_t)s_p[m] * g.ldy + n0 + l32;
#pragma unroll
                    for (int ct = 0; ct < 2; ++ct)
                        if (n0 + 32 * ct + l32 < g.ncols) yr[32 * ct] = acc[rt][ct][i];
                }
            }
        }
    }
    g4_clock(g, 1, true);
}

// ------------------------------------------------------------------ launch
int gemm4_grid(const G2Args &g) {
    const int ntile8 = (g.max_tiles + 7) / 8;
    const int nct = g.glu ? (int)(g.I / 128) : (int)((g.ncols + G4_NWG - 1) / G4_NWG);
    return 8 * nct * ntile8;
}

int launch_gemm4(const G2Args &g, hipStream_t st) {
    if (g.max_tiles <= 0) return 0;
    if (g.a.K % QK) return -6;
    if (g.ids && ((g.bm != G4_BM_SMALL && g.bm != G4_BM_TINY) || g.nids <= 0 || g.nids > G4_SD_IDS ||
                  g.n_expert <= 0 || g.n_expert > G4_THREADS))
        return -6;
    if (g.bm == G4_BM_TINY && !g.ids) return -6;   // tiny tiles only without a dispatch
    if (g.bm != G4_BM && g.bm != G4_BM_MID && g.bm != G4_BM_SMALL && g.bm != G4_BM_TINY) return -6;
    const int64_t lim = 0x7fffffff;
    // byte offsets of the buffer loads are 32-bit
    if (g.xrows <= 0 || g.xrows * g.a.K * 2 > lim || g.a.mat_bytes + 4 > lim) return -6;
    // tiled: whole 32-row groups, matrices without padding between them
    // (Q6_K: the down product only, 288 bytes per 256 values)
    if (g.tiled && g.a.type == 14 &&
        (g.glu || g.a.N % 32 || g.a.row_bytes != Q6X_ROW_BYTES * (g.a.K / QK) ||
         g.a.mat_bytes != g.a.N * g.a.row_bytes))
        return -6;
    if (g.tiled && g.a.type != 14 && (g.a.type != 12 || g.a.N % 32 || g.a.mat_bytes != g.a.N * g.a.row_bytes ||
                    (g.glu && !g.fused &&
                     (g.b.type != 12 || g.b.N % 32 || g.b.mat_bytes != g.b.N * g.b.row_bytes))))
        return -6;
    if (g.q8src && (g.glu || g.bm > G4_BM_SMALL || g.q8ld % 4 || (uintptr_t)g.q8src % 8 || (uintptr_t)g.xh % 16))
        return -6;
    const int ntile8 = (g.max_tiles + 7) / 8;
    if (g.glu) {
        // GLU values out (fp32 to y or fp16 to yh, ldy); the work-group covers
        // 128 act columns
        if (g.a.type != 12 || (g.I % 128)) return -6;
        if (g.yh ? (g.ldy % 8 || (uintptr_t)g.yh % 16) : (g.ldy % 4 || (uintptr_t)g.y % 16)) return -6;
        if (!g.fused && (g.b.mat_bytes > lim || g.b.type != 12 || g.b.row_bytes != g.a.row_bytes)) return -6;
        if ((uintptr_t)g.a.data % 4 || g.a.mat_bytes % 4 || g.a.row_bytes % 4) return -6;
        if (!g.fused && ((uintptr_t)g.b.data % 4 || g.b.mat_bytes % 4)) return -6;
        const int nct = (int)(g.I / 128);
        const dim3 grid((unsigned)(8 * nct * ntile8));
        if (g.bm == G4_BM_TINY) hipLaunchKernelGGL(k_g4_glu<G4_BM_TINY>, grid, dim3(G4_THREADS), 0, st, g);
        else if (g.bm == G4_BM_SMALL) hipLaunchKernelGGL(k_g4_glu<G4_BM_SMALL>, grid, dim3(G4_THREADS), 0, st, g);
        else if (g.bm == G4_BM_MID) hipLaunchKernelGGL(k_g4_glu<G4_BM_MID>, grid, dim3(G4_THREADS), 0, st, g);
        else hipLaunchKernelGGL(k_g4_glu<G4_BM>, grid, dim3(G4_THREADS), 0, st, g);
    } else {
        const int nct = (int)((g.ncols + G4_NWG - 1) / G4_NWG);
        const dim3 grid((unsigned)(8 * nct * ntile8));
        if (g.yh && (g.ncols % G4_NWG || g.ldy % 8 || (uintptr_t)g.yh % 16)) return -6;
        const bool sm = g.bm == G4_BM_SMALL, mid = g.bm == G4_BM_MID;
        if (g.a.type == 12) {
            if ((uintptr_t)g.a.data % 4 || g.a.mat_bytes % 4 || g.a.row_bytes % 4) return -6;
            if (g.bm == G4_BM_TINY) hipLaunchKernelGGL((k_g4_store<12, G4_BM_TINY>), grid, dim3(G4_THREADS), 0, st, g);
            else if (sm) hipLaunchKernelGGL((k_g4_store<12, G4_BM_SMALL>), grid, dim3(G4_THREADS), 0, st, g);
            else if (mid) hipLaunchKernelGGL((k_g4_store<12, G4_BM_MID>), grid, dim3(G4_THREADS), 0, st, g);
            else hipLaunchKernelGGL((k_g4_store<12, G4_BM>), grid, dim3(G4_THREADS), 0, st, g);
        } else if (g.bm == G4_BM_TINY) {
            return -6;   // (tiny tiles: Q4_K down tables only)
        } else if (g.a.type == 14 && g.tiled) {
            if ((uintptr_t)g.a.data % 16) return -6;
            if (sm) hipLaunchKernelGGL((k_g4_store<15, G4_BM_SMALL>), grid, dim3(G4_THREADS), 0, st, g);
            else if (mid) hipLaunchKernelGGL((k_g4_store<15, G4_BM_MID>), grid, dim3(G4_THREADS), 0, st, g);
            else hipLaunchKernelGGL((k_g4_store<15, G4_BM>), grid, dim3(G4_THREADS), 0, st, g);
        } else if (g.a.type == 14) {
            if (sm) hipLaunchKernelGGL((k_g4_store<14, G4_BM_SMALL>), grid, dim3(G4_THREADS), 0, st, g);
            else if (mid) hipLaunchKernelGGL((k_g4_store<14, G4_BM_MID>), grid, dim3(G4_THREADS), 0, st, g);
            else hipLaunchKernelGGL((k_g4_store<14, G4_BM>), grid, dim3(G4_THREADS), 0, st, g);
        } else {
            return -3;
        }
    }
    return hip_check_launch();
}

}  // namespace mimoe
