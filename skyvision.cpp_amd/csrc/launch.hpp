// launch.hpp - host-side launchers of the MoE kernels (one per kernel family)
// and the shared HIP error bookkeeping.  Every launcher returns 0 or a
// negative mi_moe_status.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "norm.hpp"

namespace mimoe {

// tile rows and longest K of the skinny grouped products (k_gs.hip)
constexpr int GS_BM = 16;
constexpr int GS_KMAX = 2048;

// records the HIP error string for mi_last_hip_error(); returns MI_MOE_ERR_HIP (-5)
int record_hip_error(hipError_t e);
// check hipGetLastError() after a launch
int hip_check_launch();

// ---- data preparation (k_data.hip)
int launch_fill_normal(float *out, int64_t n, uint64_t seed, uint64_t stream, float mean, float sd,
                       hipStream_t st);
int launch_quantize(int type, const float *src, void *dst, int64_t nblocks, hipStream_t st);
// dst = n_mat Q4_K matrices of rows (a multiple of 32) rows of rb bytes in
// the tiled order of the grouped GEMMs (G2Args::tiled); 16-byte aligned
int launch_tile_q4k(const void *src, void *dst, int64_t n_mat, int64_t rows, int64_t rb, hipStream_t st);
// dst = n_mat Q6_K matrices of rows (a multiple of 32) rows of rb bytes in
// the down GEMM's tiled order (9216 bytes per 32-row group and block)
int launch_tile_q6k(const void *src, void *dst, int64_t n_mat, int64_t rows, int64_t rb, hipStream_t st);
constexpr int Q6X_ROW_BYTES = 288;   // bytes per 256 values of a row in the Q6_K tiled order
// y = x / sqrt(mean(x^2) + eps) per row of D (x may equal y)
int launch_rmsnorm(const float *x, int64_t T, int D, float eps, float *y, hipStream_t st);
// y = norm(x) per row of D <= 4096 (norm.hpp; x may equal y)
int launch_norm(const NormParams &p, const float *x, int64_t T, int D, float *y, hipStream_t st);

// ---- routing (k_route.hip)
struct Q8Out {
    int8_t *q8 = nullptr;        // [rows][K] natural order (GEMV path)
    float *d8 = nullptr;         // [rows][K/256]
    int16_t *bsums = nullptr;    // [rows][K/16]
    _Float16 *xh = nullptr;      // [rows][K] fp16(d*q) in MFMA K order of wtype (GEMM path)
    int wtype = 12;              // consumer weight type for xh order
    int order = 0;               // 0: 16x16x32 K order, 1: 32x32x16 K order
    int exact = 0;               // 1: xh holds the codes q (exact), d8 and xbs the scales / block sums
    _Float16 *xbs = nullptr;     // [rows][K/16] block sums of 16 codes, as fp16 (exact)
    int pre_act = 0;             // 4 (ACT_RELU_SQR): quantize relu(v)^2 instead of v
    int32_t *range_total = nullptr;   // [1] or null: blocks whose xh saturated at the fp16 range
};
// quantize rows of src (row r at src + r*ld values, fp32 or fp16) to Q8_K
int launch_q8k_rows(const float *src, int64_t ld, int64_t nrows, int64_t K, const Q8Out &o, hipStream_t st);
int launch_q8k_rows(const _Float16 *src, int64_t ld, int64_t nrows, int64_t K, const Q8Out &o, hipStream_t st);
// router logits, fixed fp64 order; W: [E][D], x rows at x + t*ldx
int launch_router(const float *W, const float *b, const float *x, int64_t ldx, int64_t T, int D, int E,
                  float *logits, hipStream_t st);
// router logits plus (qx) the Q8_K of the x rows in one launch; -6 when the
// shape is outside the kernel (D > 2048, or qx with D % 256)
int launch_front(const float *W, const float *b, const float *x, int64_t ldx, int64_t T, int D, int E,
                 float *logits, const Q8Out *qx, hipStream_t st);
// top-k (descending, ties -> lower id) and softmax over the selected logits;
// w may be NULL (op-level top_k)
struct Gating;
int launch_topk_softmax(const float *logits, int64_t ld_logits, int64_t T, int E, int K, int32_t *sel,
                        int64_t ld_sel, float *w, hipStream_t st, const Gating &gt);
// small batches: the router's chunk partials parts[D / 64][T][E] (fp64) by
// tiles split over the chunks (cps chunks per work-group) plus (qx) the Q8_K
// of x; then the logits (chunk order, + b) and the top-k / softmax of
// launch_topk_softmax from them (logits [T][E] written too; E <= 128)
int launch_front_parts(const float *W, const float *x, int64_t ldx, int64_t T, int D, int E, int cps,
                       double *parts, const Q8Out *qx, hipStream_t st);
int launch_topk_parts(const double *parts, int D, const float *bias, float *logits, int64_t T, int E, int K,
                      int32_t *sel, int64_t ld_sel, float *w, hipStream_t st, const Gating &gt);

struct Dispatch {
    int32_t *counts;     // [E]
    int32_t *offsets;    // [E+1]
    int32_t *perm;       // [T*K] value t*K+k, per expert token-ascending
    int32_t *tile_e;     // [max_tiles] expert of each GEMM M-tile
    int32_t *tile_r0;    // [max_tiles] first list row of each tile (within its expert's list)
    int32_t *tile_start; // [max_tiles] its first row in perm (offsets[e] + tile_r0)
    int32_t *tile_rows;  // [max_tiles] its row count
    int32_t *tile_perm;  // or null: [max_tiles][GS_BM] the tile's perm entries (balanced tiles of at most GS_BM rows)
    int32_t *n_tiles;    // [1]
    int32_t *active_e;   // [E] experts with count > 0, ascending
    int32_t *n_active;   // [1]
    int32_t *bad_ids;    // [1] number of ids outside [0, E) (skipped)
    int32_t *bad_total;  // [1] or null: running count of such ids (never reset by the kernel)
    float *zero_rows;    // or null: row p (p = flat id index) of zero_n floats at zero_rows + p * zero_ld
    int64_t zero_ld, zero_n;   // is zeroed for every id outside [0, E)
};
// balanced = 0: per expert floor(cnt / BM) full tiles, then one partial tile
// per expert with cnt % BM rows (largest first); balanced = 1: per expert
// ceil(cnt / BM) tiles of equal size (the first cnt % n one row longer), in
// expert order
int launch_dispatch(const int32_t *ids, int64_t T, int K, int E, int BM, int balanced, const Dispatch &d,
                    hipStream_t st);

// out[t][n] = res[t][n] + (sum_k (double)(z[t*K+k][n] * w[t][k]) + add[t][n])   (res, add may be NULL)
// ids_a / ids_b (or null): slot k of token t is live only if both ids lie in
// [0, E); dead slots add nothing
struct CombineIds {
    const int32_t *a = nullptr, *b = nullptr;
    int E = 0;
};
// z: fp32 slot rows, or (z == NULL) fp16 slot rows zh
int launch_combine(const float *z, const float *w, const float *res, float *out, int64_t T, int K, int D,
                   hipStream_t st, const CombineIds &ids = CombineIds{}, const float *add = nullptr,
                   const _Float16 *zh = nullptr);
// shared expert's routing: ids[t] = 0, w[t] = logit ? fl32(1 / (1 + exp(-logit[t]))) (fp64) : 1
int launch_shared_gate(const float *logit, int64_t T, int32_t *ids, float *w, hipStream_t st);

// ---- expert products
struct ExpertMat {
    const uint8_t *data;  // E matrices
    int type;             // 12 Q4_K, 14 Q6_K, 0 F32
    int64_t row_bytes;    // nb[1]
    int64_t mat_bytes;    // nb[2]
    int64_t K;            // ne[0]
    int64_t N;            // ne[1]
};

// epilogue modes of the grouped products
enum { EPI_STORE = 0, EPI_GLU = 1 };

struct GemvArgs {
    ExpertMat a;          // gate (or fused gate|up) / down / generic
    ExpertMat b;          // up (separate gate/up GLU); data == nullptr when fused
    int epi;              // EPI_STORE: y[p][n]; EPI_GLU: act[p][i]
    int act;              // mi_act for EPI_GLU
    int64_t I;            // GLU width (output columns)
    int fused;            // gate holds [h | g] rows
    // activations (Q8_K rows)
    const int8_t *q8;
    const float *d8;
    const int16_t *bsums;
    int ne11;             // 1: row = t; else row = t*K + k
    int K;                // slots per token
    // dispatch
    const int32_t *counts, *offsets, *perm, *active_e, *n_active;
    int max_active;
    // output rows p = t*K + k, row stride ldy floats
    float *y;
    int64_t ldy;
    int64_t ncols;        // N (EPI_STORE) or I (EPI_GLU)
};
int launch_gemv(const GemvArgs &g, hipStream_t st);

struct GemmArgs {
    ExpertMat a;          // gate (or fused gate|up) / down / generic
    ExpertMat b;          // up (separate gate/up); data == nullptr when fused
    int epi;
    int act;
    int64_t I;
    int fused;
    const _Float16 *xh;   // activations fp16 in MFMA K order of a.type
    int ne11;
    int K;
    const int32_t *counts, *offsets, *perm, *tile_e, *tile_r0, *n_tiles;
    int max_tiles;
    // EPI_STORE output: fp32 rows p, stride ldy
    float *y;
    int64_t ldy;
    // EPI_GLU output: Q8_K-quantized activations as fp16 in the MFMA K order
    // of `next_type`, rows p, stride I
    _Float16 *acth;
    int next_type;
    int64_t ncols;
    int32_t *range_total;   // [1] or null: activation blocks saturated at the fp16 range
};
constexpr int GEMM_BM = 64;
int launch_gemm(const GemmArgs &g, hipStream_t st);

// 4-wave grouped GEMMs on 32x32x16 MFMA (k_gemm4.hip), tiles of at most
// G4_BM rows from a balanced dispatch.  Both take fp16 activations in the
// weight type's 32x32x16 MFMA K order (xh; xd, xbs, acth and next_type are
// not read).  glu = 1: Q4_K gate/up (fused [h | g] or separate), writes the
// GLU rows (fp32 to y or fp16 to yh, ldy), whose Q8_K the caller computes
// (launch_q8k_rows) for the down product; glu = 0: Q4_K / Q6_K product, rows
// to y (fp32) or yh (fp16).
struct G2Args {
    ExpertMat a;
    ExpertMat b;
    int glu, fused, act;
    int64_t I;
    const _Float16 *xh;
    const float *xd;
    const _Float16 *xbs;
    int ne11, K;
    const int32_t *counts, *offsets, *perm, *tile_e, *tile_r0, *n_tiles;
    const int32_t *tile_start, *tile_rows;   // the tiles' perm starts and row counts
    const int32_t *tile_perm;                // skinny products: [max_tiles][GS_BM] the tiles' perm entries
    int max_tiles;
    int bm;               // tile rows of the dispatch: G4_BM, G4_BM_MID, or G4_BM_SMALL (few rows
                          // per expert), or G4_BM_TINY (with ids)
    // or NULL: with bm = G4_BM_SMALL or G4_BM_TINY, no dispatch launch - every work-group
    // derives its tile (the balanced dispatch's) from the call's nids <= 1024
    // flat expert ids in [0, n_expert), n_expert <= 256; the dispatch
    // pointers above are then not read
    const int32_t *ids;
    int nids, n_expert;
    // or NULL: with bm <= G4_BM_SMALL and glu = 0, the activation rows xh of
    // the tile are first made by its work-groups - the Q8_K of these fp16
    // rows [.][q8ld] (the down product's GLU rows) in xh's order, the same
    // bits the separate Q8_K pass writes (work-groups of column tile 0 count
    // its saturations)
    const _Float16 *q8src;
    int64_t q8ld;
    // 1: a (and b) hold tables in the tiled order (launch_tile_q4k: the 32
    // rows of a column tile give block b as 4608 contiguous bytes, the LDS
    // image of one column tile's weight loads; launch_tile_q6k: 9216 bytes,
    // the merged codes' LDS image and the lanes' fp16 scales)
    int tiled;
    int64_t xrows;        // rows of xh (glu = 1: tokens)
    float *y;
    int64_t ldy;
    _Float16 *acth;
    int next_type;
    int64_t ncols;
    // or NULL: y written as fp16 here instead, saturated at the fp16 range
    // (waves that saturate are counted in range_total); needs ldy % 8 == 0, a
    // 16-byte aligned yh and, for glu = 0, ncols % 256 == 0
    _Float16 *yh;
    int32_t *range_total;
    // profiling only (else NULL): per work-group {shader clock, wall clock} at
    // its start and end, 4 words per work-group of the grid (dead ones write 0)
    uint64_t *clk;
    int clk_n;            // work-groups clk holds
};
constexpr int G4_BM = 192;
constexpr int G4_BM_SMALL = 32;   // tiles of few rows per expert (G2Args::bm)
constexpr int G4_BM_MID = 64;     // two work-groups per CU (G2Args::bm; Q4_K weights)
constexpr int G4_BM_TINY = 8;     // tiles of at most 8 rows (G2Args::bm; only with ids: no dispatch launch)
constexpr int G4_SD_IDS = 1024;    // most ids of a call whose GEMM work-groups find their tiles themselves (G2Args::ids)
int launch_gemm4(const G2Args &g, hipStream_t st);
int gemm4_grid(const G2Args &g);   // work-groups launch_gemm4 launches

// Skinny grouped Q4_K products (k_gs.hip) on tiles of at most GS_BM rows
// from a balanced dispatch (G2Args::bm = GS_BM), same arguments and outputs
// as launch_gemm4 (glu = 1: the GLU rows; glu = 0: the plain product, whose
// ncols must be a multiple of 16); K <= GS_KMAX.  splits: work-groups per
// tile, each taking an equal share of the tile's 16-column groups.
int launch_gemm_gs(const G2Args &g, int splits, hipStream_t st);
// waves per work-group and work-groups per CU of the skinny products (glu: gate/up)
int gemm_gs_waves(int glu);
int gemm_gs_wgs_per_cu(int glu);

// ---- 32-value block formats (Q4_0 = 2, Q5_0 = 6, Q8_0 = 8) and F16 (1)
// expert tables (k_b32.hip)
// weight rows of 32-value blocks (F16: 32 values per "block"), bit for bit the
// CPU oracle's ggml _ref quantizers / fp16 rounding
int launch_quantize_b32(int type, const float *src, void *dst, int64_t nblocks, hipStream_t st);
// the activation operands of one consumer weight type
enum { B32_PREP_CODES = 0, B32_PREP_DQ = 1, B32_PREP_F16 = 2 };
struct B32Prep {
    int mode;                  // CODES: Q8_0 codes + scales (GEMV of Q4_0/Q5_0/Q8_0); DQ: fp16(d q) rows
                               // (their GEMM); F16: fp16(x) rows (F16 tables, both paths)
    int8_t *q8 = nullptr;      // CODES: [rows][K]
    uint16_t *dh = nullptr;    // CODES: [rows][K/32] fp16 scale bits
    _Float16 *xh = nullptr;    // DQ / F16: [rows][K]
    int pre_act = 0;           // 4 (ACT_RELU_SQR): relu(v)^2 first
};
int launch_prep_b32(const float *src, int64_t ld, int64_t nrows, int64_t K, const B32Prep &o, hipStream_t st);
struct B32Args {
    ExpertMat a, b;            // b: up table (separate gate/up GLU), else unused
    int glu, fused, act;
    int64_t I;
    const int8_t *q8;          // GEMV of Q4_0/Q5_0/Q8_0: Q8_0 codes [rows][K] and
    const uint16_t *dh;        //   fp16 scales [rows][K/32]
    const _Float16 *xh;        // GEMM (and F16 GEMV): fp16 rows [rows][K]
    int ne11, K;
    const int32_t *counts, *offsets, *perm, *active_e, *n_active;   // GEMV
    int max_active;
    const int32_t *tile_e, *tile_start, *tile_rows, *n_tiles;       // GEMM: balanced tiles of G4_BM rows
    int max_tiles;
    float *y;                  // rows p (glu: act rows [p][I]), stride ldy
    int64_t ldy, ncols;
};
int launch_gemv_b32(const B32Args &g, hipStream_t st);
int launch_gemm_b32(const B32Args &g, hipStream_t st);

// Single-token MoE block in one kernel (k_decode.hip).
struct DecArgs {
    const float *rw, *rb, *x;     // router W [E][D], bias [E] or NULL, tokens [T][D]
    int D, E, K, I;
    int T;                        // tokens (k_decode1: 1; k_decodeb: 2 .. DECB_T_MAX)
    ExpertMat gate, up, down;     // Q4_K gate (or fused [h | g]) / up; Q4_K or Q6_K down
    int fused, act;
    const float *res;             // [T][D] or NULL
    float *out;                   // [T][D]
    int P, C;                     // (h, g) row pairs per WG; down columns per WG (k_decodeb: per C unit)
    // workspace / routing outputs
    float *logits;                // [T][E]
    int32_t *sel;                 // [T][K]
    float *w;                     // [T][K]
    int32_t *counts, *offsets, *perm;
    int8_t *xq;                   // Q8_K of x: codes [T][D], scales [T][D/256], block sums [T][D/16]
    float *xd;
    int16_t *xbs;
    float *actf;                  // GLU output fp32 [T K][I]
    uint64_t *tw;                 // epoch-tagged logits [E] and gate/up unit completions, launch counters
    uint64_t *tw2;                // k_decodeb's epoch-tagged unit words (decodeb_tw_words)
    uint32_t *epoch;              // [grid] per-WG launch epochs
    unsigned *err;                // set when a wait gave up (output is NaN)
    unsigned rescue_polls;        // polls for another WG's unit before computing it here
    NormParams norm;              // k_decode1: the norm of x applied in the kernel (kind NORM_NONE: x as given)
};
constexpr int DEC_MAX_GRID = 1024;
// epoch-tagged words: the E router logits, then one per gate/up unit
constexpr int DEC_TW_LOGIT = 0, DEC_TW_BDONE = 256;
constexpr int DEC_TW_WORDS = DEC_TW_BDONE + DEC_MAX_GRID;
constexpr unsigned DEC_RESCUE_POLLS = 64;
constexpr int DEC_LIMIT_GU_BYTES = 9 * 1024;   // LDS per wave of gate/up rows
constexpr int DEC_LIMIT_DN_BYTES = 7 * 1024;   // LDS per slot of down rows
constexpr int DEC_LIMIT_UNPACKED_BYTES = 10 * 1024;   // LDS per slot of dot-ready down rows
// k_decodeb: 2 .. DECB_T_MAX tokens in one kernel (plain launch, no
// co-residency needed: as k_decode1)
constexpr int DECB_T_MAX = 16;
// words of tw2 for T tokens (A units E T + T D/256, then I/4 per distinct expert)
constexpr int64_t decodeb_tw_words(int64_t T, int64_t D, int64_t E, int64_t K, int64_t I) {
    return E * T + T * (D / 256) + T * K * (I / 4);
}
int launch_decodeb(const DecArgs &g, int grid, hipStream_t st);
// a plain launch of one WG per CU (the kernel needs no co-residency: a WG
// computes any unit it waited too long for)
int launch_decode1(const DecArgs &g, int grid, hipStream_t st);
// work-groups of the decode grid (one per CU), 0 if one per CU cannot be resident
int decode1_max_grid(int device, int *grid);

}  // namespace mimoe
