// api.cpp - the C ABI (include/mi_moe.h, include/mi_moe_util.h).
//
// Validates arguments the way the reference's graph builders do
// (moe_compute.cpp:102-120: bad shapes / types -> error, nothing enqueued),
// then enqueues the kernel chain on the caller's stream:
//   router -> top-k/softmax -> dispatch -> Q8_K(x) -> gate/up (+GLU, +Q8_K)
//   -> down -> weighted combine (+residual)
// Decode-sized calls use the grouped integer-dot GEMV kernels, larger calls
// the grouped MFMA GEMM kernels (use_gemm: by default from half a dispatched
// row per expert on average for Q4_K / Q6_K tables, use_gemm_wide: from 1.25
// for the others).
// All workspace comes from mi_moe_ctx_reserve; forward calls never allocate.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <atomic>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/mi_moe.h"
#include "../../include/mi_moe_util.h"
#include "common.hpp"
#include "launch.hpp"
#include "wave_ops.hpp"

namespace mimoe {
int launch_mm_id_f32(const GemvArgs &g, const float *b, int64_t ldb, hipStream_t st);
int launch_glu_rows(const float *h, int64_t ldh, const float *gg, int64_t ldg, float *out, int64_t ldo,
                    int64_t rows, int64_t I, int act, hipStream_t st);

static thread_local std::string g_last_error;

int record_hip_error(hipError_t e) {
    g_last_error = hipGetErrorString(e);
    return MI_MOE_ERR_HIP;
}
int hip_check_launch() {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : record_hip_error(e);
}
}  // namespace mimoe

using namespace mimoe;

#define HIP_TRY(x)                                         \
    do {                                                   \
        const hipError_t e_ = (x);                         \
        if (e_ != hipSuccess) return record_hip_error(e_); \
    } while (0)
#define TRY(x)                \
    do {                      \
        const int r_ = (x);   \
        if (r_) return r_;    \
    } while (0)

namespace {

constexpr int kMaxStages = 16;
constexpr int kClkWGs = 16384;   // clock records per GEMM launch (profiling)

struct ActBuf {                // one Q8_K activation set
    int8_t *q8 = nullptr;
    float *d8 = nullptr;
    int16_t *bs = nullptr;
    _Float16 *h = nullptr;
    _Float16 *bsh = nullptr;   // block sums as fp16 (exact MFMA path)
};

struct DispBuf {
    int32_t *counts, *offsets, *perm, *tile_e, *tile_r0, *tile_start, *tile_rows, *tile_perm, *n_tiles, *active_e,
        *n_active, *bad;
    int32_t *bad_total;   // the context's running count (mi_moe_ctx_take_errors)
    Dispatch view() const {
        Dispatch d;
        d.counts = counts; d.offsets = offsets; d.perm = perm; d.tile_e = tile_e; d.tile_r0 = tile_r0;
        d.tile_start = tile_start; d.tile_rows = tile_rows; d.tile_perm = tile_perm;
        d.n_tiles = n_tiles; d.active_e = active_e; d.n_active = n_active; d.bad_ids = bad;
        d.bad_total = bad_total; d.zero_rows = nullptr; d.zero_ld = 0; d.zero_n = 0;
        return d;
    }
};

}  // namespace

struct mi_moe_ctx {
    int device = 0;
    bool reserved = false;
    int64_t cap_T = 0;
    int32_t cap_D = 0, cap_I = 0, cap_E = 0, cap_K = 0;
    int64_t cap_rows = 0, cap_kmax = 0, cap_tiles = 0;
    int64_t cap_z = 0;   // floats of z
    void *ws = nullptr;
    size_t ws_bytes = 0;

    float *logits = nullptr;
    int32_t *sel = nullptr;
    float *w = nullptr;
    float *xn = nullptr;      // [cap_T][D] normalized rows where a norm cannot be fused
    DispBuf disp[2];
    ActBuf ax, aact;
    float *f1 = nullptr;      // [rows][max(2I, kmax)]  GLU / F32 scratch
    float *f2 = nullptr;      // [rows][I]
    float *z = nullptr;       // [rows][max(D, 2I)]
    // shared expert: its output [cap_T][D], routing (all tokens -> expert 0) and gate row
    float *sh_out = nullptr, *sh_w = nullptr, *sh_logit = nullptr;
    int32_t *sh_ids = nullptr;
    int32_t *bad_total = nullptr;   // caller ids outside [0, E) since the last take
    int32_t *range_total = nullptr; // GEMM-path Q8_K blocks saturated at the fp16 range
    int64_t gemm_threshold = 0;   // 0: the shape rule of use_gemm
    int gemm_tiles = 0;           // Q4_K GEMM row tiles: 0 by shape, 1 G4_BM, 2 G4_BM_SMALL, 3 GS_BM (k_gs), 4 G4_BM_TINY, 5 G4_BM_MID
    int n_cu = 0;                 // compute units of the device
    // single-token fused kernel (k_decode.hip)
    int fused_decode = MI_DECODE_FUSED;
    int dec_grid = 0;          // fused decode grid (one WG per CU), 0: unavailable
    uint64_t *dec_tw = nullptr;
    uint32_t *dec_epoch = nullptr;
    unsigned dec_rescue_polls = DEC_RESCUE_POLLS;
    unsigned *dec_err = nullptr;
    // batched fused kernel (k_decodeb): its unit words
    uint64_t *decb_tw = nullptr;
    int64_t decb_words = 0;

    bool profiling = false;
    hipEvent_t ev[kMaxStages + 1] = {};
    const char *stage_name[kMaxStages] = {};
    int n_stages = 0;
    hipStream_t prof_stream = nullptr;
    // profiling: per-work-group clock records of the two grouped GEMMs
    // (gate_up, down) of the last forward on the 4-wave GEMM path
    uint64_t *clk = nullptr;        // [2][kClkWGs][4]
    int clk_grid[2] = {0, 0};       // work-groups the last launch recorded, 0: none
};

namespace {

void stage_begin(mi_moe_ctx *c, hipStream_t st) {
    if (!c->profiling) return;
    c->n_stages = 0;
    c->clk_grid[0] = c->clk_grid[1] = 0;
    c->prof_stream = st;
    (void)hipEventRecord(c->ev[0], st);
}
void stage_end(mi_moe_ctx *c, const char *name, hipStream_t st) {
    if (!c->profiling || c->n_stages >= kMaxStages) return;
    c->stage_name[c->n_stages] = name;
    c->n_stages++;
    (void)hipEventRecord(c->ev[c->n_stages], st);
}

// profiling: point the GEMM's clock records at the context's buffer k
void prof_clock(mi_moe_ctx *c, G2Args &g, int k) {
    if (!c->profiling || !c->clk) return;
    g.clk = c->clk + (size_t)k * 4 * kClkWGs;
    g.clk_n = kClkWGs;
    c->clk_grid[k] = gemm4_grid(g);
}

bool is_kquant(int t) { return t == MI_TYPE_Q4_K || t == MI_TYPE_Q6_K; }
// 32-value block formats and F16: the k_b32.hip kernels
bool is_b32(int t) { return t == MI_TYPE_Q4_0 || t == MI_TYPE_Q5_0 || t == MI_TYPE_Q8_0; }
bool is_b32f(int t) { return is_b32(t) || t == MI_TYPE_F16; }
// the table families one layer's products may mix: 0 F32, 1 k-quants, 2 the b32 / F16 family
int type_family(int t) { return is_kquant(t) ? 1 : is_b32f(t) ? 2 : 0; }

size_t type_row_size(int32_t type, int64_t n) {
    switch (type) {
    case MI_TYPE_F32: return (size_t)n * 4;
    case MI_TYPE_F16: return (size_t)n * 2;
    case MI_TYPE_Q4_K: return n % QK ? 0 : (size_t)(n / QK) * Q4K_BYTES;
    case MI_TYPE_Q6_K: return n % QK ? 0 : (size_t)(n / QK) * Q6K_BYTES;
    case MI_TYPE_Q4_0: return n % 32 ? 0 : (size_t)(n / 32) * 18;
    case MI_TYPE_Q5_0: return n % 32 ? 0 : (size_t)(n / 32) * 22;
    case MI_TYPE_Q8_0: return n % 32 ? 0 : (size_t)(n / 32) * 34;
    default: return 0;
    }
}

// an expert table ne=[K, N, E] with ggml strides
int check_table(const mi_tensor &t, int64_t K, int64_t N, int64_t E) {
    if (!t.data) return MI_MOE_ERR_NULL;
    if (!is_kquant(t.type) && !is_b32f(t.type) && t.type != MI_TYPE_F32) return MI_MOE_ERR_TYPE;
    if (is_b32f(t.type) && K % 32) return MI_MOE_ERR_UNSUPPORTED;   // whole 32-value blocks (F16: the kernels' unit)
    if (t.ne[0] != K || t.ne[1] != N || t.ne[2] < E || t.ne[3] != 1) return MI_MOE_ERR_SHAPE;
    const size_t rs = type_row_size(t.type, K);
    if (rs == 0) return MI_MOE_ERR_SHAPE;
    if (t.nb[1] < rs || t.nb[2] < t.nb[1] * (size_t)N) return MI_MOE_ERR_SHAPE;
    if (t.type == MI_TYPE_Q4_K && ((uintptr_t)t.data % 16 || t.nb[1] % 16 || t.nb[2] % 16))
        return MI_MOE_ERR_UNSUPPORTED;   // Q4_K rows are read with 16-byte loads
    if (t.type == MI_TYPE_Q6_K && ((uintptr_t)t.data % 4 || t.nb[1] % 2 || t.nb[2] % 2))
        return MI_MOE_ERR_UNSUPPORTED;
    if (t.type == MI_TYPE_F32 && ((uintptr_t)t.data % 4 || t.nb[1] % 4)) return MI_MOE_ERR_UNSUPPORTED;
    if (t.type == MI_TYPE_F16 && ((uintptr_t)t.data % 16 || t.nb[1] % 16 || t.nb[2] % 16))
        return MI_MOE_ERR_UNSUPPORTED;   // F16 rows are read with 16-byte loads
    if (is_b32(t.type) && ((uintptr_t)t.data % 2 || t.nb[1] % 2 || t.nb[2] % 2)) return MI_MOE_ERR_UNSUPPORTED;
    return MI_MOE_OK;
}

ExpertMat as_mat(const mi_tensor &t) {
    ExpertMat m;
    m.data = (const uint8_t *)t.data;
    m.type = t.type;
    m.row_bytes = (int64_t)t.nb[1];
    m.mat_bytes = (int64_t)t.nb[2];
    m.K = t.ne[0];
    m.N = t.ne[1];
    return m;
}

bool act_gated(int act) { return act != MI_ACT_RELU_SQR; }

// the expert tables of a layer (routed, or the shared expert as E = 1)
int check_experts(const mi_tensor &gate, const mi_tensor &up, const mi_tensor &down, int fused, int act, int64_t D,
                  int64_t I, int64_t E) {
    if (act < MI_ACT_SILU || act > MI_ACT_RELU_SQR) return MI_MOE_ERR_ARG;
    const bool gated = act_gated(act);
    if (!gated && fused) return MI_MOE_ERR_ARG;   // one product: gate holds ffn_up_exps
    const int64_t Ng = gated && fused ? 2 * I : I;
    TRY(check_table(gate, D, Ng, E));
    if (gated && !fused) {
        TRY(check_table(up, D, I, E));
        if (up.type != gate.type) return MI_MOE_ERR_TYPE;   // gate/up interchangeable (moe_compute.cpp:114-116)
    }
    TRY(check_table(down, I, D, E));
    // one family per layer: F32, k-quants, or the 32-value formats with F16
    if (type_family(gate.type) != type_family(down.type)) return MI_MOE_ERR_UNSUPPORTED;
    return MI_MOE_OK;
}

// the descriptor of src's tiled copy (type and ne of src, the copy's row
// strides), for a Q4_K or Q6_K table of whole 32-row groups
int tiled_desc(const mi_tensor &src, mi_tensor &d) {
    if (src.type != MI_TYPE_Q4_K && src.type != MI_TYPE_Q6_K) return MI_MOE_ERR_TYPE;
    const int64_t K = src.ne[0], N = src.ne[1];
    if (K <= 0 || K % QK || N <= 0 || N % 32 || src.ne[2] <= 0 || src.ne[3] <= 0) return MI_MOE_ERR_SHAPE;
    d = src;
    d.data = nullptr;
    d.nb[0] = src.type == MI_TYPE_Q4_K ? (size_t)Q4K_BYTES : (size_t)Q6X_ROW_BYTES;
    d.nb[1] = d.nb[0] * (size_t)(K / QK);
    d.nb[2] = d.nb[1] * (size_t)N;
    d.nb[3] = d.nb[2] * (size_t)src.ne[2];
    return MI_MOE_OK;
}

// an optional tiled copy of table t (mi_moe_layer.gate_tiled ..): absent, or
// mi_moe_tile's descriptor of t (Q4_K gate / up, Q4_K or Q6_K down)
int check_tiled(const mi_tensor &tiled, const mi_tensor &t, bool q6k_ok) {
    if (!tiled.data) return MI_MOE_OK;
    if (tiled.type != t.type || (t.type != MI_TYPE_Q4_K && !(q6k_ok && t.type == MI_TYPE_Q6_K)))
        return MI_MOE_ERR_TYPE;
    mi_tensor want;
    TRY(tiled_desc(t, want));
    for (int i = 0; i < 4; ++i)
        if (tiled.ne[i] != want.ne[i] || (tiled.nb[i] != want.nb[i] && (i < 3 || want.ne[3] > 1)))
            return MI_MOE_ERR_SHAPE;
    if ((uintptr_t)tiled.data % 16) return MI_MOE_ERR_UNSUPPORTED;
    return MI_MOE_OK;
}

// shared: validate the shared-expert fields too (the forward; the table form ignores them)
int validate_layer(const mi_moe_ctx *c, const mi_moe_layer *L, bool need_router, bool shared) {
    if (!L) return MI_MOE_ERR_NULL;
    const int64_t D = L->n_embd, E = L->n_expert, K = L->n_expert_used, I = L->n_ff;
    if (D <= 0 || E <= 0 || K <= 0 || I <= 0 || K > E) return MI_MOE_ERR_SHAPE;
    if (E > 256 || K > 64) return MI_MOE_ERR_UNSUPPORTED;
    if (L->gating < MI_GATING_SOFTMAX_TOPK || L->gating > MI_GATING_SOFTMAX_ALL) return MI_MOE_ERR_ARG;
    if (need_router && !L->router_w) return MI_MOE_ERR_NULL;
    TRY(check_experts(L->gate, L->up, L->down, L->fused_gate_up, L->act, D, I, E));
    TRY(check_tiled(L->gate_tiled, L->gate, false));
    TRY(check_tiled(L->down_tiled, L->down, true));
    if (act_gated(L->act) && !L->fused_gate_up) {
        TRY(check_tiled(L->up_tiled, L->up, false));
        if (!L->gate_tiled.data != !L->up_tiled.data) return MI_MOE_ERR_ARG;   // both or neither
    }
    if (act_gated(L->act) && L->fused_gate_up && L->gate_tiled.data && I % 32)
        return MI_MOE_ERR_SHAPE;   // the g half of [h | g] starts on a 32-row group
    if (shared && L->sh_n_ff < 0) return MI_MOE_ERR_SHAPE;
    if (shared && L->sh_n_ff > 0) TRY(check_experts(L->sh_gate, L->sh_up, L->sh_down, 0, L->sh_act, D, L->sh_n_ff, 1));
    if (!c->reserved) return MI_MOE_ERR_CAPACITY;
    if (D > c->cap_D || I > c->cap_I || E > c->cap_E || K > c->cap_K) return MI_MOE_ERR_CAPACITY;
    if (shared && (int64_t)L->sh_n_ff > (int64_t)c->cap_I * c->cap_K) return MI_MOE_ERR_CAPACITY;
    return MI_MOE_OK;
}

// Single-token fused kernel: shape and layout conditions, and the work split
// (P (h, g) row pairs per WG for gate/up, C output columns per WG for down).
bool plan_decode1(const mi_moe_ctx *c, const mi_moe_layer *L, const float *x, int &P, int &C) {
    const int64_t D = L->n_embd, E = L->n_expert, K = L->n_expert_used, I = L->n_ff;
    const int G = c->dec_grid;
    if (!c->fused_decode || G <= 0) return false;
    // the fused kernel ranks and weights with the default gating only, runs
    // gated experts and no shared expert
    if (L->gating != MI_GATING_SOFTMAX_TOPK || L->expert_scale) return false;
    if (!act_gated(L->act) || L->sh_n_ff > 0) return false;
    if (L->gate.type != MI_TYPE_Q4_K || (!L->fused_gate_up && L->up.type != MI_TYPE_Q4_K)) return false;
    if (L->down.type != MI_TYPE_Q4_K && L->down.type != MI_TYPE_Q6_K) return false;
    if (D % QK || I % QK || K > 8 || E > 256) return false;
    if (E > G || D / QK > E) return false;   // one router row per WG; x-quant WGs also route
    const int64_t NB = D / QK, NBI = I / QK;
    if (!(NB == 1 || NB == 2 || NB == 4 || NB == 8) || NBI > 8) return false;
    auto al16 = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
    if (!al16(x) || !al16(L->router_w) || !al16(L->gate.data) || !al16(L->down.data)) return false;
    if (L->gate.nb[2] % 16 || L->down.nb[2] % 16) return false;
    if (!L->fused_gate_up && (!al16(L->up.data) || L->up.nb[2] % 16)) return false;
    P = 0;
    for (int64_t p = 4; p <= 64; p += 4)
        if (I % p == 0 && (K * I) / p <= G) { P = (int)p; break; }
    if (!P || (P / 4) * (int64_t)L->gate.nb[1] > DEC_LIMIT_GU_BYTES) return false;
    if (!L->fused_gate_up && (P / 4) * (int64_t)L->up.nb[1] > DEC_LIMIT_GU_BYTES) return false;
    C = 0;
    for (int64_t cc = 1; cc <= 64; ++cc)
        if (D % cc == 0 && D / cc <= G) { C = (int)cc; break; }
    if (!C || C * (int64_t)L->down.nb[1] + 15 > DEC_LIMIT_DN_BYTES) return false;
    if (C * (I + 16 + NBI * 40) > DEC_LIMIT_UNPACKED_BYTES) return false;   // unpacked down rows of a slot
    return true;
}

int run_decode1(mi_moe_ctx *c, const mi_moe_layer *L, const float *x, const float *res, float *out, int P,
                int C, const NormParams &np, hipStream_t st) {
    DecArgs g = {};
    g.rw = L->router_w; g.rb = L->router_b; g.x = x;
    g.D = L->n_embd; g.E = L->n_expert; g.K = L->n_expert_used; g.I = L->n_ff;
    g.gate = as_mat(L->gate);
    if (!L->fused_gate_up) g.up = as_mat(L->up);
    g.down = as_mat(L->down);
    g.fused = L->fused_gate_up; g.act = L->act;
    g.res = res; g.out = out; g.P = P; g.C = C;
    g.logits = c->logits; g.sel = c->sel; g.w = c->w;
    g.counts = c->disp[0].counts; g.offsets = c->disp[0].offsets; g.perm = c->disp[0].perm;
    g.xq = c->ax.q8; g.xd = c->ax.d8; g.xbs = c->ax.bs;
    g.actf = c->f1;
    g.tw = c->dec_tw; g.epoch = c->dec_epoch; g.err = c->dec_err; g.rescue_polls = c->dec_rescue_polls;
    g.norm = np;
    TRY(launch_decode1(g, c->dec_grid, st));
    stage_end(c, "decode1", st);
    return MI_MOE_OK;
}

// The batched fused kernel for 2..16 tokens: the same layer kinds as the
// single-token kernel (default gating, gated Q4_K gate/up, Q4_K / Q6_K down,
// no shared expert) with D <= 2048 and I <= 1024 in whole 256-blocks; cc: the
// output columns per C unit (as many units as work-groups where D allows)
bool plan_decodeb(const mi_moe_ctx *c, const mi_moe_layer *L, const float *x, int64_t T, int &cc) {
    const int64_t D = L->n_embd, E = L->n_expert, K = L->n_expert_used, I = L->n_ff;
    const int G = c->dec_grid;
    if (!c->fused_decode || G <= 0 || T < 2 || T > DECB_T_MAX) return false;
    // Experts of more than 2 MiB (the model shapes): at most one dispatched
    // row per expert on average.  The kernel reads an expert's rows once per
    // token routed to it, the grouped GEMMs on 32-row tiles once per call:
    // above that they are as fast or faster (moondream3 Q6_K down, T = 12:
    // 105.7 vs 91.8 us; qwen3omni T = 16, one row per expert: 92.2 vs 101.1).
    const int64_t ebytes = L->gate.nb[2] + (L->fused_gate_up ? 0 : L->up.nb[2]) + L->down.nb[2];
    if (ebytes > (2LL << 20) && T * L->n_expert_used > L->n_expert) return false;
    // With tiled table copies the chain's GEMMs stream faster: past 8 tokens
    // they win (qwen3omni, same box: T = 9 / 10 / 12 / 16 chain 66.2 / 66.9 /
    // 71.2 / 79.6 against 71.1 / 72.8 / 78.6 / 87.3 us; T = 8: 64.8 vs 55.9).
    if (ebytes > (2LL << 20) && L->gate_tiled.data && T > 8) return false;
    if (decodeb_tw_words(T, D, E, K, I) > c->decb_words) return false;
    if (L->gating != MI_GATING_SOFTMAX_TOPK || L->expert_scale) return false;
    if (!act_gated(L->act) || L->sh_n_ff > 0) return false;
    if (L->gate.type != MI_TYPE_Q4_K || (!L->fused_gate_up && L->up.type != MI_TYPE_Q4_K)) return false;
    if (L->down.type != MI_TYPE_Q4_K && L->down.type != MI_TYPE_Q6_K) return false;
    if (D % QK || I % QK || K > 8 || E > 256) return false;
    const int64_t NB = D / QK, NBI = I / QK;
    if (!(NB == 1 || NB == 2 || NB == 4 || NB == 8) || NBI > 4) return false;
    auto al16 = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
    if (!al16(x) || !al16(L->router_w) || !al16(L->gate.data) || L->gate.nb[2] % 16) return false;
    if (!L->fused_gate_up && (!al16(L->up.data) || L->up.nb[2] % 16)) return false;
    if (L->down.type == MI_TYPE_Q4_K ? (!al16(L->down.data) || L->down.nb[2] % 16)
                                     : ((uintptr_t)L->down.data % 2 || L->down.nb[2] % 2))
        return false;
    cc = 64;
    while (cc > 8 && T * (D / cc) < G) cc /= 2;
    return D % cc == 0;
}

int run_decodeb(mi_moe_ctx *c, const mi_moe_layer *L, const float *x, int64_t T, const float *res, float *out,
                int cc, hipStream_t st) {
    DecArgs g = {};
    g.rw = L->router_w; g.rb = L->router_b; g.x = x;
    g.D = L->n_embd; g.E = L->n_expert; g.K = L->n_expert_used; g.I = L->n_ff; g.T = (int)T;
    g.gate = as_mat(L->gate);
    if (!L->fused_gate_up) g.up = as_mat(L->up);
    g.down = as_mat(L->down);
    g.fused = L->fused_gate_up; g.act = L->act;
    g.res = res; g.out = out; g.C = cc;
    g.logits = c->logits; g.sel = c->sel; g.w = c->w;
    g.counts = c->disp[0].counts; g.offsets = c->disp[0].offsets; g.perm = c->disp[0].perm;
    g.xq = c->ax.q8; g.xd = c->ax.d8; g.xbs = c->ax.bs;
    g.actf = c->f1;
    g.tw = c->dec_tw; g.tw2 = c->decb_tw; g.epoch = c->dec_epoch; g.err = c->dec_err;
    g.rescue_polls = c->dec_rescue_polls;
    TRY(launch_decodeb(g, c->dec_grid, st));
    stage_end(c, "decodeb", st);
    return MI_MOE_OK;
}

// How the expert path consumes x: false for fp32 expert tables, else the
// Q8_K form it reads (GEMV: codes, scales, block sums; GEMM: fp16 d*q in the
// gate weight's MFMA K order).
bool use_gemm(const mi_moe_ctx *c, int64_t T, int K, int E) {
    // Measured crossover (MI355X, Q4_K tables, 16 rotated layer copies, the
    // GEMMs on 32-row tiles): the grouped GEMM pays per M-tile, the GEMV per
    // token and row, so the switch follows the rows per expert T*K/E:
    // qwen3omni (E 128, K 8) GEMV faster up to T = 6 (72.1 / 73.0 us), GEMM
    // from 8 (79.9 / 82.8 us); moondream3 (E 64, K 8) GEMV up to 3, GEMM from
    // 4 (63.9 / 67.8 us).  The rule takes the GEMM from half a row per expert.
    if (c->gemm_threshold > 0) return T >= c->gemm_threshold;
    return 2 * T * K >= (int64_t)E;
}
// The switch of the products still on 192-row tiles (mul_mat_id) and of
// the Q4_0 / Q5_0 / Q8_0 / F16 tables, as measured on them: the GEMM above
// 1.25 dispatched rows per expert.
bool use_gemm_wide(const mi_moe_ctx *c, int64_t T, int K, int E) {
    if (c->gemm_threshold > 0) return T >= c->gemm_threshold;
    return 4 * T * K > 5 * (int64_t)E;
}

// the grouped MFMA GEMMs (else the grouped GEMV) for a k-quant layer
bool gemm_path(const mi_moe_ctx *c, const mi_moe_layer *L, int64_t T) {
    return use_gemm(c, T, L->n_expert_used, L->n_expert) || L->n_embd > 8 * QK || L->n_ff > 8 * QK;
}
// the 4-wave 32x32x16 GEMMs (Q4_K gate/up GLU, and every one-product layer);
// else the 16x16x32 GEMM with its fused GLU + Q8_K epilogue (Q6_K gate/up)
bool g4_path(const mi_moe_layer *L) { return L->gate.type == MI_TYPE_Q4_K || !act_gated(L->act); }

// Row tiles of the 4-wave GEMMs: 32-row tiles (52 KB of LDS with Q4_K
// weights: three work-groups per CU keep more of the weight stream in flight) when the call
// dispatches at most G4_SMALL_ROWS rows per expert on average (qwen3omni up
// to 128 tokens, moondream3 up to 64), where the products are bound by that
// stream; 192-row balanced tiles above.
constexpr int64_t G4_SMALL_ROWS = 8;
// logits (T x E) up to which the router may split its chunks: beyond, the
// partials' round trip costs more than the split saves (qwen3omni T = 128:
// +0.8 us per layer; moondream3 T = 128, half the partials: -3.2 us)
constexpr int64_t FRONT_SPLIT_TE_MAX = 8192;
bool g4_small_tiles(const mi_moe_ctx *c, const mi_moe_layer *L, int64_t T) {
    if (c->gemm_tiles == 1 || c->gemm_tiles == 2 || c->gemm_tiles == 4 || c->gemm_tiles == 5)
        return c->gemm_tiles == 2 || c->gemm_tiles == 4;
    return T * L->n_expert_used <= G4_SMALL_ROWS * L->n_expert;
}
// 8-row tiles (G4_BM_TINY) where the 32-row tiles would run without a
// dispatch launch and a call dispatches at most G4_TINY_ROWS rows per expert
// on average: 40 KB of LDS with Q4_K weights, four work-groups per CU (a
// third more of the weight stream in flight than three), at the cost of a
// second tile (and a second read of the weights) for an expert with more
// than 8 rows.  Q4_K down tables only for the down product (a Q6_K one
// keeps 32-row tiles: its LDS allows two work-groups either way).
constexpr int64_t G4_TINY_ROWS = 4;
bool g4_tiny_tiles(const mi_moe_ctx *c, const mi_moe_layer *L, int64_t T) {
    if (c->gemm_tiles == 4) return true;
    if (c->gemm_tiles != 0) return false;
    return T * L->n_expert_used <= G4_TINY_ROWS * L->n_expert;
}

// 64-row tiles (G4_BM_MID: 68 KB of LDS with Q4_K weights, two work-groups
// per CU, one's dequant beside the other's MFMA) past G4_SMALL_ROWS and up to
// G4_MID_ROWS dispatched rows per expert on average: nearly every expert is
// still one tile, so the weights stream once as with 192-row tiles.
// Measured (qwen3omni, tiled copies, same box, layer us): T = 256 / 512
// 136.9 / 155.7 -> 116.0 / 133.6 (gate/up 66.5 / 74.0 -> 55.3 / 63.3, down
// 45.8 / 50.2 -> 35.3 / 40.6); at 64 rows per expert (T = 1024) 192.3 ->
// 198.6 and moondream3 at 128, 184.7 -> 231: experts split into several
// tiles stream their weights again.
constexpr int64_t G4_MID_ROWS = 48;
bool g4_mid_tiles(const mi_moe_ctx *c, const mi_moe_layer *L, int64_t T) {
    if (c->gemm_tiles != 0) return c->gemm_tiles == 5;
    return T * L->n_expert_used <= G4_MID_ROWS * L->n_expert;
}

// The skinny products (k_gs.hip: 16-row tiles, one work-group per CU, each
// wave's weight stream held several blocks ahead in registers) for Q4_K
// layers (gate/up and down) with K <= GS_KMAX, on request only
// (mi_moe_ctx_set_gemm_tiles kind 3): measured against the 4-wave GEMMs on
// 32-row tiles at 16 to 128 tokens of the qwen3omni layer they were within a
// few percent either way from box to box.
bool gs_path(const mi_moe_ctx *c, const mi_moe_layer *L, int64_t T) {
    (void)T;
    if (L->gate.type != MI_TYPE_Q4_K || L->down.type != MI_TYPE_Q4_K) return false;
    if (act_gated(L->act) && !L->fused_gate_up && L->up.type != MI_TYPE_Q4_K) return false;
    if (L->n_embd > GS_KMAX || L->n_ff > GS_KMAX || L->n_ff % 16 || L->n_embd % 16) return false;
    return c->gemm_tiles == 3;
}

// work-groups per tile of the skinny products: about one work-group per CU
// (they run one per CU) for the tiles a call of `rows` rows over E experts
// is expected to make (uniform routing: the experts hit plus one tile per
// further GS_BM rows), at least one column group per wave (waves per
// work-group)
int gs_splits(const mi_moe_ctx *c, int64_t rows, int E, int64_t ncols, int glu) {
    const double hit = E * (1.0 - std::pow(1.0 - 1.0 / E, (double)rows));
    const double tiles = std::max(1.0, hit + std::max(0.0, (double)rows - hit * GS_BM) / GS_BM);
    const int cap = (int)std::max<int64_t>(1, ncols / 16 / gemm_gs_waves(glu));
    const int slots = std::max(1, c->n_cu) * gemm_gs_wgs_per_cu(glu);
    return std::max(1, std::min(cap, (int)std::lround(slots / tiles)));
}

// Small batches: the router's D / 64 chunks split over work-groups when the
// (16-token, 16-expert) tiles alone would leave at least half of the CUs
// idle (launch_front_parts); the chunk partials live in z, which is free
// until the down product.  The chunks per work-group, or 0 for the
// one-launch front.  Measured (layer us, same box, 16 rotated copies, the
// default product paths): qwen3omni T = 1 / 4 / 16 / 32 / 64: 40.2 / 60.9 /
// 100.6 / 114.2 / 118.5 -> 38.0 / 58.4 / 97.6 / 112.1 / 118.4; moondream3
// 42.2 / 63.9 / 86.8 / 87.9 / 88.7 -> 38.1 / 60.6 / 82.2 / 85.1 / 85.9.
int front_split_cps(const mi_moe_ctx *c, int64_t T, int D, int E) {
    const int nch = (D + 63) / 64;
    if (nch > 32 || T * E > FRONT_SPLIT_TE_MAX || E > 128) return 0;
    const int64_t tiles = ((T + 15) / 16) * ((E + 15) / 16);
    int nsp = 1;
    while (2 * nsp <= nch && tiles * 2 * nsp <= std::max(1, c->n_cu)) nsp *= 2;
    if (nsp < 2 || (int64_t)nch * T * E * 2 > c->cap_z) return 0;
    return (nch + nsp - 1) / nsp;
}

bool x_q8_spec(const mi_moe_ctx *c, const mi_moe_layer *L, int64_t T, Q8Out &qx) {
    if (!is_kquant(L->gate.type)) return false;
    qx = Q8Out{};
    if (!gemm_path(c, L, T)) {
        qx.q8 = c->ax.q8; qx.d8 = c->ax.d8; qx.bsums = c->ax.bs;
    } else {
        qx.xh = c->ax.h; qx.wtype = L->gate.type; qx.order = g4_path(L) ? 1 : 0;
        qx.range_total = c->range_total;
    }
    return true;
}

// routed FFN body of a layer with Q4_0 / Q5_0 / Q8_0 / F16 tables (k_b32.hip):
// the rows converted to each product's ggml vec_dot_type (Q8_0 or fp16), the
// grouped GEMV below the GEMM threshold, the grouped MFMA GEMM above it, GLU
// rows in fp32, fp32 slot rows into the combine.  Arguments as run_experts.
int run_experts_b32(mi_moe_ctx *c, const mi_moe_layer *L, const float *x, int64_t T, const int32_t *ids_gu,
                    const int32_t *ids_dn, const float *w, const float *res, float *out, hipStream_t st,
                    bool check_ids, const float *add) {
    const int D = L->n_embd, E = L->n_expert, K = L->n_expert_used, I = L->n_ff;
    const int64_t rows = T * K;
    const int max_active = (int)std::min<int64_t>(E, rows);
    const bool same_ids = ids_gu == ids_dn;
    const bool gated = act_gated(L->act);
    const bool gemm = use_gemm_wide(c, T, K, E);
    const int max_tiles = (int)((rows + G4_BM - 1) / G4_BM + max_active);
    TRY(launch_dispatch(ids_gu, T, K, E, G4_BM, 1, c->disp[0].view(), st));
    if (!same_ids) TRY(launch_dispatch(ids_dn, T, K, E, G4_BM, 1, c->disp[1].view(), st));
    const DispBuf &dg = c->disp[0];
    const DispBuf &dd = same_ids ? c->disp[0] : c->disp[1];
    stage_end(c, "dispatch", st);
    // an activation set in the operand form of a consumer type on this path
    auto prep_for = [&](int wtype, ActBuf &ab, int pre_act) {
        B32Prep o;
        o.pre_act = pre_act;
        if (wtype == MI_TYPE_F16) { o.mode = B32_PREP_F16; o.xh = ab.h; }
        else if (gemm) { o.mode = B32_PREP_DQ; o.xh = ab.h; }
        else { o.mode = B32_PREP_CODES; o.q8 = ab.q8; o.dh = (uint16_t *)ab.bs; }
        return o;
    };
    auto args_for = [&](const ExpertMat &a, const DispBuf &d, const ActBuf &ab, int ne11) {
        B32Args g = {};
        g.a = a; g.ne11 = ne11; g.K = K; g.act = L->act; g.I = I;
        g.q8 = ab.q8; g.dh = (const uint16_t *)ab.bs; g.xh = ab.h;
        g.counts = d.counts; g.offsets = d.offsets; g.perm = d.perm; g.active_e = d.active_e;
        g.n_active = d.n_active; g.max_active = max_active;
        g.tile_e = d.tile_e; g.tile_start = d.tile_start; g.tile_rows = d.tile_rows; g.n_tiles = d.n_tiles;
        g.max_tiles = max_tiles;
        return g;
    };
    TRY(launch_prep_b32(x, D, T, D, prep_for(L->gate.type, c->ax, 0), st));
    stage_end(c, "q8_x", st);
    B32Args a = args_for(as_mat(L->gate), dg, c->ax, 1);
    if (gated && !L->fused_gate_up) a.b = as_mat(L->up);
    a.glu = gated ? 1 : 0;
    a.fused = L->fused_gate_up;
    a.y = c->f1; a.ldy = I; a.ncols = I;
    TRY(gemm ? launch_gemm_b32(a, st) : launch_gemv_b32(a, st));
    stage_end(c, "gate_up", st);
    // one product (relu^2 experts): its rows are squared on the way to the down operand
    TRY(launch_prep_b32(c->f1, I, rows, I, prep_for(L->down.type, c->aact, gated ? 0 : MI_ACT_RELU_SQR), st));
    stage_end(c, "q8_act", st);
    B32Args d = args_for(as_mat(L->down), dd, c->aact, K);
    d.glu = 0;
    d.y = c->z; d.ldy = D; d.ncols = D;
    TRY(gemm ? launch_gemm_b32(d, st) : launch_gemv_b32(d, st));
    stage_end(c, "down", st);
    CombineIds ci;
    if (check_ids) { ci.a = ids_gu; ci.b = ids_dn; ci.E = E; }
    TRY(launch_combine(c->z, w, res, out, T, K, D, st, ci, add));
    stage_end(c, "combine", st);
    return MI_MOE_OK;
}

// routed FFN body: ids (device [T][K]; gate/up and down may differ) and
// weights w [T][K]; x_done: x is already in the x_q8_spec form; check_ids:
// the ids come from the caller (dead slots are left out of the combine);
// add: [T][D] added to the routed sum before the residual (or null)
int run_experts(mi_moe_ctx *c, const mi_moe_layer *L, const float *x, int64_t T, const int32_t *ids_gu,
                const int32_t *ids_dn, const float *w, const float *res, float *out, hipStream_t st,
                bool x_done = false, bool check_ids = false, const float *add = nullptr,
                bool disp_out = true) {
    if (is_b32f(L->gate.type)) return run_experts_b32(c, L, x, T, ids_gu, ids_dn, w, res, out, st, check_ids, add);
    const int D = L->n_embd, E = L->n_expert, K = L->n_expert_used, I = L->n_ff;
    const int64_t rows = T * K;
    const int max_active = (int)std::min<int64_t>(E, rows);
    const bool same_ids = ids_gu == ids_dn;
    const bool kq = is_kquant(L->gate.type);
    const bool gated = act_gated(L->act);
    const bool gemm = kq && gemm_path(c, L, T);
    // GEMM M-tiles: balanced tiles of at most G4_BM rows for the 4-wave GEMMs,
    // GEMM_BM-row tiles otherwise
    const bool g4 = gemm && g4_path(L);
    const bool gs = g4 && gs_path(c, L, T);
    const int bm = !g4 ? GEMM_BM : gs ? GS_BM : g4_small_tiles(c, L, T) ? G4_BM_SMALL : g4_mid_tiles(c, L, T) ? G4_BM_MID : G4_BM;
    const int max_tiles = (int)((rows + bm - 1) / bm + max_active);
    // Small calls on the 32-row tiles, ids from the router: no dispatch
    // launch, each GEMM work-group finds its tile from the ids itself
    // (g4_self_tile), unless the caller wants the dispatch's outputs.
    // Measured (layer us, kernel chain, same box): qwen3omni T = 8 / 16 / 32
    // / 64: 78.3 / 100.1 / 115.9 / 120.6 -> 74.8 / 96.7 / 113.0 / 118.3;
    // moondream3 79.3 / 84.3 / 87.9 / 88.5 -> 76.5 / 80.6 / 85.5 / 85.8.
    const bool self_disp = bm == G4_BM_SMALL && !gs && same_ids && !check_ids && !disp_out && rows <= G4_SD_IDS &&
                           E <= 256;
    // without a dispatch, each product may take 8-row tiles (its own tiles
    // from the ids; the tile tables are not used)
    const bool tiny = self_disp && g4_tiny_tiles(c, L, T);
    const int bm_gu = tiny ? G4_BM_TINY : bm;
    const int bm_dn = tiny && L->down.type == MI_TYPE_Q4_K ? G4_BM_TINY : bm;
    if (!self_disp) {
        TRY(launch_dispatch(ids_gu, T, K, E, bm, g4, c->disp[0].view(), st));
        if (!same_ids) TRY(launch_dispatch(ids_dn, T, K, E, bm, g4, c->disp[1].view(), st));
    }
    const DispBuf &dg = c->disp[0];
    const DispBuf &dd = same_ids ? c->disp[0] : c->disp[1];
    stage_end(c, "dispatch", st);
    Q8Out qx;
    if (x_q8_spec(c, L, T, qx) && !x_done) {
        TRY(launch_q8k_rows(x, D, T, D, qx, st));
        stage_end(c, "q8k_x", st);
    }

    const ExpertMat gate = as_mat(L->gate), down = as_mat(L->down);
    ExpertMat up = {};
    if (gated && !L->fused_gate_up) up = as_mat(L->up);

    if (!kq) {
        // fp32 expert tables: reference semantics without activation quantization
        const int64_t Ng = gated && L->fused_gate_up ? 2LL * I : I;
        GemvArgs a = {};
        a.a = gate; a.ne11 = 1; a.K = K;
        a.counts = dg.counts; a.offsets = dg.offsets; a.perm = dg.perm; a.active_e = dg.active_e;
        a.n_active = dg.n_active; a.max_active = max_active;
        a.y = c->f1; a.ldy = Ng; a.ncols = Ng;
        TRY(launch_mm_id_f32(a, x, D, st));
        const float *hbuf = c->f1, *gbuf = gated && L->fused_gate_up ? c->f1 + I : c->f1;
        int64_t ldh = Ng, ldg = Ng;
        if (gated && !L->fused_gate_up) {
            a.a = up; a.y = c->f2; a.ldy = I; a.ncols = I;
            TRY(launch_mm_id_f32(a, x, D, st));
            gbuf = c->f2;
            ldg = I;
        }
        // act into z scratch rows [rows][I] (RELU_SQR reads only the first operand)
        float *act = c->z;
        TRY(launch_glu_rows(hbuf, ldh, gbuf, ldg, act, I, rows, I, L->act, st));
        stage_end(c, "gate_up", st);
        GemvArgs d = {};
        d.a = down; d.ne11 = K; d.K = K;
        d.counts = dd.counts; d.offsets = dd.offsets; d.perm = dd.perm; d.active_e = dd.active_e;
        d.n_active = dd.n_active; d.max_active = max_active;
        d.y = c->f1; d.ldy = D; d.ncols = D;
        TRY(launch_mm_id_f32(d, act, I, st));
        stage_end(c, "down", st);
        CombineIds ci;
        if (check_ids) { ci.a = ids_gu; ci.b = ids_dn; ci.E = E; }
        TRY(launch_combine(c->f1, w, res, out, T, K, D, st, ci, add));
        stage_end(c, "combine", st);
        return MI_MOE_OK;
    }

    _Float16 *zh = nullptr;   // fp16 slot rows (4-wave GEMM path), else fp32 in c->z
    if (!gemm) {
        GemvArgs a = {};
        a.a = gate; a.b = up; a.epi = gated ? EPI_GLU : EPI_STORE; a.act = L->act; a.I = I;
        a.fused = L->fused_gate_up;
        a.q8 = c->ax.q8; a.d8 = c->ax.d8; a.bsums = c->ax.bs; a.ne11 = 1; a.K = K;
        a.counts = dg.counts; a.offsets = dg.offsets; a.perm = dg.perm; a.active_e = dg.active_e;
        a.n_active = dg.n_active; a.max_active = max_active;
        a.y = c->f1; a.ldy = I; a.ncols = I;
        TRY(launch_gemv(a, st));
        stage_end(c, "gate_up", st);
        // Q8_K of the activation rows (one product: of relu(u)^2)
        Q8Out qa;
        qa.q8 = c->aact.q8; qa.d8 = c->aact.d8; qa.bsums = c->aact.bs; qa.pre_act = gated ? 0 : MI_ACT_RELU_SQR;
        TRY(launch_q8k_rows(c->f1, I, rows, I, qa, st));
        stage_end(c, "q8k_act", st);
        GemvArgs d = {};
        d.a = down; d.epi = EPI_STORE;
        d.q8 = c->aact.q8; d.d8 = c->aact.d8; d.bsums = c->aact.bs; d.ne11 = K; d.K = K;
        d.counts = dd.counts; d.offsets = dd.offsets; d.perm = dd.perm; d.active_e = dd.active_e;
        d.n_active = dd.n_active; d.max_active = max_active;
        d.y = c->z; d.ldy = D; d.ncols = D;
        TRY(launch_gemv(d, st));
        stage_end(c, "down", st);
    } else if (g4) {
        // 4-wave GEMMs on 32x32x16 MFMA: fp16 dequantized weights x fp16
        // d*q of the Q8_K activations; gated: the GLU fused into the gate/up
        // GEMM, one product: the plain GEMM; then Q8_K of the activation rows
        // (ggml: the down mul_mat_id quantizes its F32 input) for the down GEMM
        G2Args a = {};
        a.a = gate; a.b = up; a.glu = gated ? 1 : 0; a.fused = L->fused_gate_up; a.act = L->act; a.I = I;
        if (L->gate_tiled.data) {
            // the tables' tiled copies
            a.a.data = (const uint8_t *)L->gate_tiled.data;
            if (gated && !L->fused_gate_up) a.b.data = (const uint8_t *)L->up_tiled.data;
            a.tiled = 1;
        }
        a.xh = c->ax.h; a.ne11 = 1; a.K = K;
        a.counts = dg.counts; a.offsets = dg.offsets; a.perm = dg.perm; a.tile_e = dg.tile_e;
        a.tile_r0 = dg.tile_r0; a.tile_start = dg.tile_start; a.tile_rows = dg.tile_rows; a.n_tiles = dg.n_tiles; a.max_tiles = max_tiles;
        a.tile_perm = dg.tile_perm;
        a.bm = bm_gu;
        if (self_disp) {
            a.ids = ids_gu; a.nids = (int)rows; a.n_expert = E;
            a.max_tiles = (int)((rows + bm_gu - 1) / bm_gu + max_active);
        }
        a.y = c->f1; a.ldy = I; a.ncols = I; a.xrows = T;
        // gated: the GLU rows as fp16 (half the bytes of their round trip to
        // the Q8_K pass; saturation at the fp16 range is counted)
        if (gated) { a.yh = (_Float16 *)c->f1; a.range_total = c->range_total; }
        if (!gs) prof_clock(c, a, 0);   // (the skinny kernels record no clocks)
        TRY(gs ? launch_gemm_gs(a, gs_splits(c, rows, E, gated ? I : a.ncols, a.glu), st) : launch_gemm4(a, st));
        stage_end(c, "gate_up", st);
        // the 32-row down product quantizes its own rows (gated: fp16 GLU rows)
        const bool own_q8 = bm_dn <= G4_BM_SMALL && !gs && gated;
        Q8Out qa;
        qa.xh = c->aact.h; qa.wtype = down.type; qa.order = 1; qa.pre_act = gated ? 0 : MI_ACT_RELU_SQR;
        qa.range_total = c->range_total;
        if (own_q8) {
            // (no pass: the down product's work-groups quantize their rows)
        } else if (gated) {
            TRY(launch_q8k_rows((const _Float16 *)c->f1, I, rows, I, qa, st));
        } else {
            TRY(launch_q8k_rows(c->f1, I, rows, I, qa, st));
        }
        stage_end(c, "q8k_act", st);
        G2Args d = {};
        d.a = down; d.glu = 0; d.xh = c->aact.h; d.ne11 = K; d.K = K;
        if (L->down_tiled.data) { d.a = as_mat(L->down_tiled); d.tiled = 1; }
        if (own_q8) { d.q8src = (const _Float16 *)c->f1; d.q8ld = I; }
        d.counts = dd.counts; d.offsets = dd.offsets; d.perm = dd.perm; d.tile_e = dd.tile_e;
        d.tile_r0 = dd.tile_r0; d.tile_start = dd.tile_start; d.tile_rows = dd.tile_rows; d.n_tiles = dd.n_tiles; d.max_tiles = max_tiles; d.xrows = (int64_t)T * K;
        d.tile_perm = dd.tile_perm;
        d.bm = bm_dn;
        if (self_disp) {
            d.ids = ids_dn; d.nids = (int)rows; d.n_expert = E;
            d.max_tiles = (int)((rows + bm_dn - 1) / bm_dn + max_active);
        }
        // the slot rows as fp16 (half the bytes of the round trip to the
        // combine; saturation at the fp16 range is counted)
        d.y = c->z; d.yh = zh = (_Float16 *)c->z; d.range_total = c->range_total; d.ldy = D; d.ncols = D;
        if (!gs) prof_clock(c, d, 1);
        TRY(gs ? launch_gemm_gs(d, gs_splits(c, rows, E, D, 0), st) : launch_gemm4(d, st));
        stage_end(c, "down", st);
    } else {
        // Q6_K gate/up: fp16 dequant on 16x16x32 MFMA
        GemmArgs a = {};
        a.a = gate; a.b = up; a.epi = EPI_GLU; a.act = L->act; a.I = I; a.fused = L->fused_gate_up;
        a.xh = c->ax.h; a.ne11 = 1; a.K = K;
        a.counts = dg.counts; a.offsets = dg.offsets; a.perm = dg.perm; a.tile_e = dg.tile_e;
        a.tile_r0 = dg.tile_r0; a.n_tiles = dg.n_tiles; a.max_tiles = max_tiles;
        a.acth = c->aact.h; a.next_type = down.type; a.ncols = I; a.range_total = c->range_total;
        TRY(launch_gemm(a, st));
        stage_end(c, "gate_up", st);
        GemmArgs d = {};
        d.a = down; d.epi = EPI_STORE; d.xh = c->aact.h; d.ne11 = K; d.K = K;
        d.counts = dd.counts; d.offsets = dd.offsets; d.perm = dd.perm; d.tile_e = dd.tile_e;
        d.tile_r0 = dd.tile_r0; d.n_tiles = dd.n_tiles; d.max_tiles = max_tiles;
        d.y = c->z; d.ldy = D; d.ncols = D;
        TRY(launch_gemm(d, st));
        stage_end(c, "down", st);
    }
    CombineIds ci;
    if (check_ids) { ci.a = ids_gu; ci.b = ids_dn; ci.E = E; }
    TRY(launch_combine(zh ? nullptr : c->z, w, res, out, T, K, D, st, ci, add, zh));
    stage_end(c, "combine", st);
    return MI_MOE_OK;
}

// The shared expert of every token into c->sh_out: a one-expert layer whose
// tokens all select expert 0 with weight 1 or the sigmoid of the scalar gate
// row (a one-expert router in the router's fixed fp64 order).
int run_shared(mi_moe_ctx *c, const mi_moe_layer *L, const float *x, int64_t T, hipStream_t st) {
    mi_moe_layer S = {};
    S.n_embd = L->n_embd;
    S.n_expert = 1;
    S.n_expert_used = 1;
    S.n_ff = L->sh_n_ff;
    S.gate = L->sh_gate;
    S.up = L->sh_up;
    S.down = L->sh_down;
    S.fused_gate_up = 0;
    S.act = L->sh_act;
    const float *lg = nullptr;
    if (L->sh_gate_inp) {
        TRY(launch_router(L->sh_gate_inp, nullptr, x, L->n_embd, T, L->n_embd, 1, c->sh_logit, st));
        lg = c->sh_logit;
    }
    TRY(launch_shared_gate(lg, T, c->sh_ids, c->sh_w, st));
    TRY(run_experts(c, &S, x, T, c->sh_ids, c->sh_ids, c->sh_w, nullptr, c->sh_out, st));
    stage_end(c, "shared_expert", st);
    return MI_MOE_OK;
}

template <typename T>
T *carve(char *&p, size_t n) {
    T *r = (T *)p;
    size_t bytes = (sizeof(T) * n + 255) & ~(size_t)255;
    p += bytes;
    return r;
}
template <typename T>
constexpr size_t carve_size(size_t n) {
    return (sizeof(T) * n + 255) & ~(size_t)255;
}

// Workspace of a context sized for max_tokens tokens of layers up to these
// dims: every piece 256-byte aligned, in the order carve_workspace lays them out.
constexpr size_t ws_bytes(int64_t max_tokens, int64_t D, int64_t I, int64_t E, int64_t K) {
    const int64_t rows = max_tokens * K;
    const int64_t kmax = D > I ? D : I;
    const int64_t kmax_q = (kmax + QK - 1) / QK * QK;
    const int64_t wide = (D > 2 * I ? D : 2 * I) > kmax ? (D > 2 * I ? D : 2 * I) : kmax;
    const int64_t tiles = (rows + GS_BM - 1) / GS_BM + (E < rows ? E : rows);
    const int64_t iq = (I + QK - 1) / QK * QK;
    size_t need = 0;
    need += carve_size<float>(max_tokens * E) + carve_size<int32_t>(rows) + carve_size<float>(rows);
    need += carve_size<float>(max_tokens * D);
    for (int s = 0; s < 2; ++s)
        need += carve_size<int32_t>(E) + carve_size<int32_t>(E + 1) + carve_size<int32_t>(rows) +
                4 * carve_size<int32_t>(tiles) + carve_size<int32_t>(tiles * GS_BM) + carve_size<int32_t>(1) +
                carve_size<int32_t>(E) +
                2 * carve_size<int32_t>(1);
    need += 2 * carve_size<int32_t>(1);   // bad_total, range_total
    // activation sets: x/b rows (rows x kmax) and act rows (rows x I)
    need += carve_size<int8_t>(rows * kmax_q) + carve_size<float>(rows * kmax_q / QK) +
            carve_size<int16_t>(rows * kmax_q / 16) + carve_size<_Float16>(rows * kmax_q) +
            carve_size<_Float16>(rows * kmax_q / 16);
    need += carve_size<int8_t>(rows * iq) + carve_size<float>(rows * iq / QK) +
            carve_size<int16_t>(rows * iq / 16) + carve_size<_Float16>(rows * iq);
    need += carve_size<float>(rows * wide) + carve_size<float>(rows * I) + carve_size<float>(rows * wide);
    need += carve_size<uint64_t>(DEC_TW_WORDS) + carve_size<uint32_t>(DEC_MAX_GRID) + carve_size<unsigned>(1);
    need += carve_size<uint64_t>(decodeb_tw_words(max_tokens < DECB_T_MAX ? max_tokens : DECB_T_MAX, D, E, K, I));
    need += carve_size<float>(max_tokens * D) + 2 * carve_size<float>(max_tokens) + carve_size<int32_t>(max_tokens);
    return need;
}

// Lays the workspace of ws_bytes(...) bytes at base out into c's pointers and
// records the capacities; false if the layout and ws_bytes disagree.
bool carve_workspace(mi_moe_ctx *c, char *base, int64_t max_tokens, int32_t D, int32_t I, int32_t E, int32_t K) {
    const int64_t rows = max_tokens * K;
    const int64_t kmax = std::max<int64_t>(D, I);
    const int64_t kmax_q = (kmax + QK - 1) / QK * QK;
    const int64_t wide = std::max<int64_t>(std::max<int64_t>(D, 2LL * I), kmax);
    const int64_t tiles = (rows + GS_BM - 1) / GS_BM + std::min<int64_t>(E, rows);
    const int64_t iq = (I + QK - 1) / QK * QK;
    char *q = base;
    c->logits = carve<float>(q, max_tokens * E);
    c->sel = carve<int32_t>(q, rows);
    c->w = carve<float>(q, rows);
    c->xn = carve<float>(q, max_tokens * D);
    for (int s = 0; s < 2; ++s) {
        DispBuf &d = c->disp[s];
        d.counts = carve<int32_t>(q, E);
        d.offsets = carve<int32_t>(q, E + 1);
        d.perm = carve<int32_t>(q, rows);
        d.tile_e = carve<int32_t>(q, tiles);
        d.tile_r0 = carve<int32_t>(q, tiles);
        d.tile_start = carve<int32_t>(q, tiles);
        d.tile_rows = carve<int32_t>(q, tiles);
        d.tile_perm = carve<int32_t>(q, tiles * GS_BM);
        d.n_tiles = carve<int32_t>(q, 1);
        d.active_e = carve<int32_t>(q, E);
        d.n_active = carve<int32_t>(q, 1);
        d.bad = carve<int32_t>(q, 1);
    }
    c->bad_total = carve<int32_t>(q, 1);
    c->disp[0].bad_total = c->disp[1].bad_total = c->bad_total;
    c->range_total = carve<int32_t>(q, 1);
    c->ax.q8 = carve<int8_t>(q, rows * kmax_q);
    c->ax.d8 = carve<float>(q, rows * kmax_q / QK);
    c->ax.bs = carve<int16_t>(q, rows * kmax_q / 16);
    c->ax.h = carve<_Float16>(q, rows * kmax_q);
    c->ax.bsh = carve<_Float16>(q, rows * kmax_q / 16);
    c->aact.q8 = carve<int8_t>(q, rows * iq);
    c->aact.d8 = carve<float>(q, rows * iq / QK);
    c->aact.bs = carve<int16_t>(q, rows * iq / 16);
    c->aact.h = carve<_Float16>(q, rows * iq);
    c->f1 = carve<float>(q, rows * wide);
    c->f2 = carve<float>(q, rows * I);
    c->z = carve<float>(q, rows * wide);
    c->dec_tw = carve<uint64_t>(q, DEC_TW_WORDS);
    c->dec_epoch = carve<uint32_t>(q, DEC_MAX_GRID);
    c->dec_err = carve<unsigned>(q, 1);
    c->decb_words = decodeb_tw_words(std::min<int64_t>(max_tokens, DECB_T_MAX), D, E, K, I);
    c->decb_tw = carve<uint64_t>(q, c->decb_words);
    c->sh_out = carve<float>(q, max_tokens * D);
    c->sh_w = carve<float>(q, max_tokens);
    c->sh_logit = carve<float>(q, max_tokens);
    c->sh_ids = carve<int32_t>(q, max_tokens);
    c->cap_T = max_tokens;
    c->cap_D = D;
    c->cap_I = I;
    c->cap_E = E;
    c->cap_K = K;
    c->cap_rows = rows;
    c->cap_kmax = kmax_q;
    c->cap_tiles = tiles;
    c->cap_z = rows * wide;
    return (size_t)(q - base) == ws_bytes(max_tokens, D, I, E, K);
}

}  // namespace

extern "C" {

int mi_moe_abi_version(void) { return MI_MOE_ABI_VERSION; }

const char *mi_moe_status_string(int s) {
    switch (s) {
    case MI_MOE_OK: return "ok";
    case MI_MOE_ERR_NULL: return "null pointer";
    case MI_MOE_ERR_SHAPE: return "bad shape";
    case MI_MOE_ERR_TYPE: return "unsupported type";
    case MI_MOE_ERR_CAPACITY: return "exceeds reserved capacity";
    case MI_MOE_ERR_HIP: return "HIP error";
    case MI_MOE_ERR_UNSUPPORTED: return "unsupported";
    case MI_MOE_ERR_DEVICE: return "bad device";
    case MI_MOE_ERR_ARG: return "bad argument";
    case MI_MOE_ERR_FORMAT: return "bad or unreadable file";
    default: return "unknown";
    }
}

size_t mi_row_size(int32_t type, int64_t n) { return type_row_size(type, n); }

int mi_moe_ctx_create(mi_moe_ctx **out, int device) {
    if (!out) return MI_MOE_ERR_NULL;
    *out = nullptr;
    int n = 0;
    HIP_TRY(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return MI_MOE_ERR_DEVICE;
    HIP_TRY(hipSetDevice(device));
    mi_moe_ctx *c = new mi_moe_ctx();
    c->device = device;
    if (decode1_max_grid(device, &c->dec_grid)) c->dec_grid = 0;
    if (hipDeviceGetAttribute(&c->n_cu, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) c->n_cu = 256;
    for (int i = 0; i <= kMaxStages; ++i) {
        const hipError_t e = hipEventCreate(&c->ev[i]);
        if (e != hipSuccess) {
            for (int j = 0; j < i; ++j) (void)hipEventDestroy(c->ev[j]);
            delete c;
            return record_hip_error(e);
        }
    }
    *out = c;
    return MI_MOE_OK;
}

void mi_moe_ctx_destroy(mi_moe_ctx *c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->ws) (void)hipFree(c->ws);
    if (c->clk) (void)hipFree(c->clk);
    for (int i = 0; i <= kMaxStages; ++i)
        if (c->ev[i]) (void)hipEventDestroy(c->ev[i]);
    delete c;
}

int mi_moe_ctx_reserve(mi_moe_ctx *c, int64_t max_tokens, int32_t D, int32_t I, int32_t E, int32_t K) {
    if (!c) return MI_MOE_ERR_NULL;
    if (max_tokens <= 0 || D <= 0 || I <= 0 || E <= 0 || K <= 0 || K > E) return MI_MOE_ERR_SHAPE;
    if (E > 256 || K > 64) return MI_MOE_ERR_UNSUPPORTED;
    HIP_TRY(hipSetDevice(c->device));
    const size_t need = ws_bytes(max_tokens, D, I, E, K);
    if (c->ws) {
        (void)hipFree(c->ws);
        c->ws = nullptr;
        c->reserved = false;
    }
    void *p = nullptr;
    HIP_TRY(hipMalloc(&p, need));
    c->ws = p;
    c->ws_bytes = need;
    if (!carve_workspace(c, (char *)p, max_tokens, D, I, E, K)) return MI_MOE_ERR_UNSUPPORTED;
    HIP_TRY(hipMemset(p, 0, need));
    c->reserved = true;
    return MI_MOE_OK;
}

int mi_moe_ctx_take_errors(mi_moe_ctx *c, int64_t *bad_ids, int64_t *wait_failures, int64_t *fp16_saturated) {
    if (!c) return MI_MOE_ERR_NULL;
    if (bad_ids) *bad_ids = 0;
    if (wait_failures) *wait_failures = 0;
    if (fp16_saturated) *fp16_saturated = 0;
    if (!c->reserved) return MI_MOE_OK;
    HIP_TRY(hipSetDevice(c->device));
    HIP_TRY(hipDeviceSynchronize());
    int32_t b = 0, r = 0;
    unsigned f = 0;
    HIP_TRY(hipMemcpy(&b, c->bad_total, sizeof(b), hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(&f, c->dec_err, sizeof(f), hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(&r, c->range_total, sizeof(r), hipMemcpyDeviceToHost));
    HIP_TRY(hipMemset(c->bad_total, 0, sizeof(b)));
    HIP_TRY(hipMemset(c->dec_err, 0, sizeof(f)));
    HIP_TRY(hipMemset(c->range_total, 0, sizeof(r)));
    HIP_TRY(hipDeviceSynchronize());
    if (bad_ids) *bad_ids = b;
    if (wait_failures) *wait_failures = f;
    if (fp16_saturated) *fp16_saturated = r;
    return MI_MOE_OK;
}

int mi_moe_ctx_set_gemm_threshold(mi_moe_ctx *c, int64_t t) {
    if (!c) return MI_MOE_ERR_NULL;
    if (t < 0) return MI_MOE_ERR_ARG;
    c->gemm_threshold = t;
    return MI_MOE_OK;
}

int mi_moe_ctx_set_gemm_tiles(mi_moe_ctx *c, int kind) {
    if (!c) return MI_MOE_ERR_NULL;
    if (kind < 0 || kind > 5) return MI_MOE_ERR_ARG;
    c->gemm_tiles = kind;
    return MI_MOE_OK;
}

int mi_moe_ctx_set_fused_decode(mi_moe_ctx *c, int on) {
    if (!c) return MI_MOE_ERR_NULL;
    if (on < MI_DECODE_CHAIN || on > MI_DECODE_FUSED) return MI_MOE_ERR_ARG;
    if (on == MI_DECODE_FUSED_COOPERATIVE) return MI_MOE_ERR_UNSUPPORTED;   // retired: the plain launch is faster
    c->fused_decode = on;
    return MI_MOE_OK;
}

int mi_moe_ctx_set_decode_rescue(mi_moe_ctx *c, int polls) {
    if (!c) return MI_MOE_ERR_NULL;
    if (polls < 0) return MI_MOE_ERR_ARG;
    c->dec_rescue_polls = (unsigned)polls;
    return MI_MOE_OK;
}

int mi_moe_ctx_set_profiling(mi_moe_ctx *c, int on) {
    if (!c) return MI_MOE_ERR_NULL;
    if (on && !c->clk) {
        HIP_TRY(hipSetDevice(c->device));
        HIP_TRY(hipMalloc(&c->clk, sizeof(uint64_t) * 2 * 4 * kClkWGs));
    }
    c->profiling = on != 0;
    c->n_stages = 0;
    c->clk_grid[0] = c->clk_grid[1] = 0;
    return MI_MOE_OK;
}

int mi_moe_ctx_stage_clock(mi_moe_ctx *c, const char *stage, double *ghz, int *n_wg) {
    if (!c || !stage || !ghz) return MI_MOE_ERR_NULL;
    *ghz = 0.0;
    if (n_wg) *n_wg = 0;
    const int k = std::strcmp(stage, "gate_up") == 0 ? 0 : std::strcmp(stage, "down") == 0 ? 1 : -1;
    if (k < 0) return MI_MOE_ERR_ARG;
    if (!c->profiling || c->clk_grid[k] == 0 || c->n_stages == 0) return MI_MOE_ERR_ARG;
    HIP_TRY(hipSetDevice(c->device));
    HIP_TRY(hipEventSynchronize(c->ev[c->n_stages]));
    int wall_khz = 0;
    HIP_TRY(hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, c->device));
    if (wall_khz <= 0) return MI_MOE_ERR_ARG;
    const int n = std::min(c->clk_grid[k], kClkWGs);
    std::vector<uint64_t> h((size_t)4 * n);
    HIP_TRY(hipMemcpy(h.data(), c->clk + (size_t)k * 4 * kClkWGs, h.size() * sizeof(uint64_t),
                      hipMemcpyDeviceToHost));
    // the clock over the work-groups' summed lifetimes: shader cycles / wall ticks
    double cyc = 0.0, ticks = 0.0;
    int live = 0;
    for (int i = 0; i < n; ++i) {
        const uint64_t *r = &h[(size_t)4 * i];
        if (r[1] == 0 || r[3] <= r[1] || r[2] <= r[0]) continue;
        cyc += (double)(r[2] - r[0]);
        ticks += (double)(r[3] - r[1]);
        ++live;
    }
    if (live == 0 || ticks <= 0.0) return MI_MOE_ERR_ARG;
    *ghz = cyc / ticks * (double)wall_khz * 1e-6;
    if (n_wg) *n_wg = live;
    return MI_MOE_OK;
}

int mi_moe_ctx_stage_times(mi_moe_ctx *c, int max_stages, const char **names, float *ms, int *n_stages) {
    if (!c || !n_stages) return MI_MOE_ERR_NULL;
    *n_stages = 0;
    if (!c->profiling || c->n_stages == 0) return MI_MOE_OK;
    HIP_TRY(hipEventSynchronize(c->ev[c->n_stages]));
    const int n = std::min(max_stages, c->n_stages);
    for (int i = 0; i < n; ++i) {
        if (names) names[i] = c->stage_name[i];
        if (ms) HIP_TRY(hipEventElapsedTime(&ms[i], c->ev[i], c->ev[i + 1]));
    }
    *n_stages = n;
    return MI_MOE_OK;
}

}  // extern "C"

namespace {

// the forward with an optional norm of its input (np.kind != NORM_NONE).  A
// single token on the fused kernel normalizes x inside it (every work-group
// computes the statistics in k_norm_rows' order while its router row loads
// stream, and stages the normed row in LDS): no norm launch.  Otherwise the
// rows are normalized into the workspace once and the forward runs as usual.
// (Applying the norm where the prefill router reads x was built and measured
// slower: each of a token slab's expert-tile work-groups recomputed the rows'
// statistics before its chunk loop, config-4 prefill 9.96 vs 9.57 ms.)
// xr: the rows the router reads when they differ from the experts' input
// (null: x; the norm, if any, applies to x only).
int forward_impl(mi_moe_ctx *c, const mi_moe_layer *L, const float *x, int64_t T, const float *res, float *out,
                 const mi_moe_routing *routing, const NormParams &np, hipStream_t st, const float *xr = nullptr) {
    if (!c) return MI_MOE_ERR_NULL;
    if (T < 0) return MI_MOE_ERR_SHAPE;
    TRY(validate_layer(c, L, true, true));
    if (T == 0) return MI_MOE_OK;
    if (!x || !out) return MI_MOE_ERR_NULL;
    if (T > c->cap_T) return MI_MOE_ERR_CAPACITY;
    const int D = L->n_embd, E = L->n_expert, K = L->n_expert_used;
    if (np.kind != NORM_NONE && D > 4096) return MI_MOE_ERR_UNSUPPORTED;
    HIP_TRY(hipSetDevice(c->device));
    stage_begin(c, st);
    if (xr == x) xr = nullptr;
    int P = 0, C = 0;
    // the fused decode kernels route on the rows they quantize for the experts
    const bool dec1 = T == 1 && !xr && plan_decode1(c, L, x, P, C);
    // The single-token kernel normalizes x itself only when out does not
    // overlap x: a work-group that computes a late router row or Q8_K block
    // re-reads x, possibly after other work-groups wrote their out columns.
    const uintptr_t xb = (uintptr_t)x, ob = (uintptr_t)out, row = sizeof(float) * (uintptr_t)D;
    const bool fuse_norm = dec1 && np.kind != NORM_NONE && (ob + row <= xb || xb + row <= ob);
    if (np.kind != NORM_NONE && !fuse_norm) {
        TRY(launch_norm(np, x, T, D, c->xn, st));
        stage_end(c, "norm", st);
        x = c->xn;
    }
    // the shared expert first (its own Q8_K of x; the routed block's follows)
    const float *add = nullptr;
    if (L->sh_n_ff > 0) {
        TRY(run_shared(c, L, x, T, st));
        add = c->sh_out;
    }
    int cc = 0;
    if (dec1) {
        TRY(run_decode1(c, L, x, res, out, P, C, fuse_norm ? np : NormParams{}, st));
    } else if (!xr && plan_decodeb(c, L, x, T, cc)) {
        TRY(run_decodeb(c, L, x, T, res, out, cc, st));
    } else {
        // router + Q8_K(x) in one launch where the shape fits (the router's
        // own rows: the router alone, the experts quantize x themselves)
        Q8Out qx;
        const bool xq = !xr && x_q8_spec(c, L, T, qx);
        const float *xrow = xr ? xr : x;
        Gating gt;
        gt.kind = L->gating;
        gt.sel_bias = L->sel_bias;
        gt.expert_scale = L->expert_scale;
        gt.scaling = L->routed_scaling != 0.f ? L->routed_scaling : 1.f;
        gt.eps = L->gate_eps;
        const int cps = front_split_cps(c, T, D, E);
        bool x_done = false;   // the Q8_K of x came with the router
        if (cps > 0) {
            double *parts = (double *)c->z;   // free until the down product
            TRY(launch_front_parts(L->router_w, xrow, D, T, D, E, cps, parts, xq ? &qx : nullptr, st));
            x_done = xq;
            stage_end(c, "router", st);
            TRY(launch_topk_parts(parts, D, L->router_b, c->logits, T, E, K, c->sel, K, c->w, st, gt));
        } else {
            const int rc = launch_front(L->router_w, L->router_b, xrow, D, T, D, E, c->logits, xq ? &qx : nullptr, st);
            if (rc == -6) TRY(launch_router(L->router_w, L->router_b, xrow, D, T, D, E, c->logits, st));
            else TRY(rc);
            x_done = xq && rc == 0;
            stage_end(c, "router", st);
            TRY(launch_topk_softmax(c->logits, E, T, E, K, c->sel, K, c->w, st, gt));
        }
        stage_end(c, "topk_softmax", st);
        TRY(run_experts(c, L, x, T, c->sel, c->sel, c->w, res, out, st, x_done, false, add,
                        routing && (routing->counts || routing->offsets || routing->perm)));
    }
    if (routing) {
        const DispBuf &d = c->disp[0];
        if (routing->logits)
            HIP_TRY(hipMemcpyAsync(routing->logits, c->logits, sizeof(float) * T * E, hipMemcpyDeviceToDevice, st));
        if (routing->sel)
            HIP_TRY(hipMemcpyAsync(routing->sel, c->sel, sizeof(int32_t) * T * K, hipMemcpyDeviceToDevice, st));
        if (routing->weights)
            HIP_TRY(hipMemcpyAsync(routing->weights, c->w, sizeof(float) * T * K, hipMemcpyDeviceToDevice, st));
        if (routing->counts)
            HIP_TRY(hipMemcpyAsync(routing->counts, d.counts, sizeof(int32_t) * E, hipMemcpyDeviceToDevice, st));
        if (routing->offsets)
            HIP_TRY(hipMemcpyAsync(routing->offsets, d.offsets, sizeof(int32_t) * (E + 1),
                                   hipMemcpyDeviceToDevice, st));
        if (routing->perm)
            HIP_TRY(hipMemcpyAsync(routing->perm, d.perm, sizeof(int32_t) * T * K, hipMemcpyDeviceToDevice, st));
    }
    return MI_MOE_OK;
}

int norm_params(const mi_moe_norm *norm, NormParams &np) {
    np = NormParams{};
    if (!norm || norm->kind == MI_NORM_NONE) return MI_MOE_OK;
    if (norm->kind != MI_NORM_RMS && norm->kind != MI_NORM_LAYER) return MI_MOE_ERR_ARG;
    np.kind = norm->kind == MI_NORM_RMS ? NORM_RMS : NORM_LAYER;
    np.eps = norm->eps;
    np.w = norm->weight;
    np.b = norm->kind == MI_NORM_LAYER ? norm->bias : nullptr;
    return MI_MOE_OK;
}

}  // namespace

extern "C" {

int mi_moe_forward(mi_moe_ctx *c, const mi_moe_layer *L, const float *x, int64_t T, const float *res,
                   float *out, const mi_moe_routing *routing, mi_stream_t stream) {
    return forward_impl(c, L, x, T, res, out, routing, NormParams{}, (hipStream_t)stream);
}

// ---------------------------------------------------------------- no allocation
// mi_moe_forward_noalloc: the workspace of a context reserved for the limits
// below lives in one file-scope device array per GPU (scratch).  In host code
// `scratch` names a host-side stand-in, not device memory: the array's device
// address comes from hipGetSymbolAddress, once per device with that device
// current (the first call on it), and only that address is used.  Single
// tokens run the kernel chain (no grid-wide waits, no cooperative launch), and
// every buffer a call reads it writes first in the same call, so nothing in
// the array has to start at zero.
}  // extern "C"

namespace {
constexpr int64_t NA_T = MI_NOALLOC_MAX_TOKENS;
constexpr int32_t NA_D = 2048, NA_I = 1024, NA_E = 128, NA_K = 8;
constexpr size_t NA_BYTES = ws_bytes(NA_T, NA_D, NA_I, NA_E, NA_K);
static_assert(NA_BYTES == 16973312, "mi_moe.h states the no-allocation workspace size");
constexpr int NA_MAX_DEVICES = 64;

struct NoallocDevice {
    std::mutex mu;
    std::atomic<bool> ready{false};
    mi_moe_ctx ctx;   // workspace pointers into this device's scratch; never destroyed
};
NoallocDevice g_noalloc[NA_MAX_DEVICES];
}  // namespace

static __device__ __attribute__((aligned(256))) char scratch[NA_BYTES];

namespace {
int noalloc_ctx(mi_moe_ctx **out) {
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= NA_MAX_DEVICES) return MI_MOE_ERR_DEVICE;
    NoallocDevice &d = g_noalloc[dev];
    if (!d.ready.load(std::memory_order_acquire)) {
        // set-up once per device; a failed lookup is not cached, the next call tries again
        std::lock_guard<std::mutex> lock(d.mu);
        if (!d.ready.load(std::memory_order_relaxed)) {
            void *ptr = nullptr;
            const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
            if (e != hipSuccess) return record_hip_error(e);
            if (!ptr) return MI_MOE_ERR_HIP;
            mi_moe_ctx &c = d.ctx;
            c.device = dev;
            if (hipDeviceGetAttribute(&c.n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) c.n_cu = 256;
            c.fused_decode = MI_DECODE_CHAIN;
            c.ws = nullptr;   // not owned
            c.ws_bytes = NA_BYTES;
            if (!carve_workspace(&c, (char *)ptr, NA_T, NA_D, NA_I, NA_E, NA_K)) return MI_MOE_ERR_UNSUPPORTED;
            c.reserved = true;
            d.ready.store(true, std::memory_order_release);
        }
    }
    *out = &d.ctx;
    return MI_MOE_OK;
}
}  // namespace

extern "C" {

int mi_moe_forward_noalloc(const mi_moe_layer *L, const float *x, int64_t T, const float *res, float *out,
                           const mi_moe_routing *routing, mi_stream_t stream) {
    if (!L) return MI_MOE_ERR_NULL;
    mi_moe_ctx *c = nullptr;
    TRY(noalloc_ctx(&c));
    return forward_impl(c, L, x, T, res, out, routing, NormParams{}, (hipStream_t)stream);
}

int mi_moe_forward_router_input(mi_moe_ctx *c, const mi_moe_layer *L, const float *x, const float *x_router,
                                int64_t T, const float *res, float *out, const mi_moe_routing *routing,
                                mi_stream_t stream) {
    return forward_impl(c, L, x, T, res, out, routing, NormParams{}, (hipStream_t)stream, x_router);
}

int mi_moe_forward_norm(mi_moe_ctx *c, const mi_moe_layer *L, const mi_moe_norm *norm, const float *h, int64_t T,
                        const float *res, float *out, const mi_moe_routing *routing, mi_stream_t stream) {
    NormParams np;
    TRY(norm_params(norm, np));
    return forward_impl(c, L, h, T, res, out, routing, np, (hipStream_t)stream);
}

int mi_norm(mi_moe_ctx *c, const mi_moe_norm *norm, const float *x, int64_t n_rows, int32_t n_cols, float *y,
            mi_stream_t stream) {
    if (!c || !norm || !x || !y) return MI_MOE_ERR_NULL;
    if (n_rows < 0 || n_cols <= 0) return MI_MOE_ERR_SHAPE;
    if (n_cols > 4096) return MI_MOE_ERR_UNSUPPORTED;
    NormParams np;
    TRY(norm_params(norm, np));
    if (np.kind == NORM_NONE) return MI_MOE_ERR_ARG;
    HIP_TRY(hipSetDevice(c->device));
    return launch_norm(np, x, n_rows, n_cols, y, (hipStream_t)stream);
}

int mi_moe_expert_ffn(mi_moe_ctx *c, const mi_moe_layer *L, const float *x, int64_t T, const float *res,
                      const int32_t *gate_up_ids, const int32_t *down_ids, const float *w, float *out,
                      mi_stream_t stream) {
    if (!c) return MI_MOE_ERR_NULL;
    if (T < 0) return MI_MOE_ERR_SHAPE;
    TRY(validate_layer(c, L, false, false));
    if (T == 0) return MI_MOE_OK;
    if (!x || !out || !gate_up_ids || !down_ids || !w) return MI_MOE_ERR_NULL;
    if (T > c->cap_T) return MI_MOE_ERR_CAPACITY;
    HIP_TRY(hipSetDevice(c->device));
    hipStream_t st = (hipStream_t)stream;
    stage_begin(c, st);
    return run_experts(c, L, x, T, gate_up_ids, down_ids, w, res, out, st, false, true);
}

int mi_top_k(mi_moe_ctx *c, const mi_tensor *a, int32_t k, mi_tensor *dst, mi_stream_t stream) {
    if (!c || !a || !dst || !a->data || !dst->data) return MI_MOE_ERR_NULL;
    if (a->type != MI_TYPE_F32 || dst->type != MI_TYPE_I32) return MI_MOE_ERR_TYPE;
    const int64_t E = a->ne[0], T = a->ne[1];
    if (E <= 0 || T < 0 || k <= 0 || k > E || a->ne[2] != 1 || a->ne[3] != 1) return MI_MOE_ERR_SHAPE;
    if (dst->ne[0] != k || dst->ne[1] != T || dst->ne[2] != 1 || dst->ne[3] != 1) return MI_MOE_ERR_SHAPE;
    if (a->nb[0] != 4 || dst->nb[0] != 4 || a->nb[1] % 4 || dst->nb[1] % 4) return MI_MOE_ERR_SHAPE;
    if (a->nb[1] < (size_t)E * 4 || dst->nb[1] < (size_t)k * 4) return MI_MOE_ERR_SHAPE;
    if (E > 256 || k > 64) return MI_MOE_ERR_UNSUPPORTED;
    if (T == 0) return MI_MOE_OK;
    HIP_TRY(hipSetDevice(c->device));
    return launch_topk_softmax((const float *)a->data, (int64_t)(a->nb[1] / 4), T, (int)E, k, (int32_t *)dst->data,
                               (int64_t)(dst->nb[1] / 4), nullptr, (hipStream_t)stream, Gating{});
}

int mi_mul_mat_id(mi_moe_ctx *c, const mi_tensor *as, const mi_tensor *b, const mi_tensor *ids, mi_tensor *dst,
                  mi_stream_t stream) {
    if (!c || !as || !b || !ids || !dst) return MI_MOE_ERR_NULL;
    if (!b->data || !ids->data || !dst->data) return MI_MOE_ERR_NULL;
    const int64_t Kin = as->ne[0], N = as->ne[1], E = as->ne[2];
    TRY(check_table(*as, Kin, N, E));
    if (as->ne[3] != 1) return MI_MOE_ERR_SHAPE;
    if (b->type != MI_TYPE_F32 || ids->type != MI_TYPE_I32 || dst->type != MI_TYPE_F32) return MI_MOE_ERR_TYPE;
    const int64_t n_used = ids->ne[0], T = ids->ne[1], ne11 = b->ne[1];
    if (b->ne[0] != Kin || b->ne[2] != T || b->ne[3] != 1) return MI_MOE_ERR_SHAPE;
    if (ne11 != 1 && ne11 != n_used) return MI_MOE_ERR_SHAPE;
    if (dst->ne[0] != N || dst->ne[1] != n_used || dst->ne[2] != T || dst->ne[3] != 1) return MI_MOE_ERR_SHAPE;
    if (n_used <= 0 || T < 0) return MI_MOE_ERR_SHAPE;
    // contiguous layouts (ggml's default strides)
    if (b->nb[0] != 4 || b->nb[1] != (size_t)Kin * 4 || b->nb[2] != (size_t)ne11 * Kin * 4) return MI_MOE_ERR_UNSUPPORTED;
    if (ids->nb[0] != 4 || ids->nb[1] != (size_t)n_used * 4) return MI_MOE_ERR_UNSUPPORTED;
    if (dst->nb[0] != 4 || dst->nb[1] != (size_t)N * 4 || dst->nb[2] != (size_t)n_used * N * 4)
        return MI_MOE_ERR_UNSUPPORTED;
    if (!c->reserved) return MI_MOE_ERR_CAPACITY;
    if (E > c->cap_E || E > 256) return MI_MOE_ERR_CAPACITY;
    if (T * n_used > c->cap_rows || T * ne11 > c->cap_rows || Kin > c->cap_kmax) return MI_MOE_ERR_CAPACITY;
    if (T == 0) return MI_MOE_OK;
    HIP_TRY(hipSetDevice(c->device));
    hipStream_t st = (hipStream_t)stream;
    const int64_t rows = T * n_used;
    const int max_active = (int)std::min<int64_t>(E, rows);
    const int max_tiles = (int)((rows + G4_BM - 1) / G4_BM + max_active);
    const DispBuf &dsp = c->disp[0];
    Dispatch dv = dsp.view();
    dv.zero_rows = (float *)dst->data;   // the rows of ids outside [0, E): zeros
    dv.zero_ld = N;
    dv.zero_n = N;
    TRY(launch_dispatch((const int32_t *)ids->data, T, (int)n_used, (int)E, G4_BM, 1, dv, st));
    const ExpertMat M = as_mat(*as);
    const float *bp = (const float *)b->data;
    if (is_b32f(as->type)) {
        // b in the table type's vec_dot_type (Q8_0 or fp16), then the grouped GEMV or GEMM
        const bool gemm = use_gemm_wide(c, T, (int)n_used, (int)E);
        B32Prep o;
        if (as->type == MI_TYPE_F16) { o.mode = B32_PREP_F16; o.xh = c->ax.h; }
        else if (gemm) { o.mode = B32_PREP_DQ; o.xh = c->ax.h; }
        else { o.mode = B32_PREP_CODES; o.q8 = c->ax.q8; o.dh = (uint16_t *)c->ax.bs; }
        TRY(launch_prep_b32(bp, Kin, T * ne11, Kin, o, st));
        B32Args a = {};
        a.a = M; a.glu = 0; a.ne11 = (int)ne11; a.K = (int)n_used;
        a.q8 = c->ax.q8; a.dh = (const uint16_t *)c->ax.bs; a.xh = c->ax.h;
        a.counts = dsp.counts; a.offsets = dsp.offsets; a.perm = dsp.perm; a.active_e = dsp.active_e;
        a.n_active = dsp.n_active; a.max_active = max_active;
        a.tile_e = dsp.tile_e; a.tile_start = dsp.tile_start; a.tile_rows = dsp.tile_rows; a.n_tiles = dsp.n_tiles;
        a.max_tiles = max_tiles;
        a.y = (float *)dst->data; a.ldy = N; a.ncols = N;
        return gemm ? launch_gemm_b32(a, st) : launch_gemv_b32(a, st);
    }
    if (as->type == MI_TYPE_F32) {
        GemvArgs a = {};
        a.a = M; a.ne11 = (int)ne11; a.K = (int)n_used;
        a.counts = dsp.counts; a.offsets = dsp.offsets; a.perm = dsp.perm; a.active_e = dsp.active_e;
        a.n_active = dsp.n_active; a.max_active = max_active;
        a.y = (float *)dst->data; a.ldy = N; a.ncols = N;
        return launch_mm_id_f32(a, bp, Kin, st);
    }
    const bool gemm = use_gemm_wide(c, T, (int)n_used, (int)E) || Kin > 8 * QK;
    if (!gemm) {
        Q8Out qx;
        qx.q8 = c->ax.q8; qx.d8 = c->ax.d8; qx.bsums = c->ax.bs;
        TRY(launch_q8k_rows(bp, Kin, T * ne11, Kin, qx, st));
        GemvArgs a = {};
        a.a = M; a.epi = EPI_STORE; a.q8 = c->ax.q8; a.d8 = c->ax.d8; a.bsums = c->ax.bs;
        a.ne11 = (int)ne11; a.K = (int)n_used;
        a.counts = dsp.counts; a.offsets = dsp.offsets; a.perm = dsp.perm; a.active_e = dsp.active_e;
        a.n_active = dsp.n_active; a.max_active = max_active;
        a.y = (float *)dst->data; a.ldy = N; a.ncols = N;
        return launch_gemv(a, st);
    }
    Q8Out qx;
    qx.xh = c->ax.h; qx.wtype = as->type; qx.order = 1; qx.range_total = c->range_total;
    TRY(launch_q8k_rows(bp, Kin, T * ne11, Kin, qx, st));
    G2Args a = {};
    a.bm = G4_BM;   // the dispatch's balanced 192-row tiles
    a.a = M; a.glu = 0; a.xh = c->ax.h; a.ne11 = (int)ne11; a.K = (int)n_used;
    a.counts = dsp.counts; a.offsets = dsp.offsets; a.perm = dsp.perm; a.tile_e = dsp.tile_e;
    a.tile_r0 = dsp.tile_r0; a.tile_start = dsp.tile_start; a.tile_rows = dsp.tile_rows; a.n_tiles = dsp.n_tiles; a.max_tiles = max_tiles; a.xrows = T * ne11;
    a.y = (float *)dst->data; a.ldy = N; a.ncols = N;
    return launch_gemm4(a, st);
}

int mi_quantize(mi_moe_ctx *c, int32_t type, const float *src, void *dst, int64_t nrows, int64_t n_per_row,
                mi_stream_t stream) {
    if (!c || !src || !dst) return MI_MOE_ERR_NULL;
    if (is_b32f(type)) {
        if (nrows < 0 || n_per_row <= 0 || n_per_row % 32) return MI_MOE_ERR_SHAPE;
        if ((uintptr_t)src % 4 || (type == MI_TYPE_F16 && (uintptr_t)dst % 4)) return MI_MOE_ERR_UNSUPPORTED;
        HIP_TRY(hipSetDevice(c->device));
        return launch_quantize_b32(type, src, dst, nrows * (n_per_row / 32), (hipStream_t)stream);
    }
    if (type != MI_TYPE_Q4_K && type != MI_TYPE_Q6_K) return MI_MOE_ERR_TYPE;
    if (nrows < 0 || n_per_row <= 0 || n_per_row % QK) return MI_MOE_ERR_SHAPE;
    if (type == MI_TYPE_Q4_K && ((uintptr_t)dst % 4)) return MI_MOE_ERR_UNSUPPORTED;
    if ((uintptr_t)src % 4) return MI_MOE_ERR_UNSUPPORTED;
    HIP_TRY(hipSetDevice(c->device));
    return launch_quantize(type, src, dst, nrows * (n_per_row / QK), (hipStream_t)stream);
}

int64_t mi_moe_tiled_bytes(const mi_tensor *src) {
    if (!src) return MI_MOE_ERR_NULL;
    mi_tensor d;
    TRY(tiled_desc(*src, d));
    return (int64_t)(d.nb[3] * (size_t)src->ne[3]);
}

int mi_moe_tile(mi_moe_ctx *c, const mi_tensor *src, void *dst, mi_tensor *desc, mi_stream_t stream) {
    if (!c || !src || !src->data || !dst) return MI_MOE_ERR_NULL;
    mi_tensor d;
    TRY(tiled_desc(*src, d));
    const int64_t K = src->ne[0], N = src->ne[1], n_mat = src->ne[2] * src->ne[3];
    const size_t rb = type_row_size(src->type, K);
    if (src->nb[1] != rb || src->nb[2] != rb * (size_t)N ||
        (src->ne[3] > 1 && src->nb[3] != src->nb[2] * (size_t)src->ne[2]))
        return MI_MOE_ERR_SHAPE;
    const size_t align = src->type == MI_TYPE_Q4_K ? 16 : 2;
    if ((uintptr_t)src->data % align || (uintptr_t)dst % 16) return MI_MOE_ERR_UNSUPPORTED;
    const size_t sbytes = rb * (size_t)N * (size_t)n_mat, dbytes = d.nb[2] * (size_t)n_mat;
    const uintptr_t s0 = (uintptr_t)src->data, d0 = (uintptr_t)dst;
    if (s0 < d0 + dbytes && d0 < s0 + sbytes) return MI_MOE_ERR_ARG;   // overlapping
    HIP_TRY(hipSetDevice(c->device));
    TRY(src->type == MI_TYPE_Q4_K ? launch_tile_q4k(src->data, dst, n_mat, N, (int64_t)rb, (hipStream_t)stream)
                                  : launch_tile_q6k(src->data, dst, n_mat, N, (int64_t)rb, (hipStream_t)stream));
    if (desc) {
        d.data = dst;
        *desc = d;
    }
    return MI_MOE_OK;
}

int mi_fill_normal(mi_moe_ctx *c, float *dst, int64_t n, uint64_t seed, uint64_t stream_id, float mean,
                   float stddev, mi_stream_t stream) {
    if (!c || !dst) return MI_MOE_ERR_NULL;
    if (n < 0) return MI_MOE_ERR_SHAPE;
    HIP_TRY(hipSetDevice(c->device));
    return launch_fill_normal(dst, n, seed, stream_id, mean, stddev, (hipStream_t)stream);
}

int mi_rmsnorm(mi_moe_ctx *c, const float *x, int64_t n_rows, int32_t n_cols, float eps, float *y,
               mi_stream_t stream) {
    if (!c || !x || !y) return MI_MOE_ERR_NULL;
    if (n_rows < 0 || n_cols <= 0) return MI_MOE_ERR_SHAPE;
    HIP_TRY(hipSetDevice(c->device));
    return launch_rmsnorm(x, n_rows, n_cols, eps, y, (hipStream_t)stream);
}

// ------------------------------------------------------------------ util ABI
int mi_device_count(int *count) {
    if (!count) return MI_MOE_ERR_NULL;
    HIP_TRY(hipGetDeviceCount(count));
    return MI_MOE_OK;
}
int mi_set_device(int device) {
    HIP_TRY(hipSetDevice(device));
    return MI_MOE_OK;
}
int mi_device_info(int device, char *name, int name_len, int *cu_count, int *clock_khz, char *arch, int arch_len) {
    hipDeviceProp_t p;
    HIP_TRY(hipGetDeviceProperties(&p, device));
    if (name && name_len > 0) {
        std::strncpy(name, p.name, (size_t)name_len - 1);
        name[name_len - 1] = 0;
    }
    if (arch && arch_len > 0) {
        std::strncpy(arch, p.gcnArchName, (size_t)arch_len - 1);
        arch[arch_len - 1] = 0;
    }
    if (cu_count) *cu_count = p.multiProcessorCount;
    if (clock_khz) *clock_khz = p.clockRate;
    return MI_MOE_OK;
}
int mi_dev_malloc(void **ptr, size_t bytes) {
    if (!ptr) return MI_MOE_ERR_NULL;
    HIP_TRY(hipMalloc(ptr, bytes));
    return MI_MOE_OK;
}
int mi_dev_free(void *ptr) {
    HIP_TRY(hipFree(ptr));
    return MI_MOE_OK;
}
int mi_memcpy_h2d(void *dst, const void *src, size_t bytes) {
    HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return MI_MOE_OK;
}
int mi_memcpy_h2d_async(void *dst, const void *src, size_t bytes, mi_stream_t s) {
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)s));
    return MI_MOE_OK;
}
int mi_memcpy_d2h_async(void *dst, const void *src, size_t bytes, mi_stream_t s) {
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)s));
    return MI_MOE_OK;
}
int mi_memcpy_d2h(void *dst, const void *src, size_t bytes) {
    HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return MI_MOE_OK;
}
int mi_memcpy_d2d(void *dst, const void *src, size_t bytes) {
    HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice));
    return MI_MOE_OK;
}
int mi_memset_d(void *dst, int value, size_t bytes) {
    HIP_TRY(hipMemset(dst, value, bytes));
    return MI_MOE_OK;
}
int mi_device_synchronize(void) {
    HIP_TRY(hipDeviceSynchronize());
    return MI_MOE_OK;
}
int mi_stream_create(mi_stream_t *s) {
    if (!s) return MI_MOE_ERR_NULL;
    hipStream_t h;
    HIP_TRY(hipStreamCreate(&h));
    *s = (mi_stream_t)h;
    return MI_MOE_OK;
}
int mi_stream_destroy(mi_stream_t s) {
    HIP_TRY(hipStreamDestroy((hipStream_t)s));
    return MI_MOE_OK;
}
int mi_stream_synchronize(mi_stream_t s) {
    HIP_TRY(hipStreamSynchronize((hipStream_t)s));
    return MI_MOE_OK;
}
int mi_event_create(mi_event_t *e) {
    if (!e) return MI_MOE_ERR_NULL;
    hipEvent_t h;
    HIP_TRY(hipEventCreate(&h));
    *e = (mi_event_t)h;
    return MI_MOE_OK;
}
int mi_event_destroy(mi_event_t e) {
    HIP_TRY(hipEventDestroy((hipEvent_t)e));
    return MI_MOE_OK;
}
int mi_event_record(mi_event_t e, mi_stream_t s) {
    HIP_TRY(hipEventRecord((hipEvent_t)e, (hipStream_t)s));
    return MI_MOE_OK;
}
int mi_event_synchronize(mi_event_t e) {
    HIP_TRY(hipEventSynchronize((hipEvent_t)e));
    return MI_MOE_OK;
}
int mi_event_elapsed_ms(float *ms, mi_event_t a, mi_event_t b) {
    if (!ms) return MI_MOE_ERR_NULL;
    HIP_TRY(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
    return MI_MOE_OK;
}
int mi_stream_begin_capture(mi_stream_t s) {
    if (!s) return MI_MOE_ERR_ARG;
    HIP_TRY(hipStreamBeginCapture((hipStream_t)s, hipStreamCaptureModeRelaxed));
    return MI_MOE_OK;
}
int mi_stream_end_capture(mi_stream_t s, mi_graph_t *graph) {
    if (!graph) return MI_MOE_ERR_NULL;
    *graph = nullptr;
    hipGraph_t g = nullptr;
    HIP_TRY(hipStreamEndCapture((hipStream_t)s, &g));
    hipGraphExec_t ex = nullptr;
    const hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return record_hip_error(e);
    *graph = (mi_graph_t)ex;
    return MI_MOE_OK;
}
int mi_graph_launch(mi_graph_t graph, mi_stream_t s) {
    if (!graph) return MI_MOE_ERR_NULL;
    HIP_TRY(hipGraphLaunch((hipGraphExec_t)graph, (hipStream_t)s));
    return MI_MOE_OK;
}
int mi_graph_destroy(mi_graph_t graph) {
    if (!graph) return MI_MOE_OK;
    HIP_TRY(hipGraphExecDestroy((hipGraphExec_t)graph));
    return MI_MOE_OK;
}
const char *mi_last_hip_error(void) { return g_last_error.c_str(); }

}  // extern "C"
