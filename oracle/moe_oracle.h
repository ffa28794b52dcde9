/*
 * moe_oracle.h - CPU oracle for the routed mixture-of-experts FFN layer.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library under
 * skyvision.cpp_amd/) links, loads or calls this code.  Only tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py use it, and
 * only as the checker / the timed CPU baseline.
 *
 * What it restates.  The reference (SkyVision.cpp) runs this layer as a chain
 * of ggml ops:
 *   moondream3  src/models/moondream/moondream.cpp:509-544
 *   qwen3omni   src/models/qwen3omni/qwen3omni_model.cpp:755-780
 *   table form  src/core/engine/moe_compute.cpp:93-136
 * The arithmetic of those ops lives in ggml (ggml-org/ggml, cloned at build
 * time from branch `master`, no commit pinned: Dockerfile:36-39,
 * .github/workflows/cpu-regression.yml:53-54), which is not in the reference
 * tree.  This file restates ggml's published CPU semantics for the ops on the
 * path: quantize_row_q4_K_ref / q6_K_ref / q8_K_ref, the k-quant x Q8_K dot
 * products (generic scalar form), mul_mat_id row grouping, top_k, get_rows +
 * soft_max, the GLU variants, mul + permute + cont + sum_rows, and the add.
 *
 * Documented choices where ggml is not pinned (see each function):
 *   - router logits use one fixed fp64 reduction order (orc_router_logits),
 *     the same order the GPU kernel uses, so routing is reproducible bit for
 *     bit; ggml's own fp32 SIMD order depends on its build;
 *   - top_k returns the K largest in descending order, ties -> lower expert id
 *     (the reference's oracle convention, scripts/parity_nemotronomni_seg.py:363);
 *   - per-expert row lists are token-ascending (ggml-cpu mul_mat_id groups
 *     rows iterating tokens outer, slots inner).
 *
 * Pinning status of each function is listed in tests/test_oracle_*.py and in
 * the repository's design notes.
 */
#ifndef MOE_ORACLE_H
#define MOE_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK_K 256

/* ggml_type numbering (GGUF on-disk type ids) */
enum {
    ORC_TYPE_F32  = 0,
    ORC_TYPE_F16  = 1,
    ORC_TYPE_Q4_0 = 2,
    ORC_TYPE_Q5_0 = 6,
    ORC_TYPE_Q8_0 = 8,
    ORC_TYPE_Q4_K = 12,
    ORC_TYPE_Q6_K = 14,
    ORC_TYPE_Q8_K = 15,
    ORC_TYPE_I32  = 26,
};

/* block layouts: convert/q4k.py:9-10, convert/q6k.py:10-11 */
typedef struct {
    uint16_t d;          /* fp16 super-block scale for the 6-bit scales */
    uint16_t dmin;       /* fp16 super-block scale for the 6-bit mins   */
    uint8_t  scales[12]; /* 8 x (6-bit scale, 6-bit min), packed        */
    uint8_t  qs[128];    /* 256 x 4-bit quants                          */
} orc_block_q4_K;        /* 144 bytes */

typedef struct {
    uint8_t  ql[128];    /* low 4 bits */
    uint8_t  qh[64];     /* high 2 bits */
    int8_t   scales[16]; /* 8-bit scale per 16 values */
    uint16_t d;          /* fp16 super-block scale */
} orc_block_q6_K;        /* 210 bytes */

typedef struct {
    float    d;
    int8_t   qs[256];
    int16_t  bsums[16];  /* sum of qs in groups of 16 */
} orc_block_q8_K;        /* 292 bytes */

/* 32-value blocks (ggml QK4_0 = QK5_0 = QK8_0 = 32): the expert tables the
 * reference's converters write by default (Q8_0: convert_hf_to_gguf.py:55-57,
 * convert_qwen3omni.py:60-61,135; Q5_0: convert_nemotronomni.py:113-114;
 * Q4_0: convert_diffusiongemma.py:62).  Packed without padding. */
#define ORC_QK32 32
#pragma pack(push, 1)
typedef struct {
    uint16_t d;          /* fp16 scale */
    uint8_t  qs[16];     /* value j: low nibble of qs[j], value j+16: high nibble; x = d (q - 8) */
} orc_block_q4_0;        /* 18 bytes */

typedef struct {
    uint16_t d;          /* fp16 scale */
    uint8_t  qh[4];      /* bit j: 5th bit of value j (j < 32), little-endian uint32 */
    uint8_t  qs[16];     /* low 4 bits, as q4_0; x = d (q - 16) */
} orc_block_q5_0;        /* 22 bytes */

typedef struct {
    uint16_t d;          /* fp16 scale */
    int8_t   qs[32];     /* x = d q */
} orc_block_q8_0;        /* 34 bytes */
#pragma pack(pop)

enum {                    /* activation applied between the two expert products */
    ORC_ACT_SILU           = 0,  /* silu(gate) * up              (qwen3omni, swiglu_split)        */
    ORC_ACT_GELU_ERF_GP1   = 1,  /* gelu_erf(h) * (g + 1)        (moondream3, geglu_erf_split)    */
    ORC_ACT_GELU_TANH      = 2,  /* gelu_tanh(gate) * up         (BASELINE config-0 literal)      */
    ORC_ACT_GELU_ERF       = 3,  /* gelu_erf(gate) * up                                           */
    ORC_ACT_RELU_SQR       = 4,  /* relu(u)^2 of ONE product, non-gated (nemotronomni experts,
                                    nemotronomni_model.cpp:366-367, 372-373): the gate table holds
                                    ffn_up_exps, no up table                                       */
};
/* act uses a gate/up pair (0..3) or one product (RELU_SQR) */
#define ORC_ACT_GATED(a) ((a) != ORC_ACT_RELU_SQR)

enum {                    /* router gating */
    ORC_GATING_SOFTMAX_TOPK = 0, /* top_k on logits, softmax over the K (moondream.cpp:510-516)   */
    ORC_GATING_SIGMOID_BIAS = 1, /* sigmoid, top_k on s + bias, renorm (nemotronomni_model.cpp:344-354) */
    ORC_GATING_SOFTMAX_ALL  = 2, /* softmax over all E, top_k on the probabilities, renorm over the
                                    K (diffusiongemma_model.cpp:923-932)                          */
};

/* ---- scalar helpers ---------------------------------------------------- */
float    orc_fp16_to_fp32(uint16_t h);
uint16_t orc_fp32_to_fp16(float f);
int      orc_nearest_int(float f);

/* ---- quantizers (ggml quantize_row_*_ref) -------------------------------
 * k must be a multiple of 256.  port = 0 follows ggml.  The reference's own
 * Python ports (convert/q4k.py, convert/q6k.py) differ from ggml in a few
 * documented places; port bits select those conventions, used only to
 * compare with the golden bytes the ports produced (tests/golden):
 *   ORC_PORT_FP32_D     q6_K: requantize against the unrounded fp32 d
 *                       (convert/q6k.py:171) instead of the fp16-rounded d
 *   ORC_PORT_ZERO_L     codes of a sub-block whose scale quantized to 0 are
 *                       written as 0 (q4k.py:113, q6k.py:177) instead of
 *                       keeping the scale search's codes (ggml `continue`)
 *   ORC_PORT_FIXED_SPAN q4_K: make_qkx2_quants keeps the initial max - min
 *                       as the search span (q4k.py:43) instead of the span
 *                       of the best min found so far */
#define ORC_PORT_FP32_D     1
#define ORC_PORT_ZERO_L     2
#define ORC_PORT_FIXED_SPAN 4
void orc_quantize_row_q4_K(const float *x, void *y, int64_t k);
void orc_quantize_row_q4_K_port(const float *x, void *y, int64_t k, int port);
void orc_quantize_row_q6_K(const float *x, void *y, int64_t k, int port);
void orc_quantize_row_q8_K(const float *x, void *y, int64_t k);
/* 32-value formats (k a multiple of 32): ggml quantize_row_q4_0_ref /
 * q5_0_ref / q8_0_ref; Q8_0 is also the activation type their dots use */
void orc_quantize_row_q4_0(const float *x, void *y, int64_t k);
void orc_quantize_row_q5_0(const float *x, void *y, int64_t k);
void orc_quantize_row_q8_0(const float *x, void *y, int64_t k);
/* many rows, threaded: nrows rows of k floats -> nrows * (k/256) blocks */
void orc_quantize_rows(int type, const float *x, void *y, int64_t nrows, int64_t k, int nthreads);

void orc_dequantize_row_q4_K(const void *x, float *y, int64_t k);
void orc_dequantize_row_q6_K(const void *x, float *y, int64_t k);
void orc_dequantize_row_q8_K(const void *x, float *y, int64_t k);
void orc_dequantize_row_q4_0(const void *x, float *y, int64_t k);
void orc_dequantize_row_q5_0(const void *x, float *y, int64_t k);
void orc_dequantize_row_q8_0(const void *x, float *y, int64_t k);

size_t orc_row_size(int type, int64_t k);   /* bytes of one row of k values */

/* ---- k-quant x Q8_K dots (ggml_vec_dot_*_q8_K, generic scalar order) --- */
float orc_vec_dot_q4_K_q8_K(int n, const void *x, const void *y);
float orc_vec_dot_q6_K_q8_K(int n, const void *x, const void *y);
/* The same two dots on AVX-512 BW + VNNI, bit for bit the scalar forms (the
 * scalar forms where the host lacks them); type ORC_TYPE_Q4_K or Q6_K. */
float orc_vec_dot_kq_simd(int type, int n, const void *x, const void *y);
/* mul_mat_id's k-quant dots (so the layer) on the AVX-512 forms: on = 1 where
 * the host has AVX-512 F / BW / VNNI; returns whether they are in use.  Off by
 * default: the scalar forms are the checker's definition. */
int orc_set_simd(int on);
/* 32-value formats x Q8_0 activations (ggml_vec_dot_q{4,5,8}_0_q8_0, generic
 * scalar order: an exact integer dot per block, then the fp32 sum over
 * blocks), and F16 x F16 (ggml_vec_dot_f16 generic: fp32 products, exact,
 * summed in double) */
float orc_vec_dot_q4_0_q8_0(int n, const void *x, const void *y);
float orc_vec_dot_q5_0_q8_0(int n, const void *x, const void *y);
float orc_vec_dot_q8_0_q8_0(int n, const void *x, const void *y);
float orc_vec_dot_f16(int n, const uint16_t *x, const uint16_t *y);

/* ---- seeded synthetic data ----------------------------------------------
 * Counter-based: value i of (seed, stream) is independent of how the range
 * is split, so the GPU generator reproduces it bit for bit.  Normal values use
 * Box-Muller with log/sin/cos evaluated by fixed polynomial code in fp64 (no
 * libm), identical on CPU and GPU. */
uint64_t orc_rng_u64(uint64_t seed, uint64_t stream, uint64_t i);
void orc_fill_normal(float *out, int64_t n, uint64_t seed, uint64_t stream,
                     float mean, float stddev, int nthreads);
double orc_poly_log(double x);
void   orc_poly_sincos_2pi(double u, double *s, double *c);

/* ---- router, gating, dispatch ------------------------------------------ */
/* logits[t][e] = fl32( fl32(dot(W[e], x[t])) + b[e] ), dot in fp64 with one
 * fixed order: the 64-element chunk c contributes part_c = sum over s = 0..15
 * (outer), g = 0..3 (inner) of W[e][64c+16g+s] * x[t][64c+16g+s], each added
 * left to right; the chunk partials are then summed left to right.  fp32 x
 * fp32 products are exact in fp64, so only this order matters.  W is ggml
 * ne=[D, E] (E rows of D). */
void orc_router_logits(const float *W, const float *b, const float *x,
                       int64_t T, int D, int E, float *logits, int nthreads);
/* ggml_top_k: K largest, descending, ties -> lower id */
void orc_top_k(const float *logits, int64_t T, int E, int K, int32_t *sel);
/* ggml_get_rows + ggml_soft_max over the K selected logits */
void orc_softmax_selected(const float *logits, const int32_t *sel,
                          int64_t T, int E, int K, float *w);
/* router gating variants: kind 0 top-k on logits + softmax over the K, kind 1
 * sigmoid + selection bias + renorm with eps and scaling, kind 2 softmax over
 * all E + top-k on the probabilities + renorm over the K; expert_scale (or
 * NULL) multiplies the weights */
void orc_route_gated(const float *logits, int64_t T, int E, int K, int kind, const float *sel_bias,
                     const float *expert_scale, float scaling, float eps, int32_t *sel, float *w);
/* histogram, exclusive scan, permutation (perm value = t*K + k), lists
 * token-ascending; counts[E], offsets[E+1], perm[T*K] */
void orc_dispatch(const int32_t *sel, int64_t T, int K, int E,
                  int32_t *counts, int32_t *offsets, int32_t *perm);

/* ---- ggml_mul_mat_id ------------------------------------------------------
 * as  : E matrices of N rows, each row Kin values of `type` (ne=[Kin,N,E])
 * b   : F32, T x ne11 rows of Kin (ne=[Kin, ne11, T]); ne11 is 1 or n_used
 * ids : I32 [T][n_used]
 * dst : F32 [T][n_used][N]
 * b rows are first converted to the weight type's ggml vec_dot_type: Q8_K for
 * Q4_K / Q6_K, Q8_0 for Q4_0 / Q5_0 / Q8_0, F16 (round to nearest even) for
 * F16; F32 weights take b as given.
 * exact = 1 instead computes in fp64 on dequantized weights and unquantized b.
 * Returns 0, or -1 on bad arguments. */
int orc_mul_mat_id(int type, const void *as, int64_t Kin, int64_t N, int E,
                   const float *b, int ne11, const int32_t *ids, int n_used,
                   int64_t T, float *dst, int exact, int nthreads);

/* ---- GLU ---------------------------------------------------------------- */
float orc_act_pair(int act, float a, float b);

/* ---- the whole layer ----------------------------------------------------- */
typedef struct {
    int32_t D, E, K, I;
    const float *router_w;        /* [E][D] */
    const float *router_b;        /* [E] or NULL */
    int32_t gate_type;            /* type of gate (and up) */
    const void *gate;             /* fused: ne=[D, 2I, E]; else ne=[D, I, E] */
    const void *up;               /* ne=[D, I, E]; NULL when fused */
    int32_t fused_gate_up;
    int32_t down_type;
    const void *down;             /* ne=[I, D, E] */
    int32_t act;                  /* ORC_ACT_*; RELU_SQR: gate holds up_exps ne=[D, I, E] */
    /* router gating (orc_route_gated) */
    int32_t gating;               /* ORC_GATING_* */
    const float *sel_bias;        /* [E] or NULL (kind 1) */
    const float *expert_scale;    /* [E] or NULL */
    float routed_scaling;         /* kind 1 (0 is read as 1) */
    float gate_eps;               /* kind 1 */
    /* shared expert, applied to every token (sh_I = 0: none):
     *   sh[t] = sh_down(act(sh_gate x[t], sh_up x[t])) [* sigmoid(sh_gate_inp . x[t])]
     * nemotronomni_model.cpp:371-376 (relu^2, unscaled), qwen3omni_talker.cpp:396-402
     * (SwiGLU times the sigmoid of a scalar gate row) */
    int32_t sh_I;
    int32_t sh_act;
    int32_t sh_type;              /* type of sh_gate / sh_up */
    const void *sh_gate;          /* ne=[D, sh_I]; RELU_SQR: ffn_up_shexp */
    const void *sh_up;            /* ne=[D, sh_I] or NULL */
    int32_t sh_down_type;
    const void *sh_down;          /* ne=[sh_I, D] */
    const float *sh_gate_inp;     /* F32 [D] or NULL */
} orc_layer;

typedef struct {                  /* optional outputs; any pointer may be NULL */
    float   *logits;              /* [T][E]   */
    int32_t *sel;                 /* [T][K]   */
    float   *w;                   /* [T][K]   */
    int32_t *counts;              /* [E]      */
    int32_t *offsets;             /* [E+1]    */
    int32_t *perm;                /* [T*K]    */
    float   *act;                 /* [T][K][I] */
    float   *ff;                  /* [T][K][D] down outputs before weighting */
    float   *sh;                  /* [T][D] shared expert output (after its gate) */
} orc_debug;

/* out[t] = res[t] + (sum_k w[t][k] * down_{dsel[t][k]}(act(gate_{sel[t][k]} x[t],
 *                                                      up_{sel[t][k]} x[t]))
 *                    + sh[t])
 * res may be NULL (then out = moe only).  exact = 0: ggml semantics;
 * exact = 1: fp64 on dequantized weights with unquantized activations.
 * sel_in / w_in non-NULL: skip the router and use the given routing (the
 * build_expert_ffn_table_res contract, moe_compute.cpp:93-136); down_sel_in
 * non-NULL: the down product's ids (moe_compute.hpp:45, down_ids), else
 * dsel = sel.  Ids outside [0, E) return -1 (ggml asserts them). */
int orc_moe_forward(const orc_layer *L, const float *x, int64_t T,
                    const float *res, float *out, orc_debug *dbg,
                    const int32_t *sel_in, const int32_t *down_sel_in, const float *w_in,
                    int exact, int nthreads);

int orc_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
