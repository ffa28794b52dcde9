/*
 * mi_moe.h - C ABI of the MI355X-native routed mixture-of-experts FFN layer.
 *
 * Plain C types only (device pointers, sizes, ggml-style tensor descriptors);
 * no C++ or torch types cross this boundary.  Every entry point returns an
 * mi_moe_status (0 = success, negative = error) and never synchronizes the
 * stream it is given unless documented.  Device pointers are owned by the
 * caller; the library never frees them.  A context is not thread-safe: use
 * one context per host thread / stream (the same rule as the reference's
 * vqa::Model, src/core/vqa.hpp:121-122).
 *
 * Each entry point names the reference interface it replaces (file:line in
 * SkyVision.cpp).  Type ids follow ggml_type numbering (GGUF type ids), so a
 * ggml backend can pass tensor->type through unchanged.
 */
#ifndef MI_MOE_H
#define MI_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI_MOE_ABI_VERSION 3

/* hipStream_t without pulling in HIP headers */
typedef struct ihipStream_t *mi_stream_t;

typedef enum {
    MI_MOE_OK               = 0,
    MI_MOE_ERR_NULL         = -1,  /* a required pointer is NULL                  */
    MI_MOE_ERR_SHAPE        = -2,  /* shapes / strides inconsistent               */
    MI_MOE_ERR_TYPE         = -3,  /* tensor type not supported by this op        */
    MI_MOE_ERR_CAPACITY     = -4,  /* exceeds what mi_moe_ctx_reserve sized       */
    MI_MOE_ERR_HIP          = -5,  /* a HIP runtime call failed                   */
    MI_MOE_ERR_UNSUPPORTED  = -6,  /* valid request this build does not handle    */
    MI_MOE_ERR_DEVICE       = -7,  /* no such device / device not usable          */
    MI_MOE_ERR_ARG          = -8,  /* other invalid argument (enum out of range)  */
    MI_MOE_ERR_FORMAT       = -9,  /* file missing, unreadable or not valid GGUF  */
} mi_moe_status;

typedef enum {                     /* ggml_type ids */
    MI_TYPE_F32  = 0,
    MI_TYPE_F16  = 1,              /* expert tables: fp16 activations (ggml-cpu vec_dot_type F16) */
    MI_TYPE_Q4_0 = 2,              /*  18 B / 32 values: d f16 | qs[16];          x = d (q - 8)  */
    MI_TYPE_Q5_0 = 6,              /*  22 B / 32 values: d f16 | qh u32 | qs[16]; x = d (q - 16) */
    MI_TYPE_Q8_0 = 8,              /*  34 B / 32 values: d f16 | qs[32] i8;       x = d q        */
    MI_TYPE_Q4_K = 12,             /* 144 B / 256 values, convert/q4k.py:9-10  */
    MI_TYPE_Q6_K = 14,             /* 210 B / 256 values, convert/q6k.py:10-11 */
    MI_TYPE_I32  = 26,
} mi_type;

typedef enum {                     /* activation between the two expert products */
    MI_ACT_SILU          = 0,      /* silu(gate)*up: ggml_swiglu_split, qwen3omni_model.cpp:771     */
    MI_ACT_GELU_ERF_GP1  = 1,      /* gelu_erf(h)*(g+1): geglu_erf_split(h, g+1), moondream.cpp:534 */
    MI_ACT_GELU_TANH     = 2,      /* gelu_tanh(gate)*up                                            */
    MI_ACT_GELU_ERF      = 3,      /* gelu_erf(gate)*up: ggml_mul(ggml_unary(gu, act), up),
                                      moe_compute.cpp:127-129                                       */
    MI_ACT_RELU_SQR      = 4,      /* relu(u)^2 of ONE product, non-gated experts: ggml_sqr(ggml_relu(
                                      mul_mat_id(up_exps, x))), nemotronomni_model.cpp:366-367; the
                                      layer's gate tensor holds ffn_up_exps ne=[D, I, E],
                                      fused_gate_up must be 0 and up is ignored                     */
} mi_act;

typedef enum {
    MI_GATING_SOFTMAX_TOPK = 0,    /* top_k on logits, softmax over the K selected
                                      (moondream.cpp:510-516, qwen3omni_model.cpp:759-766);
                                      times expert_scale[e] when set */
    MI_GATING_SIGMOID_BIAS = 1,    /* s = sigmoid(logit); top_k on s + sel_bias[e] (selection
                                      only); w = s / (sum_K s + gate_eps) * routed_scaling
                                      [* expert_scale[e]] (nemotronomni_model.cpp:344-354) */
    MI_GATING_SOFTMAX_ALL  = 2,    /* p = soft_max over all E logits; top_k on p; w = p / sum_K p
                                      [* expert_scale[e]] (diffusiongemma_model.cpp:923-937): ranks
                                      the probabilities, so logits whose probabilities round to the
                                      same float tie (lower id first) */
} mi_gating;

/* Expert tables of one layer come from one family: the k-quants (Q4_K, Q6_K),
 * the 32-value formats with F16 (Q4_0, Q5_0, Q8_0, F16; rows of a multiple
 * of 32 values, F16 tables 16-byte aligned), or F32.
 * ggml_tensor stand-in: data on the device, ne fastest-first, nb in bytes. */
typedef struct {
    void    *data;
    int32_t  type;                 /* mi_type */
    int64_t  ne[4];
    size_t   nb[4];
} mi_tensor;

/* One MoE FFN layer as the reference binds it (moondream.cpp:241-251,
 * qwen3omni_model.cpp:362-364, convert_hf_to_gguf.py:177-183,
 * convert_qwen3omni.py:188-219). */
typedef struct {
    int32_t n_embd;                /* D */
    int32_t n_expert;              /* E */
    int32_t n_expert_used;         /* K */
    int32_t n_ff;                  /* I (expert inner dim) */
    const float *router_w;         /* F32 ne=[D, E]: E rows of D (ffn_gate_inp.weight) */
    const float *router_b;         /* F32 [E] or NULL (ffn_gate_inp.bias, moondream only) */
    mi_tensor gate;                /* fused_gate_up=1: ffn_up_exps ne=[D, 2I, E], rows [0,I)=h, [I,2I)=g
                                      fused_gate_up=0: ffn_gate_exps ne=[D, I, E] */
    mi_tensor up;                  /* ffn_up_exps ne=[D, I, E]; ignored when fused */
    mi_tensor down;                /* ffn_down_exps ne=[I, D, E] */
    int32_t fused_gate_up;
    int32_t act;                   /* mi_act */
    int32_t gating;                /* mi_gating */
    const float *sel_bias;         /* F32 [E] or NULL: MI_GATING_SIGMOID_BIAS selection bias */
    const float *expert_scale;     /* F32 [E] or NULL: per-expert factor on the weights */
    float routed_scaling;          /* MI_GATING_SIGMOID_BIAS: weight scale (0 is read as 1) */
    float gate_eps;                /* MI_GATING_SIGMOID_BIAS: added to the weight sum */
    /* Shared expert, applied to every token and added to the routed sum before
     * the residual: out = res + (routed + sh), sh = sh_down(act(sh_gate x, sh_up x))
     * [* sigmoid(sh_gate_inp . x)].  nemotronomni: relu^2 on ffn_up_shexp, unscaled
     * (nemotronomni_model.cpp:371-376); qwen3omni talker: SwiGLU times the sigmoid of
     * a scalar gate row (qwen3omni_talker.cpp:396-402).  sh_n_ff = 0: none.  Used by
     * mi_moe_forward / mi_moe_forward_norm; mi_moe_expert_ffn ignores it (the
     * reference's table form has none). */
    int32_t sh_n_ff;
    int32_t sh_act;                /* mi_act of the shared expert */
    mi_tensor sh_gate;             /* ne=[D, sh_n_ff] (ffn_gate_shexp; MI_ACT_RELU_SQR: ffn_up_shexp) */
    mi_tensor sh_up;               /* ne=[D, sh_n_ff]; ignored for MI_ACT_RELU_SQR */
    mi_tensor sh_down;             /* ne=[sh_n_ff, D] */
    const float *sh_gate_inp;      /* F32 [D] or NULL (unscaled) */
    /* Optional tiled copies of the gate / up (Q4_K) and down (Q4_K, Q6_K)
     * tables (mi_moe_tile: the descriptor it returns), read by the grouped
     * GEMMs instead of the tables above (the GEMV and fused decode kernels
     * keep reading those); data = NULL: none.  With separate gate and up
     * tables, both or neither; a fused [h | g] table needs n_ff a multiple
     * of 32.  The output is bit-identical with or without them; qwen3omni's
     * layer at 32 / 64 tokens: 111 / 118 -> 96 / 103 us. */
    mi_tensor gate_tiled, up_tiled, down_tiled;
} mi_moe_layer;

/* Optional routing outputs of mi_moe_forward (device pointers, any may be
 * NULL).  Layouts are row-major with tokens outermost.  Asking for counts,
 * offsets or perm makes small calls (at most 1024 ids on the 32-row GEMM
 * tiles) launch the dispatch kernel that writes them, which the products
 * otherwise do without; the results are bit-identical either way. */
typedef struct {
    float   *logits;               /* [T][E]   router logits                      */
    int32_t *sel;                  /* [T][K]   expert ids, descending logit        */
    float   *weights;              /* [T][K]   softmax over the K selected logits  */
    int32_t *counts;               /* [E]      tokens routed to each expert        */
    int32_t *offsets;              /* [E+1]    exclusive prefix sum of counts      */
    int32_t *perm;                 /* [T*K]    per-expert lists, value t*K+k,
                                               token-ascending within an expert    */
} mi_moe_routing;

/* Row norm of the layer stream in front of the MoE block (the reference
 * normalizes before routing: moondream3 LayerNorm with weight and bias,
 * moondream.cpp:405-407; qwen3omni RMSNorm times ffn_norm,
 * qwen3omni_model.cpp:756-757).  weight / bias: F32 [D] device or NULL; bias
 * is read for MI_NORM_LAYER only. */
typedef enum {
    MI_NORM_NONE  = 0,
    MI_NORM_RMS   = 1,             /* y = x / sqrt(mean(x^2) + eps) [* weight]                  */
    MI_NORM_LAYER = 2,             /* y = (x - mean) / sqrt(var(x) + eps) [* weight] [+ bias]   */
} mi_norm_kind;

typedef struct {
    int32_t      kind;             /* mi_norm_kind */
    float        eps;
    const float *weight;
    const float *bias;
} mi_moe_norm;

typedef struct mi_moe_ctx mi_moe_ctx;

/* ---- context -------------------------------------------------------------
 * Replaces the backend bring-up + graph allocator pre-grow of the reference
 * (moondream.cpp:306-353, gallocr pre-grow :340-351).  Workspace is allocated
 * only by mi_moe_ctx_reserve; forward calls never allocate. */
int  mi_moe_ctx_create(mi_moe_ctx **out, int device);
void mi_moe_ctx_destroy(mi_moe_ctx *ctx);
/* size the workspace for up to max_tokens tokens of layers with these dims
 * (a shared expert's sh_n_ff may be up to n_ff * n_expert_used) */
int  mi_moe_ctx_reserve(mi_moe_ctx *ctx, int64_t max_tokens, int32_t n_embd, int32_t n_ff,
                        int32_t n_expert, int32_t n_expert_used);
/* Errors the GPU found inside calls that returned MI_MOE_OK (the calls do not
 * synchronize, so these are reported afterwards), counted since the last take
 * and then cleared.  bad_ids: caller-supplied expert ids outside [0, E)
 * (mi_moe_expert_ffn, mi_mul_mat_id; ggml_mul_mat_id asserts them).
 * wait_failures: fused single-token calls whose waits gave up (their output
 * is NaN; not expected: a work-group computes what it waited too long for).
 * fp16_saturated: fp16 values of the grouped-GEMM path clamped to +-65504:
 * 256-value Q8_K blocks (input rows or activation rows) whose largest |value|
 * exceeds it, counted per block, and GLU values (the gate/up product's rows,
 * kept as fp16 for the activations' Q8_K) and down-product outputs (the
 * per-slot rows the weighted sum reads, kept as fp16) beyond it, counted per
 * wave of 64 values that held one.  The products of those rows are inexact (ggml's own
 * fp16 GPU paths overflow there; the integer GEMV path has no such limit: a
 * caller that sees fp16_saturated > 0 can run those calls again on it,
 * mi_moe_ctx_set_gemm_threshold(ctx, INT64_MAX): exact integer dots at any
 * token count for layers with n_embd and n_ff <= 2048, slower above the
 * switch).
 * Any pointer may be NULL.  Synchronizes the context's device. */
int  mi_moe_ctx_take_errors(mi_moe_ctx *ctx, int64_t *bad_ids, int64_t *wait_failures,
                            int64_t *fp16_saturated);

/* ---- whole MoE block ------------------------------------------------------
 * out[t] = res[t] + sum_k w[t][k] * down_{sel[t][k]}( act(gate x[t], up x[t]) )
 * Replaces the inline ggml MoE block: router mul_mat(+bias) -> top_k ->
 * get_rows -> soft_max -> mul_mat_id (gate/up) -> GLU -> mul_mat_id (down) ->
 * mul(w) -> permute/cont -> sum_rows (-> add res)
 *   moondream3: src/models/moondream/moondream.cpp:509-544 (+ residual :547)
 *   qwen3omni : src/models/qwen3omni/qwen3omni_model.cpp:759-780
 * x, res, out: F32 [T][D] device; res may be NULL (out = MoE only); out may
 * alias res.  routing may be NULL. */
int mi_moe_forward(mi_moe_ctx *ctx, const mi_moe_layer *layer, const float *x, int64_t n_tokens,
                   const float *res, float *out, const mi_moe_routing *routing,
                   mi_stream_t stream);

/* ---- the block with its own router input -----------------------------------
 * mi_moe_forward whose router reads other rows than the experts: logits =
 * W_r . x_router[t] (+ b), then the layer's gating, and the experts read x[t].
 * diffusiongemma routes on rms_norm(res) * router_scale * scale and feeds the
 * experts rms_norm(res) * ffn_norm2 (diffusiongemma_model.cpp:919-922 against
 * :937).  x_router: F32 [T][D] device; NULL (or x) is mi_moe_forward.  Calls
 * with a separate router input run the kernel chain at every token count
 * (the fused decode kernels quantize one row set for both). */
int mi_moe_forward_router_input(mi_moe_ctx *ctx, const mi_moe_layer *layer, const float *x,
                                const float *x_router, int64_t n_tokens, const float *res, float *out,
                                const mi_moe_routing *routing, mi_stream_t stream);

/* ---- the block with no context and no allocation --------------------------
 * No counterpart in the reference: mi_moe_forward for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  It calls no hipMalloc / hipFree or any
 * allocating routine: its workspace is one file-scope device array of the
 * library per GPU, 16,973,312 bytes, held until the process ends, sized for
 * calls of at most MI_NOALLOC_MAX_TOKENS tokens of layers with n_embd <= 2048,
 * n_ff <= 1024, n_expert <= 128, n_expert_used <= 8 (a shared expert's
 * sh_n_ff <= 8192); larger calls return MI_MOE_ERR_CAPACITY and enqueue
 * nothing.  Single-token calls run the kernel chain (MI_DECODE_CHAIN) and the
 * product path follows the default shape rule, so the results are bit for bit
 * those of mi_moe_forward on a context in MI_DECODE_CHAIN mode.  Every call on
 * a GPU uses that GPU's one array: calls that overlap on one GPU (other streams
 * or host threads) race.  Each call writes every part of the array it reads,
 * so nothing there has to start at zero. */
#define MI_NOALLOC_MAX_TOKENS 64
int mi_moe_forward_noalloc(const mi_moe_layer *layer, const float *x, int64_t n_tokens, const float *res,
                           float *out, const mi_moe_routing *routing, mi_stream_t stream);

/* ---- norm + MoE block in one call ----------------------------------------
 * out[t] = res[t] + MoE(norm(h[t])): the reference's ffn_norm followed by its
 * MoE block (moondream.cpp:405-407 + 509-547; qwen3omni_model.cpp:756-780),
 * in one call: the rows are normalized once into the context's workspace
 * (mi_moe_ctx_reserve sizes it), then the block runs on them; a single token
 * on the fused single-token kernel is normalized inside that kernel (no
 * separate launch).  Same results, bit for bit, as mi_norm into a buffer
 * followed by mi_moe_forward on it.  norm NULL or MI_NORM_NONE: mi_moe_forward.
 * D <= 4096 with a norm (MI_MOE_ERR_UNSUPPORTED beyond). */
int mi_moe_forward_norm(mi_moe_ctx *ctx, const mi_moe_layer *layer, const mi_moe_norm *norm, const float *h,
                        int64_t n_tokens, const float *res, float *out, const mi_moe_routing *routing,
                        mi_stream_t stream);

/* y = norm(x) over each row of n_cols <= 4096 (F32 [n_rows][n_cols] device;
 * y may equal x): the norms of mi_moe_forward_norm as an op (ggml_norm /
 * ggml_rms_norm followed by ggml_mul / ggml_add with the weight and bias). */
int mi_norm(mi_moe_ctx *ctx, const mi_moe_norm *norm, const float *x, int64_t n_rows, int32_t n_cols,
            float *y, mi_stream_t stream);

/* ---- routed FFN with caller-supplied routing ------------------------------
 * Replaces vqa::moe::build_expert_ffn_table_res (src/core/engine/moe_compute.hpp:66-71,
 * moe_compute.cpp:93-136) and the default graph B of the expert-cache decode
 * driver (moe_decode_driver.hpp:503-514):
 *   out = res + sum_k w[k] * down_{down_ids[k]}(act(gate_{gu_ids[k]} x, up_{gu_ids[k]} x))
 * gate_up_ids / down_ids: I32 [T][K] device (may be the same pointer);
 * w: F32 [T][K] device.  The layer's router and shared-expert fields are
 * ignored.  Ids must lie in [0, E): a slot whose gate/up or down id lies
 * outside contributes nothing to its token's sum (the other slots still do)
 * and is counted for mi_moe_ctx_take_errors. */
int mi_moe_expert_ffn(mi_moe_ctx *ctx, const mi_moe_layer *layer, const float *x, int64_t n_tokens,
                      const float *res, const int32_t *gate_up_ids, const int32_t *down_ids,
                      const float *w, float *out, mi_stream_t stream);

/* ---- op-level contracts (ggml op semantics) ------------------------------
 * ggml_top_k(ctx, a F32 ne=[E,T], k) -> I32 ne=[k,T] (moondream.cpp:511,
 * qwen3omni_model.cpp:761): indices of the k largest, descending, ties ->
 * lower index. */
int mi_top_k(mi_moe_ctx *ctx, const mi_tensor *a, int32_t k, mi_tensor *dst, mi_stream_t stream);

/* ggml_mul_mat_id(ctx, as ne=[Kin,N,E], b F32 ne=[Kin, 1|n_used, T],
 * ids I32 ne=[n_used, T]) -> F32 ne=[N, n_used, T]
 * (moondream.cpp:519,537; qwen3omni_model.cpp:769-774; moe_compute.cpp:124-130).
 * dst[:, k, t] = as[:, :, ids[k,t]] . b[:, k % ne11, t].  as types: Q4_K,
 * Q6_K, Q4_0, Q5_0, Q8_0, F16, F32.  b is first converted to the type's ggml
 * vec_dot_type, like ggml-cpu: Q8_K for k-quants, Q8_0 for the 32-value
 * formats, fp16 for F16 (F32 tables take b as given).
 * Ids must lie in [0, E): the dst row of an id outside is written as zeros
 * and the id is counted for mi_moe_ctx_take_errors. */
int mi_mul_mat_id(mi_moe_ctx *ctx, const mi_tensor *as, const mi_tensor *b, const mi_tensor *ids,
                  mi_tensor *dst, mi_stream_t stream);

/* ---- weight preparation ----------------------------------------------------
 * quantize_row_q4_K_ref / quantize_row_q6_K_ref (ggml; ported in
 * convert/q4k.py:27-127 and convert/q6k.py:103-193; called through
 * ggml_quantize_chunk in tools/moe_cpu_bench.cpp:141), quantize_row_q4_0_ref /
 * q5_0_ref / q8_0_ref and the fp16 rounding (the converters' gguf-py
 * quantizers, convert/_lib.py:120-130).  src: F32 [nrows][n_per_row] device
 * (n_per_row a multiple of 256 for k-quants, of 32 otherwise), dst: nrows *
 * row_size bytes device.  Byte-identical to the CPU restatement of ggml's
 * reference quantizers. */
int mi_quantize(mi_moe_ctx *ctx, int32_t type, const float *src, void *dst, int64_t nrows,
                int64_t n_per_row, mi_stream_t stream);

/* ---- tiled copies of expert tables ------------------------------------------
 * Load-time copies of Q4_K and Q6_K expert tables in the grouped GEMMs' order,
 * to attach to a layer (mi_moe_layer.gate_tiled / up_tiled / down_tiled).  No
 * counterpart in the reference (its tables are the GGUF tensors, which this
 * library reads unchanged everywhere else).  src: ne[1] a multiple of 32,
 * rows contiguous (nb[1] = row size, nb[2] = ne[1] nb[1]), 16-byte aligned
 * (Q4_K) / 2-byte aligned (Q6_K).
 *  Q4_K: the same bytes reordered - for every matrix and every 32-row group,
 *   block b (256 values, 144 bytes) of the group's 32 rows as 4608 contiguous
 *   bytes, then block b + 1.  The GEMMs read it as 1 KB runs with consecutive
 *   blocks adjacent, which the memory streams ~1.5x as fast as the rows'
 *   144-byte pieces (load-only probe: 6.1 vs 4.1 TB/s): small batches gain.
 *  Q6_K (down tables): per 32-row group and block b, 9216 bytes: the 6-bit
 *   codes merged into bytes (8 KB, in the order the GEMM's lanes take them)
 *   and the 16 sub-block scales as fp16 d * scale (1 KB); 288 bytes per 256
 *   values instead of 210.  The down GEMM then builds its fp16 operands with
 *   a third fewer instructions (prefill gains).
 * The output of a layer is bit-identical with or without the copies.
 * mi_moe_tiled_bytes: the copy's size in bytes, or a negative mi_moe_status.
 * mi_moe_tile: dst (16-byte aligned, not overlapping src) = the copy; *desc
 * (if not NULL) = its descriptor to attach (type and ne of src; nb of the
 * copy's rows: Q6_K nb[1] = 288 ne[0] / 256). */
int64_t mi_moe_tiled_bytes(const mi_tensor *src);
int mi_moe_tile(mi_moe_ctx *ctx, const mi_tensor *src, void *dst, mi_tensor *desc, mi_stream_t stream);

/* Seeded synthetic N(mean, std^2) fill: value i of (seed, stream_id) does not
 * depend on n or the launch shape.  Counterpart of the reference's seeded
 * test RNG (src/core/test/seg_test.hpp:57-68). */
int mi_fill_normal(mi_moe_ctx *ctx, float *dst, int64_t n, uint64_t seed, uint64_t stream_id,
                   float mean, float stddev, mi_stream_t stream);

/* y = x / sqrt(mean(x^2) + eps) over each row of n_cols <= 4096 (F32
 * [n_rows][n_cols] device; y may equal x): mi_norm with MI_NORM_RMS and no
 * weight.  No counterpart in the reference's MoE path: the
 * norm that feeds the synthetic layer stack (h + MoE(
 * RMSNorm(h)) with attention as identity), written here so the stack runs
 * on one device stream. */
int mi_rmsnorm(mi_moe_ctx *ctx, const float *x, int64_t n_rows, int32_t n_cols, float eps, float *y,
               mi_stream_t stream);

/* ---- GGUF expert tensors (the on-disk side of the path) --------------------
 * Replaces the reference's model load of the MoE tensors: moondream3 binds
 * blk.N.ffn_gate_inp.{weight,bias} (router; F16 promoted to F32,
 * moondream.cpp:149-172, 241-251), blk.N.ffn_up_exps (fused [h | g]) and
 * blk.N.ffn_down_exps as written by convert/convert_hf_to_gguf.py:173-183;
 * qwen3omni's converter writes blk.N.ffn_router, ffn_gate_exps, ffn_up_exps,
 * ffn_down_exps (convert/convert_qwen3omni.py:188-219).  The file is mapped
 * read-only (GGUF v2 / v3); bad or truncated files give MI_MOE_ERR_FORMAT. */
typedef struct mi_gguf mi_gguf;
int  mi_gguf_open(mi_gguf **out, const char *path);
void mi_gguf_close(mi_gguf *gguf);
/* an integer metadata value (any integer or bool type); MI_MOE_ERR_ARG if absent */
int  mi_gguf_get_int(const mi_gguf *gguf, const char *key, int64_t *value);
/* a tensor's ggml type, ne (fastest first, 1-padded) and byte size (0 for
 * types this library does not read); MI_MOE_ERR_ARG if absent */
int  mi_gguf_tensor_info(const mi_gguf *gguf, const char *name, int32_t *type, int64_t ne[4],
                         uint64_t *nbytes);
/* block `block`'s MoE layer uploaded to the current device in one allocation
 * (*device_buffer; free it with mi_dev_free when the layer is no longer
 * used): router (F32), bias if present, expert tables as stored (Q4_K,
 * Q6_K, Q8_0, Q5_0, Q4_0, F16 or F32: one family per layer, the k-quants,
 * the 32-value formats with F16, or F32), K from
 * <general.architecture>.expert_used_count, fused
 * [h | g] when the block has no ffn_gate_exps.  act: mi_act (the
 * architecture's choice: moondream3 MI_ACT_GELU_ERF_GP1, qwen3omni
 * MI_ACT_SILU). */
int  mi_gguf_load_moe_layer(const mi_gguf *gguf, int32_t block, int32_t act, mi_moe_layer *layer,
                            void **device_buffer);

/* ---- introspection ---------------------------------------------------------
 * Per-stage timing (HIP events on the call's stream) for the last forward
 * when profiling is on.  Stage names are static strings. */
int mi_moe_ctx_set_profiling(mi_moe_ctx *ctx, int on);
int mi_moe_ctx_stage_times(mi_moe_ctx *ctx, int max_stages, const char **names, float *ms,
                           int *n_stages);
/* The shader clock (GHz) the CUs ran at under one grouped GEMM of the last
 * forward when profiling is on: stage "gate_up" or "down" of the 4-wave MFMA
 * GEMM path, from each work-group's shader-clock and wall-clock counters at
 * its start and end (summed cycles / summed wall time).  n_wg (may be NULL)
 * receives the work-groups measured.  MI_MOE_ERR_ARG when that stage did not
 * run on the GEMM path.  Synchronizes with the call's stream. */
int mi_moe_ctx_stage_clock(mi_moe_ctx *ctx, const char *stage, double *ghz, int *n_wg);
/* Product path of a call: the grouped MFMA GEMM from min_tokens_for_gemm
 * tokens on, the grouped GEMV below.  0 (the default) picks by shape: for
 * k-quant layers the GEMM when 2 * T * K >= E (from half a dispatched row
 * per expert); for Q4_0 / Q5_0 / Q8_0 / F16 tables and mi_moe_mul_mat_id
 * when 4 * T * K > 5 * E (more than 1.25 rows per expert). */
int mi_moe_ctx_set_gemm_threshold(mi_moe_ctx *ctx, int64_t min_tokens_for_gemm);
/* Row tiles of the grouped GEMMs of Q4_K gate/up layers: 0 (the default) by
 * shape, 32-row tiles when the call dispatches at most 8 rows per expert on
 * average (qwen3omni up to 128 tokens, moondream3 up to 64: several
 * work-groups per CU keep more of the weight stream in flight), and within
 * those 8-row tiles (four work-groups per CU) for the products of Q4_K
 * tables at most 4 rows per expert on average when the call needs no
 * dispatch outputs (up to 1024 slots); 64-row tiles above 8 and up to 48 rows
 * per expert (two work-groups per CU with Q4_K weights, nearly every expert
 * still one tile); 192-row tiles above; 1 192-row tiles,
 * 2 32-row tiles at every size; 3 the skinny products (16-row tiles, one
 * work-group per CU, the weight stream held in registers a group of blocks
 * ahead) on layers whose tables are all Q4_K with n_embd and n_ff <= 2048
 * (others take the shape rule); 4 8-row tiles wherever they apply (else
 * 32-row); 5 64-row tiles at every size.  Kinds 0-2, 4 and 5 give the same
 * bits (the same per-row
 * arithmetic); the skinny products sum each output's products in another
 * order (fp32; the rows agree to ~2e-4 rel-L2 after the activations' fp16
 * and Q8_K roundings). */
int mi_moe_ctx_set_gemm_tiles(mi_moe_ctx *ctx, int kind);
/* Schedule of decode calls of mi_moe_forward (1 token, and batches of 2..16
 * tokens; for experts of more than 2 MiB, batches that dispatch at most one
 * row per expert on average, T * K <= E).  The fused mode runs the whole block in one kernel of one work-group per
 * CU, when the layer fits it (Q4_K gate/up, Q4_K or Q6_K down, top-k <= 8,
 * default gating, no shared expert, 16-byte aligned tables; for batches also
 * n_embd <= 2048 and n_ff <= 1024); other layers and larger batches use the
 * chain.  Inside the kernel, work-groups hand each other
 * the router logits and the gate/up activations through completion words;
 * a work-group that does not see a result after a bounded number of polls
 * computes it itself (the same bits), so the kernel needs no co-residency
 * guarantee and cannot deadlock on a GPU shared with other work.
 *   MI_DECODE_CHAIN              separate kernels
 *   MI_DECODE_FUSED              fused, plain launch (default)
 *   MI_DECODE_FUSED_COOPERATIVE  retired (MI_MOE_ERR_UNSUPPORTED): the fused
 *                                kernel through hipLaunchCooperativeKernel,
 *                                ~18 us slower per call on MI355X than the
 *                                plain launch, which needs no co-residency
 * MI_DECODE_FUSED_EXCLUSIVE is the former name of MI_DECODE_FUSED.
 * Same results in every mode; the reference has one graph per step
 * (moe_decode_driver.hpp:493-514), this only picks the GPU schedule. */
enum {
    MI_DECODE_CHAIN = 0,
    MI_DECODE_FUSED_COOPERATIVE = 1,
    MI_DECODE_FUSED = 2,
    MI_DECODE_FUSED_EXCLUSIVE = 2
};
int mi_moe_ctx_set_fused_decode(mi_moe_ctx *ctx, int mode);
/* Polls a fused single-token work-group makes for another work-group's
 * result before computing that result itself (default 64, about 50 us; the
 * normal waits take under 10 polls).  0 computes every result not ready at
 * the first look (the fallback path, for testing). */
int mi_moe_ctx_set_decode_rescue(mi_moe_ctx *ctx, int polls);
size_t      mi_row_size(int32_t type, int64_t n_per_row);
const char *mi_moe_status_string(int status);
int         mi_moe_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* MI_MOE_H */
