// k_gemv.hip - grouped k-quant GEMV for decode (few tokens per expert).
//
// Computes ggml_mul_mat_id rows (moondream.cpp:519,537; qwen3omni_model.cpp:769-774)
// the way ggml-cpu does for Q4_K / Q6_K weights: activations are Q8_K rows and
// each super-block contributes an exact integer dot scaled in fp32
// (ggml_vec_dot_q4_K_q8_K / _q6_K_q8_K).  Only the experts that received
// tokens are visited (grid.y walks the compact active-expert list), and each
// weight row is streamed once per call whatever the expert's token count.
//
// Wave layout: 8 row groups x 8 lanes.  A row group owns one weight row; its
// 8 lanes split every 256-value super-block into 32-value pieces (16 bytes of
// Q4_K qs, or 8+8+8 bytes of Q6_K ql/qh), so a row group reads each block's
// bytes with contiguous 16-byte loads.  Per token, the lanes dot their piece
// against the token's Q8_K row with v_dot4_i32_i8, scale per block, and the
// 8-lane partials are summed with cross-lane adds.
#include "act.hpp"
#include "common.hpp"
#include "kq_dot.hpp"
#include "launch.hpp"

namespace mimoe {

template <int NB, int WT>
__global__ void __launch_bounds__(256) k_gemv(GemvArgs g) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rs = lane >> 3, sl = lane & 7;
    const int j = blockIdx.y;
    if (j >= *g.n_active) return;
    const int e = g.active_e[j];
    const int cnt = g.counts[e], off = g.offsets[e];
    const bool glu = g.epi == EPI_GLU;
    const int64_t rows_per_wave = glu ? 4 : 8;
    const int64_t col0 = ((int64_t)blockIdx.x * 4 + wave) * rows_per_wave;
    // which matrix row does this row group own?
    int64_t col = col0 + (glu ? (rs & 3) : rs);
    const bool col_ok = col < g.ncols;
    if (!col_ok) col = 0;
    const ExpertMat *M = &g.a;
    int64_t wrow = col;
    if (glu && rs >= 4) {
        if (g.fused) wrow = g.I + col;
        else M = &g.b;
    }
    const uint8_t *rowp = M->data + (int64_t)e * M->mat_bytes + wrow * M->row_bytes;
    const int bbytes = WT == 12 ? Q4K_BYTES : Q6K_BYTES;

    Q4Piece w4[WT == 12 ? NB : 1];
    Q6Piece w6[WT == 14 ? NB : 1];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        if constexpr (WT == 12) load_q4_piece(rowp + b * bbytes, sl, w4[b]);
        else load_q6_piece(rowp + b * bbytes, sl, w6[b]);
    }
    const int64_t Kin = (int64_t)NB * QK;
    for (int m = 0; m < cnt; ++m) {
        const int p = g.perm[off + m];
        const int64_t arow = g.ne11 == 1 ? p / g.K : p;
        const int8_t *q8 = g.q8 + arow * Kin;
        const float *d8 = g.d8 + arow * NB;
        const int16_t *bs = g.bsums + arow * NB * 16;
        float acc = 0.f;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if constexpr (WT == 12) acc += dot_q4_piece(w4[b], sl, q8 + b * QK, d8[b], bs + b * 16);
            else acc += dot_q6_piece(w6[b], sl, q8 + b * QK, d8[b]);
        }
        acc += __shfl_xor(acc, 1, 64);
        acc += __shfl_xor(acc, 2, 64);
        acc += __shfl_xor(acc, 4, 64);
        if (glu) {
            const float other = __shfl(acc, lane + 32 < 64 ? lane + 32 : lane, 64);
            if (rs < 4 && sl == 0 && col_ok) g.y[(int64_t)p * g.ldy + col] = act_pair(g.act, acc, other);
        } else {
            if (sl == 0 && col_ok) g.y[(int64_t)p * g.ldy + col] = acc;
        }
    }
}

// fp32 expert tables (F32 ggml tensors): y = W_e . b_row in sequential fp32,
// the ggml-cpu F32 vec_dot semantics the CPU oracle restates
__global__ void __launch_bounds__(256) k_mm_id_f32(GemvArgs g, const float *b, int64_t ldb) {
    const int j = blockIdx.y;
    if (j >= *g.n_active) return;
    const int e = g.active_e[j];
    const int cnt = g.counts[e], off = g.offsets[e];
    const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= g.a.N) return;
    const float *wr = (const float *)(g.a.data + (int64_t)e * g.a.mat_bytes + n * g.a.row_bytes);
    for (int m = 0; m < cnt; ++m) {
        const int p = g.perm[off + m];
        const int64_t brow = g.ne11 == 1 ? p / g.K : p;
        const float *bb = b + brow * ldb;
        float acc = 0.f;
        for (int64_t q = 0; q < g.a.K; ++q) acc += wr[q] * bb[q];
        g.y[(int64_t)p * g.ldy + n] = acc;
    }
}

// act[r][i] = act_pair(h[r][i], g[r][i]) for the fp32 path
__global__ void __launch_bounds__(256) k_glu_rows(const float *h, int64_t ldh, const float *gg, int64_t ldg,
                                                  float *out, int64_t ldo, int64_t rows, int64_t I, int act) {
    const int64_t total = rows * I;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = idx / I, i = idx - r * I;
        out[r * ldo + i] = act_pair(act, h[r * ldh + i], gg[r * ldg + i]);
    }
}

template <int WT>
static void launch_gemv_nb(int nb, dim3 grid, const GemvArgs &g, hipStream_t st) {
    switch (nb) {
    case 1: hipLaunchKernelGGL((k_gemv<1, WT>), grid, dim3(256), 0, st, g); break;
    case 2: hipLaunchKernelGGL((k_gemv<2, WT>), grid, dim3(256), 0, st, g); break;
    case 3: hipLaunchKernelGGL((k_gemv<3, WT>), grid, dim3(256), 0, st, g); break;
    case 4: hipLaunchKernelGGL((k_gemv<4, WT>), grid, dim3(256), 0, st, g); break;
    case 5: hipLaunchKernelGGL((k_gemv<5, WT>), grid, dim3(256), 0, st, g); break;
    case 6: hipLaunchKernelGGL((k_gemv<6, WT>), grid, dim3(256), 0, st, g); break;
    case 7: hipLaunchKernelGGL((k_gemv<7, WT>), grid, dim3(256), 0, st, g); break;
    case 8: hipLaunchKernelGGL((k_gemv<8, WT>), grid, dim3(256), 0, st, g); break;
    default: break;
    }
}

int launch_gemv(const GemvArgs &g, hipStream_t st) {
    if (g.max_active <= 0) return 0;
    const int nb = (int)(g.a.K / QK);
    if (nb < 1 || nb > 8 || g.a.K % QK) return -6;
    const int64_t per_block = (g.epi == EPI_GLU ? 4 : 8) * 4;
    const dim3 grid((unsigned)((g.ncols + per_block - 1) / per_block), (unsigned)g.max_active);
    if (g.a.type == 12) launch_gemv_nb<12>(nb, grid, g, st);
    else if (g.a.type == 14) launch_gemv_nb<14>(nb, grid, g, st);
    else return -3;
    return hip_check_launch();
}

int launch_mm_id_f32(const GemvArgs &g, const float *b, int64_t ldb, hipStream_t st) {
    if (g.max_active <= 0) return 0;
    const dim3 grid((unsigned)((g.a.N + 255) / 256), (unsigned)g.max_active);
    hipLaunchKernelGGL(k_mm_id_f32, grid, dim3(256), 0, st, g, b, ldb);
    return hip_check_launch();
}

int launch_glu_rows(const float *h, int64_t ldh, const float *gg, int64_t ldg, float *out, int64_t ldo,
                    int64_t rows, int64_t I, int act, hipStream_t st) {
    if (rows <= 0) return 0;
    const int64_t total = rows * I;
    const int64_t blocks = (total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096;
    hipLaunchKernelGGL(k_glu_rows, dim3((unsigned)blocks), dim3(256), 0, st, h, ldh, gg, ldg, out, ldo, rows, I,
                       act);
    return hip_check_launch();
}

}  // namespace mimoe
