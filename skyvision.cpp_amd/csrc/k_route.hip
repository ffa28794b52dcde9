// k_route.hip - activation Q8_K quantization, router logits, top-k gating,
// token -> expert dispatch and the weighted combine.
//
// Reference ops (SkyVision.cpp):
//   router    ggml_add(ggml_mul_mat(router_w, l), router_b)   moondream.cpp:510
//             ggml_mul_mat(L.router, m)                       qwen3omni_model.cpp:759
//   top_k     ggml_top_k(rlogits, K)                          moondream.cpp:511
//   softmax   ggml_get_rows + ggml_soft_max                   moondream.cpp:512-515
//   dispatch  row grouping inside ggml_mul_mat_id (ggml-cpu)   moondream.cpp:519,537
//   combine   mul(ff3, w) -> permute/cont -> sum_rows (-> add) moondream.cpp:540-543
// Q8_K is ggml's vec_dot_type for Q4_K / Q6_K: ggml-cpu quantizes the F32
// activation rows to it before the integer dot.
#include "act.hpp"
#include "common.hpp"
#include "wave_ops.hpp"
#include "launch.hpp"
#include "q8h.hpp"

namespace mimoe {

// ---------------------------------------------------------------- Q8_K rows
// One wave per (row, group of 4 blocks): lane l holds values 16 (l % 16) ..
// + 15 of block 4 grp + l / 16 (q8k_wave4x16: every block's reduction in one
// instruction stream, each lane's 16 codes one ggml bsums entry).  Outputs:
// codes (natural order, 16 B per lane), scales, block sums, and fp16 values
// (d*q, or q when exact) in the consumer's MFMA K order through a wave-private
// LDS copy of the codes (sq: 4 * QK bytes, sd: 4 floats, private to the wave).
// XO fixes the fp16 order at compile time: XO_Q4 / XO_Q6 the 32x32x16 order of
// a Q4_K / Q6_K consumer (not exact), where a lane's 16 positions are the
// bytes of four aligned code dwords (at base and base + 32 for each of its two
// lane groups), XO_ANY whatever o asks for, element by element.

// the lane's 16 values of row group (row, grp) (zeros past the row's blocks)
template <bool VEC, typename ST>
__device__ __forceinline__ void q8k_load(const ST *__restrict__ src, int64_t ld, int64_t row, int grp, int nb,
                                         int lane, float (&v)[16], int pre_act = 0) {
    const int bl = lane >> 4, l16 = lane & 15;
    const int b = 4 * grp + bl;
    if (b < nb) {
        const ST *x = src + row * ld + (int64_t)b * QK + 16 * l16;
        if constexpr (sizeof(ST) == 2) {
            // fp16 rows: 32 bytes per lane
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint4 u = *(const uint4 *)(x + 8 * j);
                const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const half2_t hh = __builtin_bit_cast(half2_t, w[i]);
                    v[8 * j + 2 * i] = (float)hh[0];
                    v[8 * j + 2 * i + 1] = (float)hh[1];
                }
            }
        } else if (VEC) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 f = *(const float4 *)(x + 4 * j);
                v[4 * j] = f.x; v[4 * j + 1] = f.y; v[4 * j + 2] = f.z; v[4 * j + 3] = f.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = x[i];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = 0.f;
    }
    if (pre_act == ACT_RELU_SQR) {
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = relu_sqr(v[i]);
    }
}

template <int XO>
__device__ __forceinline__ void q8k_quant(const float (&v)[16], int64_t row, int grp, int nb, const Q8Out &o,
                                          int8_t *sq, float *sd, int lane) {
    int8_t *__restrict__ q8 = o.q8;
    float *__restrict__ d8 = o.d8;
    int16_t *__restrict__ bsums = o.bsums;
    _Float16 *__restrict__ xh = o.xh;
    _Float16 *__restrict__ xbs = o.xbs;
    const int wtype = o.wtype, order = o.order, exact = o.exact;
    const int bl = lane >> 4, l16 = lane & 15;
    const int b = 4 * grp + bl;
    const bool bok = b < nb;
    const int64_t K = (int64_t)nb * QK;
    int q[16], bsum;
    const float d = q8k_wave4x16(v, lane, q, bsum);
    uint32_t pk[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int qq[4] = {q[4 * j], q[4 * j + 1], q[4 * j + 2], q[4 * j + 3]};
        pk[j] = pack_i8x4(qq);
    }
    if (bok) {
        const int64_t off = row * K + (int64_t)b * QK + 16 * l16;
        if (q8) *(uint4 *)(q8 + off) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        if (d8 && l16 == 0) d8[row * nb + b] = d;
        const int64_t bi = row * (K / 16) + (int64_t)b * 16 + l16;
        if (bsums) bsums[bi] = (int16_t)bsum;
        if (xbs) xbs[bi] = (_Float16)(float)bsum;        // |s| <= 2032: exact in fp16
    }
    if (xh) {
        wave_lds_sync();   // a previous item's reads of sq / sd are done
        *(uint4 *)&sq[bl * QK + 16 * l16] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        if (l16 == 0) sd[bl] = d;
        wave_lds_sync();
        if (bok && l16 == 0 && !exact && o.range_total && f16_over(d)) atomicAdd(o.range_total, 1);
        if (bok && XO != XO_ANY) {
            const float db = sd[bl];
            const int s = l16;
            uint32_t h[8];
#pragma unroll
            for (int g = 0; g < 2; ++g) {
                const int base = XO == XO_Q4 ? 64 * (2 * (s >> 3) + g) + 4 * (s & 7)
                                             : 128 * (s >> 3) + 16 * g + 4 * ((s & 7) >> 1) + 64 * (s & 1);
                const uint32_t A = *(const uint32_t *)&sq[bl * QK + base];
                const uint32_t B = *(const uint32_t *)&sq[bl * QK + base + 32];
                // slot p = 0..7 of the lane group: Q4_K bytes A0 A2 B0 B2 A1 A3 B1 B3
                // (q4k_elem32's offsets 0 2 32 34 1 3 33 35), Q6_K A0..A3 B0..B3
                int q[8];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int sh = XO == XO_Q4 ? 16 * (k & 1) + 8 * (k >> 1) : 8 * k;
                    const int slot = XO == XO_Q4 ? (k & 1) + 4 * (k >> 1) : k;
                    q[slot] = (int)(int8_t)(A >> sh);
                    q[slot + (XO == XO_Q4 ? 2 : 4)] = (int)(int8_t)(B >> sh);
                }
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    half2_t hh;
                    hh[0] = f16_sat(db * (float)q[2 * k]);
                    hh[1] = f16_sat(db * (float)q[2 * k + 1]);
                    h[4 * g + k] = __builtin_bit_cast(uint32_t, hh);
                }
            }
            uint4 *dst = (uint4 *)(xh + row * K + (int64_t)b * QK + 16 * l16);
            dst[0] = make_uint4(h[0], h[1], h[2], h[3]);
            dst[1] = make_uint4(h[4], h[5], h[6], h[7]);
        } else if (bok) {
            const float db = sd[bl];
            uint32_t h[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                float qv[2];
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int p = 16 * l16 + 2 * i + j;
                    const int el = order ? mfma32_elem(wtype, p) : mfma_elem(wtype, p);
                    const float qf = (float)sq[bl * QK + el];
                    qv[j] = exact ? qf : db * qf;
                }
                half2_t hh;
                hh[0] = f16_sat(qv[0]);
                hh[1] = f16_sat(qv[1]);
                h[i] = __builtin_bit_cast(uint32_t, hh);
            }
            uint4 *dst = (uint4 *)(xh + row * K + (int64_t)b * QK + 16 * l16);
            dst[0] = make_uint4(h[0], h[1], h[2], h[3]);
            dst[1] = make_uint4(h[4], h[5], h[6], h[7]);
        }
    }
}

template <bool VEC, int XO>
__device__ __forceinline__ void q8k_row_group(const float *__restrict__ src, int64_t ld, int64_t row, int grp,
                                              int nb, const Q8Out &o, int8_t *sq, float *sd, int lane) {
    float v[16];
    q8k_load<VEC>(src, ld, row, grp, nb, lane, v);
    q8k_quant<XO>(v, row, grp, nb, o, sq, sd, lane);
}

// Items (row groups) per wave, all loaded before the first is quantized.  One
// is fastest for the 8192 x 1024 GLU rows of a 1024-token moondream3 layer
// (two: 12.6 vs 11.1 us; the wave count halves).
constexpr int Q8_ITEMS = 1;

template <bool VEC, int XO, typename ST>
__global__ void __launch_bounds__(256) k_q8k_rows(const ST *__restrict__ src, int64_t ld, int64_t nrows,
                                                  int nb, Q8Out o) {
    __shared__ __attribute__((aligned(16))) int8_t sq[4][4 * QK];
    __shared__ float sd[4][4];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int ngrp = (nb + 3) >> 2;
    const int64_t n_items = nrows * ngrp;
    const int64_t item0 = ((int64_t)blockIdx.x * 4 + wave) * Q8_ITEMS;
    if (item0 >= n_items) return;   // whole waves; only wave-local exchanges follow
    float v[Q8_ITEMS][16];
#pragma unroll
    for (int u = 0; u < Q8_ITEMS; ++u) {
        const int64_t item = item0 + u < n_items ? item0 + u : item0;
        const int64_t row = item / ngrp;
        q8k_load<VEC>(src, ld, row, (int)(item - row * ngrp), nb, lane, v[u], o.pre_act);
    }
#pragma unroll
    for (int u = 0; u < Q8_ITEMS; ++u) {
        const int64_t item = item0 + u;
        if (item >= n_items) break;
        const int64_t row = item / ngrp;
        q8k_quant<XO>(v[u], row, (int)(item - row * ngrp), nb, o, sq[wave], sd[wave], lane);
    }
}

// fp16 values only (o.xh in a Q4_K / Q6_K 32x32x16 order, no codes, scales or
// sums): one wave per row group of 4 blocks, 16 lanes per block, each lane
// loading its 16 values straight in the output order (q8h.hpp).
template <int XO, typename ST>
__global__ void __launch_bounds__(256) k_q8k_rows_h(const ST *__restrict__ src, int64_t ld, int64_t nrows, int nb,
                                                    Q8Out o) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int ngrp = (nb + 3) >> 2;
    const int64_t item = (int64_t)blockIdx.x * 4 + wave;
    if (item >= nrows * ngrp) return;   // whole waves; only DPP exchanges follow
    const int64_t row = ngrp == 1 ? item : item / ngrp;
    const int grp = (int)(item - row * ngrp);
    const int bl = lane >> 4, s = lane & 15;
    const int b = 4 * grp + bl;
    const bool bok = b < nb;
    float v[16];
    if (bok) {
        q8h_gather<XO>(src + row * ld + (int64_t)b * QK, s, v);
        if (o.pre_act == ACT_RELU_SQR) {
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = relu_sqr(v[i]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = 0.f;
    }
    q8h_quant_store(v, bok, o.xh + row * (int64_t)nb * QK + (int64_t)b * QK, s, o.range_total);
}

// the compile-time fp16 order for o (XO_ANY when o has no xh)
inline int q8_xo(const Q8Out &o) {
    if (!o.xh || !o.order || o.exact) return XO_ANY;
    return o.wtype == 12 ? XO_Q4 : o.wtype == 14 ? XO_Q6 : XO_ANY;
}

// o asks for the fp16 values alone (k_q8k_rows_h)
inline bool q8_h_only(const Q8Out &o, int xo) {
    return xo != XO_ANY && !o.q8 && !o.d8 && !o.bsums && !o.xbs;
}

int launch_q8k_rows(const float *src, int64_t ld, int64_t nrows, int64_t K, const Q8Out &o, hipStream_t st) {
    if (nrows <= 0) return 0;
    const int nb = (int)(K / QK);
    const int64_t items = nrows * ((nb + 3) / 4);
    const bool vec = (ld % 4 == 0) && ((uintptr_t)src % 16 == 0);
    const dim3 grid((unsigned)((items + 4 * Q8_ITEMS - 1) / (4 * Q8_ITEMS)));
    const int xo = q8_xo(o);
    // fp16 values alone: whole 256-value blocks (each lane's runs are 4 floats)
    const bool h_only = vec && q8_h_only(o, xo) && K % QK == 0;
    if (h_only && xo == XO_Q4) hipLaunchKernelGGL((k_q8k_rows_h<XO_Q4, float>), grid, dim3(256), 0, st, src, ld, nrows, nb, o);
    else if (h_only) hipLaunchKernelGGL((k_q8k_rows_h<XO_Q6, float>), grid, dim3(256), 0, st, src, ld, nrows, nb, o);
    else if (vec && xo == XO_Q4) hipLaunchKernelGGL((k_q8k_rows<true, XO_Q4, float>), grid, dim3(256), 0, st, src, ld, nrows, nb, o);
    else if (vec && xo == XO_Q6) hipLaunchKernelGGL((k_q8k_rows<true, XO_Q6, float>), grid, dim3(256), 0, st, src, ld, nrows, nb, o);
    else if (vec) hipLaunchKernelGGL((k_q8k_rows<true, XO_ANY, float>), grid, dim3(256), 0, st, src, ld, nrows, nb, o);
    else hipLaunchKernelGGL((k_q8k_rows<false, XO_ANY, float>), grid, dim3(256), 0, st, src, ld, nrows, nb, o);
    return hip_check_launch();
}

// fp16 rows (the grouped GEMM's GLU rows): whole 256-value blocks, 16-byte
// aligned rows
int launch_q8k_rows(const _Float16 *src, int64_t ld, int64_t nrows, int64_t K, const Q8Out &o, hipStream_t st) {
    if (nrows <= 0) return 0;
    if (K % QK || ld % 8 || (uintptr_t)src % 16) return -6;
    const int nb = (int)(K / QK);
    const int64_t items = nrows * ((nb + 3) / 4);
    const dim3 grid((unsigned)((items + 4 * Q8_ITEMS - 1) / (4 * Q8_ITEMS)));
    const int xo = q8_xo(o);
    if (q8_h_only(o, xo) && xo == XO_Q4) hipLaunchKernelGGL((k_q8k_rows_h<XO_Q4, _Float16>), grid, dim3(256), 0, st, src, ld, nrows, nb, o);
    else if (q8_h_only(o, xo)) hipLaunchKernelGGL((k_q8k_rows_h<XO_Q6, _Float16>), grid, dim3(256), 0, st, src, ld, nrows, nb, o);
    else if (xo == XO_Q4) hipLaunchKernelGGL((k_q8k_rows<true, XO_Q4, _Float16>), grid, dim3(256), 0, st, src, ld, nrows, nb, o);
    else if (xo == XO_Q6) hipLaunchKernelGGL((k_q8k_rows<true, XO_Q6, _Float16>), grid, dim3(256), 0, st, src, ld, nrows, nb, o);
    else hipLaunchKernelGGL((k_q8k_rows<true, XO_ANY, _Float16>), grid, dim3(256), 0, st, src, ld, nrows, nb, o);
    return hip_check_launch();
}

// ---------------------------------------------------------------- router
// logit = fl32( fl32(sum_c part_c) + b ) in fp64, one fixed order: the 64-wide
// chunk c gives part_c = sum over s = 0..15 (outer), g = 0..3 (inner) of
// W[e][64c+16g+s] * x[t][64c+16g+s] added left to right; chunk partials are
// added left to right.  fp32 x fp32 products are exact in fp64, so fma and
// mul+add agree and only this order matters.
//
// MFMA form: v_mfma_f64_16x16x4_f64 adds its four k-products to the
// accumulator one after another in k order (c + p0 + p1 + p2 + p3), so one
// instruction per s with k = g reproduces the chunk order exactly.  A wave owns
// a 16 token x 16 expert tile and whole chunks; the chunk partials meet in LDS
// and are summed in chunk order.
typedef double double4_t __attribute__((ext_vector_type(4)));
constexpr int RM_MAX_CHUNKS = 32;   // D <= 2048 (64 KB of LDS partials)

// Grid: one work-group (16 waves) per (16-token slab, 16-expert tile); the
// slab's expert tiles run on one XCD (slab s on XCD s % 8, work-groups dealt
// to the XCDs in turn), so each token's row is fetched into one L2 only.
//
// Loads: a chunk's 16 x rows and 16 W rows (64 floats each) arrive by
// coalesced loads (lane l: row 4 j + l / 16, 16-byte piece l % 16, so one
// instruction covers 4 rows x 256 B) and pass through a wave-private LDS
// stage (piece p of row r at slot p ^ r: conflict-free both ways) into the
// MFMA operand layout (lane (row, g): pieces 4 g .. 4 g + 3 of its row).  The
// next chunk's loads go out once the current one is in operand registers,
// and land while its 16 MFMAs run.
constexpr int RT_WAVES = 16;

struct RtChunk {
    float4 x[4], w[4];
};

template <bool VEC>
__device__ __forceinline__ float4 rt_piece(const float *row, int64_t off, int D, bool ok) {
    if (VEC) return ok ? *(const float4 *)(row + off) : make_float4(0.f, 0.f, 0.f, 0.f);
    float t[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) t[i] = ok && off + i < D ? row[off + i] : 0.f;
    return make_float4(t[0], t[1], t[2], t[3]);
}

// chunk c of the slab's x rows (t0 ..) and the tile's W rows (e0 ..); rows
// past T or E read as zeros
template <bool VEC>
__device__ __forceinline__ void rt_load(RtChunk &k, const float *__restrict__ x, int64_t ldx, int64_t t0, int64_t T,
                                        const float *__restrict__ W, int e0, int E, int D, int c, int lane) {
    const int64_t off = 64 * (int64_t)c + 4 * (lane & 15);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = 4 * j + (lane >> 4);
        const bool tok_ok = t0 + r < T, ex_ok = e0 + r < E;
        k.x[j] = rt_piece<VEC>(x + (tok_ok ? t0 + r : 0) * ldx, off, D, tok_ok);
        k.w[j] = rt_piece<VEC>(W + (int64_t)(ex_ok ? e0 + r : 0) * D, off, D, ex_ok);
    }
}

// a wave's four loaded pieces -> its lane's 16 operand values (stage: 256 float4)
__device__ __forceinline__ void rt_transpose(const float4 (&in)[4], float4 *stage, int lane, float (&out)[16]) {
    const int p = lane & 15;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = 4 * j + (lane >> 4);
        stage[r * 16 + (p ^ r)] = in[j];
    }
    wave_lds_sync();
    const int row = lane & 15, g = lane >> 4;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 v = stage[row * 16 + ((4 * g + q) ^ row)];
        out[4 * q] = v.x; out[4 * q + 1] = v.y; out[4 * q + 2] = v.z; out[4 * q + 3] = v.w;
    }
    wave_lds_sync();   // the stage is rewritten next
}

// The front of a forward: every work-group computes its logit tile, and with
// a Q8_K output (o.q8 or o.xh set) quantizes its share of the slab's x rows
// (row group item i = row * ngrp + grp by work-group i % net, wave i / net
// mod 16) while the rows are in this XCD's L2.  (Ranking the slab in the last
// of its work-groups to finish was measured slower than the separate top-k
// launch: the logit hand-off costs three memory round trips at the kernel's
// end.)
template <bool VEC, int XO>
__global__ void __launch_bounds__(1024) k_front(const float *__restrict__ W, const float *__restrict__ bias,
                                                const float *__restrict__ x, int64_t ldx, int64_t T, int D, int E,
                                                float *__restrict__ logits, Q8Out o) {
    __shared__ double rparts[RM_MAX_CHUNKS * 256];   // [chunk][256]
    __shared__ float4 stage[RT_WAVES][256];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nch = (D + 63) / 64;
    const int net = (E + 15) / 16;
    const int lin = blockIdx.x, q = lin >> 3;
    const int64_t slab = (int64_t)(q / net) * 8 + (lin & 7);
    if (slab * 16 >= T) return;
    const int et = q % net, e0 = et * 16;
    const int64_t t0 = slab * 16;
    float4 *stg = stage[wave];
    RtChunk cur;
    if (wave < nch) rt_load<VEC>(cur, x, ldx, t0, T, W, e0, E, D, wave, lane);
    for (int c = wave; c < nch; c += RT_WAVES) {
        float xv[16], wv[16];
        rt_transpose(cur.x, stg, lane, xv);
        rt_transpose(cur.w, stg, lane, wv);
        if (c + RT_WAVES < nch) rt_load<VEC>(cur, x, ldx, t0, T, W, e0, E, D, c + RT_WAVES, lane);
        double4_t part = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int s2 = 0; s2 < 16; ++s2)
            part = __builtin_amdgcn_mfma_f64_16x16x4f64((double)xv[s2], (double)wv[s2], part, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) rparts[c * 256 + lane * 4 + r] = part[r];
    }
    if (o.q8 || o.xh) {
        const int nb = D / QK, ngrp = (nb + 3) >> 2;
        for (int i = et + net * wave; i < 16 * ngrp; i += net * RT_WAVES) {
            const int64_t row = t0 + i / ngrp;
            if (row >= T) continue;
            int8_t *sq = (int8_t *)stg;
            float *sd = (float *)(stg + 64);
            if (XO == XO_Q4) q8k_row_group<VEC, XO_Q4>(x, ldx, row, i % ngrp, nb, o, sq, sd, lane);
            else q8k_row_group<VEC, XO_ANY>(x, ldx, row, i % ngrp, nb, o, sq, sd, lane);
        }
    }
    __syncthreads();
    if (threadIdx.x < 256) {
        // output slot (lane l, r) holds token row 4r + l/16, expert col l%16
        const int l = threadIdx.x >> 2, r = threadIdx.x & 3;
        const int64_t tt = t0 + 4 * r + (l >> 4);
        const int ee = e0 + (l & 15);
        // chunk partials added in chunk order, eight loads in flight
        double acc = 0.0;
        int c = 0;
        for (; c + 8 <= nch; c += 8) {
            double v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = rparts[(c + j) * 256 + threadIdx.x];
#pragma unroll
            for (int j = 0; j < 8; ++j) acc = acc + v[j];
        }
        for (; c < nch; ++c) acc = acc + rparts[c * 256 + threadIdx.x];
        if (tt < T && ee < E) {
            float v = (float)acc;
            if (bias) v = v + bias[ee];
            logits[tt * E + ee] = v;
        }
    }
}

// Small batches: with few 16 x 16 (token, expert) tiles k_front leaves most
// CUs idle while each of its work-groups runs the tile's D / 64 chunk chains
// (32 at D = 2048, ~4 us of fp64 MFMA on one CU).  Here a tile's chunks are
// dealt to nsp work-groups of cps waves (work-group 8 q + x: tile q / nsp,
// split q % nsp; chunk split * cps + wave); each wave computes its chunk's
// 16 x 16 partial exactly as k_front does and stores it to parts[c][t][e]
// (fp64); k_topk_parts adds a token's partials in chunk order, so the logits
// are bit-identical to k_front's.  The Q8_K of x is dealt to the slab's
// work-groups as in k_front.
template <bool VEC, int XO>
__global__ void __launch_bounds__(1024) k_front_parts(const float *__restrict__ W, const float *__restrict__ x,
                                                      int64_t ldx, int64_t T, int D, int E, int cps,
                                                      double *__restrict__ parts, Q8Out o) {
    __shared__ float4 stage[RT_WAVES][256];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nch = (D + 63) / 64, net = (E + 15) / 16, nsp = (nch + cps - 1) / cps;
    const int lin = blockIdx.x;
    const int split = lin % nsp, q = lin / nsp, et = q % net;
    const int64_t t0 = (int64_t)(q / net) * 16;
    const int e0 = et * 16;
    float4 *stg = stage[wave];
    const int c = split * cps + wave;
    if (c < nch) {
        RtChunk cur;
        rt_load<VEC>(cur, x, ldx, t0, T, W, e0, E, D, c, lane);
        float xv[16], wv[16];
        rt_transpose(cur.x, stg, lane, xv);
        rt_transpose(cur.w, stg, lane, wv);
        double4_t part = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int s2 = 0; s2 < 16; ++s2)
            part = __builtin_amdgcn_mfma_f64_16x16x4f64((double)xv[s2], (double)wv[s2], part, 0, 0, 0);
        // slot (lane, r): token row 4 r + lane / 16, expert column lane % 16
        const int ee = e0 + (lane & 15);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t tt = t0 + 4 * r + (lane >> 4);
            if (tt < T && ee < E) parts[((int64_t)c * T + tt) * E + ee] = part[r];
        }
    }
    if (o.q8 || o.xh) {
        const int nb = D / QK, ngrp = (nb + 3) >> 2;
        const int nwg = net * nsp, wg = et * nsp + split, nw = (int)(blockDim.x >> 6);
        for (int i = wg + nwg * wave; i < 16 * ngrp; i += nwg * nw) {
            const int64_t row = t0 + i / ngrp;
            if (row >= T) continue;
            int8_t *sq = (int8_t *)stg;
            float *sd = (float *)(stg + 64);
            if (XO == XO_Q4) q8k_row_group<VEC, XO_Q4>(x, ldx, row, i % ngrp, nb, o, sq, sd, lane);
            else q8k_row_group<VEC, XO_ANY>(x, ldx, row, i % ngrp, nb, o, sq, sd, lane);
        }
    }
}

// generic form (any D): thread (expert, chunk) computes one partial
__global__ void __launch_bounds__(256) k_router_split(const float *__restrict__ W, const float *__restrict__ bias,
                                                      const float *__restrict__ x, int64_t ldx, int D, int E,
                                                      int nch, int epb, float *__restrict__ logits) {
    __shared__ double parts[256];
    const int tid = threadIdx.x;
    const int el = tid / nch, c = tid % nch;
    const int64_t t = blockIdx.y;
    const int e = blockIdx.x * epb + el;
    const bool act = el < epb && e < E;
    double part = 0.0;
    if (act) {
        const float *w = W + (int64_t)e * D;
        const float *xt = x + t * ldx;
        for (int s = 0; s < 16; ++s)
            for (int g = 0; g < 4; ++g) {
                const int dd = 64 * c + 16 * g + s;
                if (dd < D) part = fma((double)w[dd], (double)xt[dd], part);
            }
    }
    parts[tid] = part;
    __syncthreads();
    if (act && c == 0) {
        double acc = 0.0;
        for (int j = 0; j < nch; j++) acc = acc + parts[el * nch + j];
        float v = (float)acc;
        if (bias) v = v + bias[e];
        logits[t * E + e] = v;
    }
}

int launch_front(const float *W, const float *b, const float *x, int64_t ldx, int64_t T, int D, int E,
                 float *logits, const Q8Out *qx, hipStream_t st) {
    if (T <= 0) return 0;
    const int nch = (D + 63) / 64;
    if (nch > RM_MAX_CHUNKS || T > (int64_t)1 << 30) return -6;
    if (qx && D % QK) return -6;
    const bool vec = (D % 64 == 0) && (ldx % 4 == 0) && ((uintptr_t)x % 16 == 0) && ((uintptr_t)W % 16 == 0);
    const int64_t net = (E + 15) / 16, nslab = (T + 15) / 16;
    const int64_t blocks = 8 * net * ((nslab + 7) / 8);
    if (blocks > 0x7fffffff) return -6;
    const Q8Out o = qx ? *qx : Q8Out{};
    if (vec && q8_xo(o) == XO_Q4)
        hipLaunchKernelGGL((k_front<true, XO_Q4>), dim3((unsigned)blocks), dim3(64 * RT_WAVES), 0, st, W, b, x, ldx,
                           T, D, E, logits, o);
    else if (vec)
        hipLaunchKernelGGL((k_front<true, XO_ANY>), dim3((unsigned)blocks), dim3(64 * RT_WAVES), 0, st, W, b, x,
                           ldx, T, D, E, logits, o);
    else
        hipLaunchKernelGGL((k_front<false, XO_ANY>), dim3((unsigned)blocks), dim3(64 * RT_WAVES), 0, st, W, b, x,
                           ldx, T, D, E, logits, o);
    return hip_check_launch();
}

int launch_front_parts(const float *W, const float *x, int64_t ldx, int64_t T, int D, int E, int cps,
                       double *parts, const Q8Out *qx, hipStream_t st) {
    if (T <= 0) return 0;
    const int nch = (D + 63) / 64;
    if (nch > RM_MAX_CHUNKS || cps < 1 || cps > RT_WAVES || T > (int64_t)1 << 24) return -6;
    if (qx && D % QK) return -6;
    const bool vec = (D % 64 == 0) && (ldx % 4 == 0) && ((uintptr_t)x % 16 == 0) && ((uintptr_t)W % 16 == 0);
    const int64_t nsp = (nch + cps - 1) / cps, net = (E + 15) / 16, nslab = (T + 15) / 16;
    const int64_t blocks = nslab * net * nsp;
    if (blocks > 0x7fffffff) return -6;
    const Q8Out o = qx ? *qx : Q8Out{};
    const dim3 grid((unsigned)blocks), block((unsigned)(64 * cps));
    if (vec && q8_xo(o) == XO_Q4)
        hipLaunchKernelGGL((k_front_parts<true, XO_Q4>), grid, block, 0, st, W, x, ldx, T, D, E, cps, parts, o);
    else if (vec)
        hipLaunchKernelGGL((k_front_parts<true, XO_ANY>), grid, block, 0, st, W, x, ldx, T, D, E, cps, parts, o);
    else
        hipLaunchKernelGGL((k_front_parts<false, XO_ANY>), grid, block, 0, st, W, x, ldx, T, D, E, cps, parts, o);
    return hip_check_launch();
}

int launch_router(const float *W, const float *b, const float *x, int64_t ldx, int64_t T, int D, int E,
                  float *logits, hipStream_t st) {
    if (T <= 0) return 0;
    const int nch = (D + 63) / 64;
    if (nch <= RM_MAX_CHUNKS && T <= (int64_t)1 << 30)
        return launch_front(W, b, x, ldx, T, D, E, logits, nullptr, st);
    if (nch > 256 || T > 65535) return -6;
    const int epb = 256 / nch;
    hipLaunchKernelGGL(k_router_split, dim3((unsigned)((E + epb - 1) / epb), (unsigned)T), dim3(256), 0, st, W, b,
                       x, ldx, D, E, nch, epb, logits);
    return hip_check_launch();
}

// ---------------------------------------------------------------- top-k
// One wave per token: top-k by K rounds of the wave's largest remaining
// value (largest value, lowest id on ties; topk_softmax_wave), then softmax
// over the K selected logits: max, expf(v - max), sum in fp64 in slot order,
// scale by (float)(1.0 / sum) - the ggml_soft_max order.
__global__ void __launch_bounds__(256) k_topk_softmax(const float *__restrict__ logits, int64_t ldl, int64_t T,
                                                      int E, int K, int32_t *__restrict__ sel, int64_t lds,
                                                      float *__restrict__ w, Gating gt) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t t = (int64_t)blockIdx.x * 4 + wave;
    if (t >= T) return;   // whole waves; the routine works inside its own wave
    int mysel;
    float myw;
    topk_softmax_wave(logits + t * ldl, E, K, lane, mysel, myw, w != nullptr, gt);
    if (lane < K) {
        sel[t * lds + lane] = mysel;
        if (w) w[t * K + lane] = myw;
    }
}

int launch_topk_softmax(const float *logits, int64_t ld_logits, int64_t T, int E, int K, int32_t *sel,
                        int64_t ld_sel, float *w, hipStream_t st, const Gating &gt) {
    if (T <= 0) return 0;
    if (E > 64 * TOPK_MAX_PER_LANE || K > 64 || K > E || K <= 0) return -6;
    if (gt.kind < 0 || gt.kind > 2) return -6;
    hipLaunchKernelGGL(k_topk_softmax, dim3((unsigned)((T + 3) / 4)), dim3(256), 0, st, logits, ld_logits, T, E,
                       K, sel, ld_sel, w, gt);
    return hip_check_launch();
}

// The same on the chunk partials of k_front_parts, one token per wave and
// work-group (E <= 64 NPER): lane l first adds its experts' partials in
// chunk order (fp64, as k_front: every load issued before the first add),
// rounds to fp32, adds the bias and writes the logits.
template <int NPER>
__global__ void __launch_bounds__(64) k_topk_parts(const double *__restrict__ parts, int nch,
                                                   const float *__restrict__ bias, float *__restrict__ logits,
                                                   int64_t T, int E, int K, int32_t *__restrict__ sel, int64_t lds,
                                                   float *__restrict__ w, Gating gt) {
    static_assert(NPER <= TOPK_MAX_PER_LANE, "experts per lane");
    const int lane = threadIdx.x;
    const int64_t t = blockIdx.x;
    const int64_t cs = T * E;
    double pv[NPER][RM_MAX_CHUNKS];
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
        const int e = lane + 64 * i;
        const double *p = parts + t * E + (e < E ? e : 0);
        // branch-free: chunks past nch re-load the last one (never added), so
        // no load waits for an earlier one (nch >= 1)
#pragma unroll
        for (int c = 0; c < RM_MAX_CHUNKS; ++c) pv[i][c] = p[(int64_t)(c < nch ? c : nch - 1) * cs];
    }
    float raw[TOPK_MAX_PER_LANE];
#pragma unroll
    for (int i = 0; i < TOPK_MAX_PER_LANE; ++i) raw[i] = 0.f;
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
        const int e = lane + 64 * i;
        double acc = 0.0;
#pragma unroll
        for (int c = 0; c < RM_MAX_CHUNKS; ++c)
            if (c < nch) acc = acc + pv[i][c];
        float v = (float)acc;
        if (e < E) {
            if (bias) v = v + bias[e];
            raw[i] = v;
            logits[t * E + e] = v;
        }
    }
    int mysel;
    float myw;
    topk_softmax_regs(raw, E, K, lane, mysel, myw, w != nullptr, gt);
    if (lane < K) {
        sel[t * lds + lane] = mysel;
        if (w) w[t * K + lane] = myw;
    }
}

int launch_topk_parts(const double *parts, int D, const float *bias, float *logits, int64_t T, int E, int K,
                      int32_t *sel, int64_t ld_sel, float *w, hipStream_t st, const Gating &gt) {
    if (T <= 0) return 0;
    if (E > 128 || K > 64 || K > E || K <= 0 || T > 0x7fffffff) return -6;
    if (gt.kind < 0 || gt.kind > 2) return -6;
    const int nch = (D + 63) / 64;
    if (nch > RM_MAX_CHUNKS) return -6;
    if (E <= 64)
        hipLaunchKernelGGL(k_topk_parts<1>, dim3((unsigned)T), dim3(64), 0, st, parts, nch, bias, logits, T, E, K, sel,
                           ld_sel, w, gt);
    else
        hipLaunchKernelGGL(k_topk_parts<2>, dim3((unsigned)T), dim3(64), 0, st, parts, nch, bias, logits, T, E, K, sel,
                           ld_sel, w, gt);
    return hip_check_launch();
}

// ---------------------------------------------------------------- dispatch
// One work-group of 1024 threads per expert.  The ids pass through LDS in
// chunks of at most DISPATCH_IDS (coalesced loads); every work-group counts
// all of them (LDS atomics), scans the counts, writes its own expert's entries
// (count, offset, GEMM tiles, active-list slot), and then lists its expert's
// slots in flat (t*K + k) order: per 1024 ids, a wave ballot of the ids equal
// to the expert, wave totals in LDS, positions = running base + waves before
// + lanes before.  The list is the stable counting sort of the flat ids
// (token-ascending, then slot-ascending; ids repeated inside a token keep
// their slot order).  Ids outside [0, E) are counted in bad_ids and skipped.
// GEMM tiles of at most BM rows: every expert's full tiles first (expert
// order), then one partial tile per expert with cnt % BM rows, by decreasing
// row count (ties: lower expert first), so the longest work-groups start
// first; or (balanced) ceil(cnt / BM) equal tiles per expert.
constexpr int DISPATCH_THREADS = 1024;
constexpr int DISPATCH_WAVES = DISPATCH_THREADS / 64;
constexpr int DISPATCH_MAX_E = 256;
constexpr int DISPATCH_IDS = 8192;                         // ids per staged chunk (32 KB)

// ids[0 .. m) -> sid (m <= DISPATCH_IDS); independent loads, one latency
__device__ __forceinline__ void dispatch_stage(const int32_t *__restrict__ src, int m, int *sid, int tid) {
    int v[DISPATCH_IDS / DISPATCH_THREADS];
#pragma unroll
    for (int j = 0; j < DISPATCH_IDS / DISPATCH_THREADS; ++j) {
        const int i = j * DISPATCH_THREADS + tid;
        v[j] = i < m ? src[i] : 0;
    }
#pragma unroll
    for (int j = 0; j < DISPATCH_IDS / DISPATCH_THREADS; ++j) {
        const int i = j * DISPATCH_THREADS + tid;
        if (i < m) sid[i] = v[j];
    }
}

__global__ void __launch_bounds__(DISPATCH_THREADS) k_dispatch(const int32_t *__restrict__ ids, int64_t n, int E,
                                                               int BM, int balanced, Dispatch d) {
    __shared__ int cnt[DISPATCH_MAX_E];   // counts
    __shared__ int scn[DISPATCH_MAX_E];   // inclusive scan of counts
    __shared__ int tsc[DISPATCH_MAX_E];   // inclusive scan of full (or balanced) tiles
    __shared__ int asc[DISPATCH_MAX_E];   // inclusive scan of active flags
    __shared__ int psc[DISPATCH_MAX_E];   // inclusive scan of partial-tile flags
    __shared__ int sid[DISPATCH_IDS];
    __shared__ int wsum[DISPATCH_WAVES];
    __shared__ int bad, prank;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int me = blockIdx.x;
    const bool one_chunk = n <= DISPATCH_IDS;

    for (int e = tid; e < E; e += DISPATCH_THREADS) cnt[e] = 0;
    if (tid == 0) bad = 0;
    for (int64_t c0 = 0; c0 < n; c0 += DISPATCH_IDS) {
        const int m = (int)(c0 + DISPATCH_IDS < n ? DISPATCH_IDS : n - c0);
        if (c0 > 0) __syncthreads();   // the previous chunk's counting is done
        dispatch_stage(ids + c0, m, sid, tid);
        __syncthreads();
        for (int i = tid; i < m; i += DISPATCH_THREADS) {
            const int e = sid[i];
            if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
            else atomicAdd(&bad, 1);
        }
    }
    __syncthreads();
    if (tid < E) {
        scn[tid] = cnt[tid];
        tsc[tid] = balanced ? (cnt[tid] + BM - 1) / BM : cnt[tid] / BM;
        asc[tid] = cnt[tid] > 0 ? 1 : 0;
        psc[tid] = !balanced && cnt[tid] % BM > 0 ? 1 : 0;
    }
    __syncthreads();
    if (wave < 4) {   // four inclusive scans, one per wave: lane l holds entries 4 l .. 4 l + 3
        int *arr = wave == 0 ? scn : wave == 1 ? tsc : wave == 2 ? asc : psc;
        int v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = 4 * lane + j < E ? arr[4 * lane + j] : 0;
        v[1] += v[0]; v[2] += v[1]; v[3] += v[2];
        const int ex = wave_incl_scan(v[3]) - v[3];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (4 * lane + j < E) arr[4 * lane + j] = v[j] + ex;
    }
    __syncthreads();
    const int c = cnt[me];
    const int off = scn[me] - c;
    if (tid == 0) {
        d.counts[me] = c;
        d.offsets[me] = off;
        if (c > 0) d.active_e[asc[me] - 1] = me;
        if (me == 0) {
            d.offsets[E] = scn[E - 1];
            *d.n_tiles = tsc[E - 1] + psc[E - 1];
            *d.n_active = asc[E - 1];
            *d.bad_ids = bad;
            if (bad > 0 && d.bad_total) atomicAdd(d.bad_total, bad);
        }
    }
    if (me == 0 && bad > 0 && d.zero_rows) {
        // no product writes the rows of ids outside [0, E): zeros, one row per thread
        for (int64_t i = tid; i < n; i += DISPATCH_THREADS) {
            const int e = ids[i];
            if (e < 0 || e >= E) {
                float *row = d.zero_rows + i * d.zero_ld;
                for (int64_t c2 = 0; c2 < d.zero_n; ++c2) row[c2] = 0.f;
            }
        }
    }
    // balanced tiles: nt of them, the first `extra` with base + 1 rows
    const int nt = balanced ? (c + BM - 1) / BM : 0, tb = balanced ? tsc[me] - nt : 0;
    const int base = nt ? c / nt : 0, extra = c - base * nt;
    const bool tperm = balanced && d.tile_perm && BM <= GS_BM;
    if (balanced) {
        for (int j = tid; j < nt; j += DISPATCH_THREADS) {
            const int r0 = j * base + (j < extra ? j : extra);
            d.tile_e[tb + j] = me;
            d.tile_r0[tb + j] = r0;
            d.tile_start[tb + j] = off + r0;
            d.tile_rows[tb + j] = base + (j < extra ? 1 : 0);
        }
    } else {
        const int nf = c / BM, rem = c - nf * BM;
        const int tb = tsc[me] - nf;
        for (int j = tid; j < nf; j += DISPATCH_THREADS) {
            d.tile_e[tb + j] = me;
            d.tile_r0[tb + j] = j * BM;
            d.tile_start[tb + j] = off + j * BM;
            d.tile_rows[tb + j] = BM;
        }
        if (rem > 0) {
            // rank among the partial tiles: one expert per thread, summed in LDS
            if (tid == 0) prank = 0;
            __syncthreads();
            if (tid < E) {
                const int r2 = cnt[tid] % BM;
                if ((r2 > rem) | ((r2 == rem) & (tid < me))) atomicAdd(&prank, 1);
            }
            __syncthreads();
            if (tid == 0) {
                d.tile_e[tsc[E - 1] + prank] = me;
                d.tile_r0[tsc[E - 1] + prank] = nf * BM;
                d.tile_start[tsc[E - 1] + prank] = off + nf * BM;
                d.tile_rows[tsc[E - 1] + prank] = rem;
            }
        }
    }

    // the expert's slots in flat order
    int run = off;
    for (int64_t c0 = 0; c0 < n; c0 += DISPATCH_IDS) {
        const int m = (int)(c0 + DISPATCH_IDS < n ? DISPATCH_IDS : n - c0);
        if (!one_chunk) {
            __syncthreads();   // every wave is done with the previous chunk
            dispatch_stage(ids + c0, m, sid, tid);
            __syncthreads();
        }
        // wave w takes the contiguous ids [w0, w1) (at most NIT rounds of 64):
        // its hit masks, the other waves met once for the prefix, then the
        // hits written in order from the masks
        const int span = ((m + DISPATCH_WAVES - 1) / DISPATCH_WAVES + 63) & ~63;
        const int w0 = wave * span, w1 = w0 + span < m ? w0 + span : m;
        constexpr int NIT = DISPATCH_IDS / DISPATCH_WAVES / 64;
        uint64_t hm[NIT];
        int mine = 0;
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int i = w0 + 64 * it + lane;
            const int e = i < w1 ? sid[i] : -1;
            hm[it] = __ballot(e == me);
            mine += __popcll(hm[it]);
        }
        if (lane == 0) wsum[wave] = mine;
        __syncthreads();
        int before = 0, total = 0;
#pragma unroll
        for (int w = 0; w < DISPATCH_WAVES; ++w) {
            const int v = wsum[w];
            before += w < wave ? v : 0;
            total += v;
        }
        int pos = run + before;
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const uint64_t mask = hm[it];
            if ((mask >> lane) & 1ull) {
                const int at = pos + __popcll(mask & ((1ull << lane) - 1ull));
                const int32_t val = (int32_t)(c0 + w0 + 64 * it + lane);
                d.perm[at] = val;
                if (tperm) {
                    // the entry's tile j and row within it (rank r in the expert's list)
                    const int r = at - off, r1 = extra * (base + 1);
                    const int j = r < r1 ? r / (base + 1) : extra + (r - r1) / base;
                    const int r0 = j * base + (j < extra ? j : extra);
                    d.tile_perm[(int64_t)(tb + j) * GS_BM + (r - r0)] = val;
                }
            }
            pos += __popcll(mask);
        }
        run += total;
        __syncthreads();   // wsum (and sid) are rewritten for the next chunk
    }
}

int launch_dispatch(const int32_t *ids, int64_t T, int K, int E, int BM, int balanced, const Dispatch &d,
                    hipStream_t st) {
    if (E <= 0 || E > DISPATCH_MAX_E || K <= 0 || BM <= 0) return -6;
    hipLaunchKernelGGL(k_dispatch, dim3((unsigned)E), dim3(DISPATCH_THREADS), 0, st, ids, T * (int64_t)K, E, BM,
                       balanced, d);
    return hip_check_launch();
}

// ---------------------------------------------------------------- combine
// moe[t][n] = (float)( sum_k (double)(z[t*K+k][n] * w[t][k]) ) over the live
// slots in slot order (+ add[t][n] in fp32); out = res + moe.  A slot is dead
// when a caller-supplied id of it lies outside [0, E): nothing wrote its z row.
__device__ __forceinline__ bool combine_live(const CombineIds &ci, int64_t i) {
    if (!ci.a) return true;
    const int a = ci.a[i], b = ci.b[i];
    return ((unsigned)a < (unsigned)ci.E) & ((unsigned)b < (unsigned)ci.E);
}

template <typename ZT>
__global__ void __launch_bounds__(256) k_combine(const ZT *__restrict__ z, const float *__restrict__ w,
                                                 const float *res, float *out, int64_t T, int K, int D,
                                                 CombineIds ci, const float *__restrict__ add) {
    const int64_t total = T * (int64_t)D;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = idx / D;
        const int n = (int)(idx - t * D);
        double s = 0.0;
        for (int k = 0; k < K; ++k) {
            if (!combine_live(ci, t * K + k)) continue;
            const float prod = (float)z[(t * K + k) * D + n] * w[t * K + k];
            s = s + (double)prod;
        }
        float moe = (float)s;
        if (add) moe = moe + add[idx];
        out[idx] = res ? res[idx] + moe : moe;
    }
}

// Vector form: work-group (column chunk, token), 4 consecutive columns per
// thread; the K slot rows' loads are issued before the (slot-order) sums.
__device__ __forceinline__ float4 load4(const float *p) { return *(const float4 *)p; }
__device__ __forceinline__ float4 load4(const _Float16 *p) {
    const uint2 u = *(const uint2 *)p;
    const half2_t a = __builtin_bit_cast(half2_t, u.x), b = __builtin_bit_cast(half2_t, u.y);
    return make_float4((float)a[0], (float)a[1], (float)b[0], (float)b[1]);
}
template <int KMAX, typename ZT>
__global__ void __launch_bounds__(256) k_combine4(const ZT *__restrict__ z, const float *__restrict__ w,
                                                  const float *__restrict__ res, float *__restrict__ out, int K,
                                                  int D, CombineIds ci, const float *__restrict__ add) {
    const int64_t t = blockIdx.y;
    const int n = 4 * ((int)blockIdx.x * 256 + (int)threadIdx.x);
    if (n >= D) return;
    float4 zv[KMAX];
#pragma unroll
    for (int k = 0; k < KMAX; ++k)
        if (k < K) zv[k] = load4(z + (t * K + k) * (int64_t)D + n);
    double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
        if (k < K && combine_live(ci, t * K + k)) {
            const float wk = w[t * K + k];
            s0 = s0 + (double)(zv[k].x * wk);
            s1 = s1 + (double)(zv[k].y * wk);
            s2 = s2 + (double)(zv[k].z * wk);
            s3 = s3 + (double)(zv[k].w * wk);
        }
    }
    float4 o = make_float4((float)s0, (float)s1, (float)s2, (float)s3);
    if (add) {
        const float4 a = *(const float4 *)(add + t * D + n);
        o.x = o.x + a.x; o.y = o.y + a.y; o.z = o.z + a.z; o.w = o.w + a.w;
    }
    if (res) {
        const float4 r = *(const float4 *)(res + t * D + n);
        o.x = r.x + o.x; o.y = r.y + o.y; o.z = r.z + o.z; o.w = r.w + o.w;
    }
    *(float4 *)(out + t * D + n) = o;
}

// fp16 slot rows: 8 consecutive columns per thread (16-byte loads of each
// slot row, two float4 stores)
template <int KMAX>
__global__ void __launch_bounds__(256) k_combine8h(const _Float16 *__restrict__ z, const float *__restrict__ w,
                                                   const float *__restrict__ res, float *__restrict__ out, int K,
                                                   int D, CombineIds ci, const float *__restrict__ add) {
    const int64_t t = blockIdx.y;
    const int n = 8 * ((int)blockIdx.x * 256 + (int)threadIdx.x);
    if (n >= D) return;
    uint4 zv[KMAX];
#pragma unroll
    for (int k = 0; k < KMAX; ++k)
        if (k < K) zv[k] = *(const uint4 *)(z + (t * K + k) * (int64_t)D + n);
    double s[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
        if (k < K && combine_live(ci, t * K + k)) {
            const float wk = w[t * K + k];
            const uint32_t u[4] = {zv[k].x, zv[k].y, zv[k].z, zv[k].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const half2_t h = __builtin_bit_cast(half2_t, u[j]);
                s[2 * j] = s[2 * j] + (double)((float)h[0] * wk);
                s[2 * j + 1] = s[2 * j + 1] + (double)((float)h[1] * wk);
            }
        }
    }
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        float4 o = make_float4((float)s[4 * hh], (float)s[4 * hh + 1], (float)s[4 * hh + 2], (float)s[4 * hh + 3]);
        if (add) {
            const float4 a = *(const float4 *)(add + t * D + n + 4 * hh);
            o.x = o.x + a.x; o.y = o.y + a.y; o.z = o.z + a.z; o.w = o.w + a.w;
        }
        if (res) {
            const float4 r = *(const float4 *)(res + t * D + n + 4 * hh);
            o.x = r.x + o.x; o.y = r.y + o.y; o.z = r.z + o.z; o.w = r.w + o.w;
        }
        *(float4 *)(out + t * D + n + 4 * hh) = o;
    }
}

template <typename ZT>
static int combine_t(const ZT *z, const float *w, const float *res, float *out, int64_t T, int K, int D,
                     hipStream_t st, const CombineIds &ci, const float *add) {
    if constexpr (sizeof(ZT) == 2) {
        const bool vec8 = D % 8 == 0 && (uintptr_t)z % 16 == 0 && (uintptr_t)out % 16 == 0 &&
                          (!res || (uintptr_t)res % 16 == 0) && (!add || (uintptr_t)add % 16 == 0) && T <= 65535;
        if (vec8 && K <= 16) {
            const dim3 grid((unsigned)((D / 8 + 255) / 256), (unsigned)T);
            if (K <= 8) hipLaunchKernelGGL((k_combine8h<8>), grid, dim3(256), 0, st, z, w, res, out, K, D, ci, add);
            else hipLaunchKernelGGL((k_combine8h<16>), grid, dim3(256), 0, st, z, w, res, out, K, D, ci, add);
            return hip_check_launch();
        }
    }
    const bool vec = D % 4 == 0 && (uintptr_t)z % (4 * sizeof(ZT)) == 0 && (uintptr_t)out % 16 == 0 &&
                     (!res || (uintptr_t)res % 16 == 0) && (!add || (uintptr_t)add % 16 == 0) && T <= 65535;
    if (vec && K <= 16) {
        const dim3 grid((unsigned)((D / 4 + 255) / 256), (unsigned)T);
        if (K <= 8) hipLaunchKernelGGL((k_combine4<8, ZT>), grid, dim3(256), 0, st, z, w, res, out, K, D, ci, add);
        else hipLaunchKernelGGL((k_combine4<16, ZT>), grid, dim3(256), 0, st, z, w, res, out, K, D, ci, add);
        return hip_check_launch();
    }
    const int64_t total = T * (int64_t)D;
    const int64_t blocks = (total + 255) / 256 < 8192 ? (total + 255) / 256 : 8192;
    hipLaunchKernelGGL(k_combine<ZT>, dim3((unsigned)blocks), dim3(256), 0, st, z, w, res, out, T, K, D, ci, add);
    return hip_check_launch();
}

int launch_combine(const float *z, const float *w, const float *res, float *out, int64_t T, int K, int D,
                   hipStream_t st, const CombineIds &ci, const float *add, const _Float16 *zh) {
    if (T <= 0) return 0;
    return z ? combine_t(z, w, res, out, T, K, D, st, ci, add) : combine_t(zh, w, res, out, T, K, D, st, ci, add);
}

// ---------------------------------------------------------------- shared expert
// The shared expert runs as a one-expert layer whose every token selects
// expert 0 with weight 1, or with the sigmoid of its scalar gate row
// (qwen3omni_talker.cpp:399-401), evaluated in fp64 and rounded once.
__global__ void __launch_bounds__(256) k_shared_gate(const float *__restrict__ logit, int64_t T,
                                                     int32_t *__restrict__ ids, float *__restrict__ w) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= T) return;
    ids[t] = 0;
    w[t] = logit ? gating_sigmoid(logit[t]) : 1.f;
}

int launch_shared_gate(const float *logit, int64_t T, int32_t *ids, float *w, hipStream_t st) {
    if (T <= 0) return 0;
    hipLaunchKernelGGL(k_shared_gate, dim3((unsigned)((T + 255) / 256)), dim3(256), 0, st, logit, T, ids, w);
    return hip_check_launch();
}

}  // namespace mimoe
