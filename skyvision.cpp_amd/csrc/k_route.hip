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
#include "common.hpp"
#include "launch.hpp"

namespace mimoe {

// ---------------------------------------------------------------- Q8_K rows
// One wave per (row, 256-block).  Lane l holds elements 4l..4l+3.
__global__ void __launch_bounds__(256) k_q8k_rows(const float *__restrict__ src, int64_t ld, int64_t nrows,
                                                  int nb, int8_t *__restrict__ q8, float *__restrict__ d8,
                                                  int16_t *__restrict__ bsums, _Float16 *__restrict__ xh,
                                                  int wtype) {
    __shared__ int8_t sq[4][QK];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t item = (int64_t)blockIdx.x * 4 + wave;
    const bool valid = item < nrows * nb;
    const int64_t row = valid ? item / nb : 0;
    const int b = valid ? (int)(item % nb) : 0;
    const int64_t K = (int64_t)nb * QK;

    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (valid) {
        const float *x = src + row * ld + (int64_t)b * QK + 4 * lane;
        for (int j = 0; j < 4; ++j) v[j] = x[j];
    }
    AmaxIdx a{-1.f, 1 << 30, 0.f};
    for (int j = 0; j < 4; ++j) {
        AmaxIdx c{fabsf(v[j]), 4 * lane + j, v[j]};
        a = amax_better(a, c);
    }
    a = wave_amax_idx(a);
    const float amax = a.ax, max = a.val;
    int q[4] = {0, 0, 0, 0};
    float d = 0.f;
    if (amax != 0.f) {
        const float iscale = -127.f / max;
        for (int j = 0; j < 4; ++j) q[j] = imin(127, nearest_int(iscale * v[j]));
        d = 1 / iscale;
    }
    if (valid) {
        const int64_t o = row * K + (int64_t)b * QK + 4 * lane;
        if (q8) {
            const uint32_t packed = (uint32_t)(uint8_t)q[0] | ((uint32_t)(uint8_t)q[1] << 8) |
                                    ((uint32_t)(uint8_t)q[2] << 16) | ((uint32_t)(uint8_t)q[3] << 24);
            *(uint32_t *)(q8 + o) = packed;
        }
        if (d8 && lane == 0) d8[row * nb + b] = d;
    }
    if (bsums) {
        int s = q[0] + q[1] + q[2] + q[3];
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        if (valid && (lane & 3) == 0) bsums[row * (K / 16) + (int64_t)b * 16 + (lane >> 2)] = (int16_t)s;
    }
    if (xh) {
        for (int j = 0; j < 4; ++j) sq[wave][4 * lane + j] = (int8_t)q[j];
        __syncthreads();
        if (valid) {
            half2_t h01, h23;
            const int p0 = 4 * lane;
            h01[0] = (_Float16)(d * (float)sq[wave][mfma_elem(wtype, p0 + 0)]);
            h01[1] = (_Float16)(d * (float)sq[wave][mfma_elem(wtype, p0 + 1)]);
            h23[0] = (_Float16)(d * (float)sq[wave][mfma_elem(wtype, p0 + 2)]);
            h23[1] = (_Float16)(d * (float)sq[wave][mfma_elem(wtype, p0 + 3)]);
            uint2 pk;
            pk.x = __builtin_bit_cast(uint32_t, h01);
            pk.y = __builtin_bit_cast(uint32_t, h23);
            *(uint2 *)(xh + row * K + (int64_t)b * QK + p0) = pk;
        }
    }
}

int launch_q8k_rows(const float *src, int64_t ld, int64_t nrows, int64_t K, const Q8Out &o, hipStream_t st) {
    if (nrows <= 0) return 0;
    const int nb = (int)(K / QK);
    const int64_t items = nrows * nb;
    hipLaunchKernelGGL(k_q8k_rows, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, st, src, ld, nrows, nb, o.q8,
                       o.d8, o.bsums, o.xh, o.wtype);
    return hip_check_launch();
}

// ---------------------------------------------------------------- router
// logit = fl32( fl32(sum_c part_c) + b ), part_c = sequential fp64 sum over the
// 64-wide chunk c, chunk partials summed left to right.  fp32 x fp32 products
// are exact in fp64, so fma and mul+add agree and only the order matters.

// split form (small T): thread (expert, chunk) computes one partial
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
        const int d0 = c * 64, d1 = imin(D, d0 + 64);
        for (int dd = d0; dd < d1; dd++) part = fma((double)w[dd], (double)xt[dd], part);
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

// tile form (large T): a block holds TT = (256/E)*4 tokens and every expert;
// thread (expert e, group gi) accumulates 4 tokens.  W and x are staged in LDS
// one 64-wide chunk at a time.
constexpr int RT_TPT = 4;
__global__ void __launch_bounds__(256) k_router_tile(const float *__restrict__ W, const float *__restrict__ bias,
                                                     const float *__restrict__ x, int64_t ldx, int64_t T, int D,
                                                     int E, float *__restrict__ logits) {
    extern __shared__ float rsm[];
    const int G = 256 / E;
    const int TT = G * RT_TPT;
    float *Ws = rsm;               // [E][65]
    float *xs = rsm + E * 65;      // [TT][64]
    const int tid = threadIdx.x;
    const int e = tid % E, gi = tid / E;
    const bool act = gi < G;
    const int64_t t0 = (int64_t)blockIdx.x * TT;
    double acc[RT_TPT];
    for (int j = 0; j < RT_TPT; ++j) acc[j] = 0.0;
    for (int c0 = 0; c0 < D; c0 += 64) {
        const int cl = imin(64, D - c0);
        for (int i = tid; i < E * 64; i += 256) {
            const int r = i >> 6, cc = i & 63;
            Ws[r * 65 + cc] = cc < cl ? W[(int64_t)r * D + c0 + cc] : 0.f;
        }
        for (int i = tid; i < TT * 64; i += 256) {
            const int r = i >> 6, cc = i & 63;
            const int64_t tok = t0 + r;
            xs[r * 64 + cc] = (tok < T && cc < cl) ? x[tok * ldx + c0 + cc] : 0.f;
        }
        __syncthreads();
        if (act) {
            for (int j = 0; j < RT_TPT; ++j) {
                const int tl = gi + G * j;
                double part = 0.0;
                for (int dd = 0; dd < cl; ++dd)
                    part = fma((double)Ws[e * 65 + dd], (double)xs[tl * 64 + dd], part);
                acc[j] = acc[j] + part;
            }
        }
        __syncthreads();
    }
    if (act) {
        for (int j = 0; j < RT_TPT; ++j) {
            const int64_t tok = t0 + gi + G * j;
            if (tok < T) {
                float v = (float)acc[j];
                if (bias) v = v + bias[e];
                logits[tok * E + e] = v;
            }
        }
    }
}

int launch_router(const float *W, const float *b, const float *x, int64_t ldx, int64_t T, int D, int E,
                  float *logits, hipStream_t st) {
    if (T <= 0) return 0;
    const int nch = (D + 63) / 64;
    if (T >= 32 && E >= 16 && E <= 256) {   // LDS: E*65 + (256/E)*4*64 floats <= 64 KB
        const int G = 256 / E;
        const int TT = G * RT_TPT;
        const size_t smem = sizeof(float) * ((size_t)E * 65 + (size_t)TT * 64);
        hipLaunchKernelGGL(k_router_tile, dim3((unsigned)((T + TT - 1) / TT)), dim3(256), smem, st, W, b, x, ldx,
                           T, D, E, logits);
    } else {
        if (nch > 256) return -6;
        const int epb = 256 / nch;
        hipLaunchKernelGGL(k_router_split, dim3((unsigned)((E + epb - 1) / epb), (unsigned)T), dim3(256), 0, st, W,
                           b, x, ldx, D, E, nch, epb, logits);
    }
    return hip_check_launch();
}

// ---------------------------------------------------------------- top-k
// One wave per token.  K rounds of a wave arg-max (largest value, lowest id on
// ties) over the not-yet-taken experts; then softmax over the K selected
// logits: max, expf(v - max), sum in fp64 in slot order, scale by
// (float)(1.0 / sum) - the ggml_soft_max order.
constexpr int TOPK_MAX_PER_LANE = 4;   // E <= 256
__global__ void __launch_bounds__(256) k_topk_softmax(const float *__restrict__ logits, int64_t ldl, int64_t T,
                                                      int E, int K, int32_t *__restrict__ sel, int64_t lds,
                                                      float *__restrict__ w) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t t = (int64_t)blockIdx.x * 4 + wave;
    if (t >= T) return;
    const float *l = logits + t * ldl;
    float v[TOPK_MAX_PER_LANE];
    bool avail[TOPK_MAX_PER_LANE];
    for (int i = 0; i < TOPK_MAX_PER_LANE; ++i) {
        const int e = lane + 64 * i;
        avail[i] = e < E;
        v[i] = avail[i] ? l[e] : 0.f;
    }
    int mysel = 0;
    float myval = 0.f;
    for (int k = 0; k < K; ++k) {
        float bv = 0.f;
        int bi = 0x7fffffff;
        for (int i = 0; i < TOPK_MAX_PER_LANE; ++i) {
            const int e = lane + 64 * i;
            if (avail[i] && (bi == 0x7fffffff || v[i] > bv)) {
                bv = v[i];
                bi = e;
            }
        }
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
            const bool take = oi != 0x7fffffff && (bi == 0x7fffffff || ov > bv || (ov == bv && oi < bi));
            if (take) {
                bv = ov;
                bi = oi;
            }
        }
        if (bi != 0x7fffffff && (bi & 63) == lane) {
            for (int i = 0; i < TOPK_MAX_PER_LANE; ++i)
                if (lane + 64 * i == bi) avail[i] = false;
        }
        if (lane == k) {
            mysel = bi;
            myval = bv;
        }
    }
    if (lane < K) sel[t * lds + lane] = mysel;
    if (w) {
        float mx = lane < K ? myval : -INFINITY;
        mx = wave_max(mx);
        const float val = lane < K ? expf(myval - mx) : 0.f;
        double sum = 0.0;
        for (int k = 0; k < K; ++k) sum = sum + (double)__shfl(val, k, 64);
        sum = 1.0 / sum;
        const float s = (float)sum;
        if (lane < K) w[t * K + lane] = val * s;
    }
}

int launch_topk_softmax(const float *logits, int64_t ld_logits, int64_t T, int E, int K, int32_t *sel,
                        int64_t ld_sel, float *w, hipStream_t st) {
    if (T <= 0) return 0;
    if (E > 64 * TOPK_MAX_PER_LANE || K > 64 || K > E || K <= 0) return -6;
    hipLaunchKernelGGL(k_topk_softmax, dim3((unsigned)((T + 3) / 4)), dim3(256), 0, st, logits, ld_logits, T, E,
                       K, sel, ld_sel, w);
    return hip_check_launch();
}

// ---------------------------------------------------------------- dispatch
// Single work-group of 1024 threads.  Stable: within an expert the list is in
// flat (t*K + k) order, i.e. token-ascending then slot-ascending.
constexpr int DISPATCH_THREADS = 1024;
constexpr int DISPATCH_WAVES = DISPATCH_THREADS / 64;

__device__ inline void block_exclusive_scan(int *buf, int n, int tid) {
    // Hillis-Steele inclusive scan over buf[0..n) (n <= blockDim), then shift
    for (int off = 1; off < n; off <<= 1) {
        int add = 0;
        if (tid < n && tid >= off) add = buf[tid - off];
        __syncthreads();
        if (tid < n) buf[tid] += add;
        __syncthreads();
    }
}

__global__ void __launch_bounds__(DISPATCH_THREADS) k_dispatch(const int32_t *__restrict__ ids, int64_t n, int E,
                                                               int BM, Dispatch d) {
    extern __shared__ int dsm[];
    int *cnt = dsm;                                // [E]
    int *run = cnt + E;                            // [E]
    int *scan = run + E;                           // [E]  inclusive scan of counts
    int *tscan = scan + E;                         // [E]  inclusive scan of tiles
    int *ascan = tscan + E;                        // [E]  inclusive scan of active flags
    int *wcnt = ascan + E;                         // [16][E]
    int *wbase = wcnt + DISPATCH_WAVES * E;        // [16][E]
    __shared__ int bad;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;

    for (int e = tid; e < E; e += DISPATCH_THREADS) cnt[e] = 0;
    if (tid == 0) bad = 0;
    __syncthreads();
    for (int64_t i = tid; i < n; i += DISPATCH_THREADS) {
        const int e = ids[i];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
        else atomicAdd(&bad, 1);
    }
    __syncthreads();
    if (tid < E) {
        scan[tid] = cnt[tid];
        tscan[tid] = (cnt[tid] + BM - 1) / BM;
        ascan[tid] = cnt[tid] > 0 ? 1 : 0;
    }
    __syncthreads();
    block_exclusive_scan(scan, E, tid);
    block_exclusive_scan(tscan, E, tid);
    block_exclusive_scan(ascan, E, tid);
    if (tid < E) {
        const int c = cnt[tid];
        const int off = scan[tid] - c;
        d.counts[tid] = c;
        d.offsets[tid] = off;
        run[tid] = off;
        const int nt = (c + BM - 1) / BM;
        const int tb = tscan[tid] - nt;
        for (int j = 0; j < nt; ++j) {
            d.tile_e[tb + j] = tid;
            d.tile_r0[tb + j] = j * BM;
        }
        if (c > 0) d.active_e[ascan[tid] - 1] = tid;
        if (tid == E - 1) {
            d.offsets[E] = scan[tid];
            *d.n_tiles = tscan[tid];
            *d.n_active = ascan[tid];
            *d.bad_ids = bad;
        }
    }
    __syncthreads();

    for (int64_t base = 0; base < n; base += DISPATCH_THREADS) {
        const int64_t i = base + tid;
        const int e = i < n ? ids[i] : -1;
        const bool valid = e >= 0 && e < E;
        for (int j = tid; j < DISPATCH_WAVES * E; j += DISPATCH_THREADS) wcnt[j] = 0;
        __syncthreads();
        uint64_t todo = __ballot(valid);
        int rank = 0;
        while (todo) {
            const int leader = __ffsll((unsigned long long)todo) - 1;
            const int el = __shfl(e, leader, 64);
            const uint64_t m = __ballot(valid && e == el);
            if (valid && e == el) rank = __popcll(m & ((1ull << lane) - 1ull));
            if (lane == leader) wcnt[wave * E + el] = __popcll(m);
            todo &= ~m;
        }
        __syncthreads();
        for (int e2 = tid; e2 < E; e2 += DISPATCH_THREADS) {
            int r = run[e2];
            for (int w2 = 0; w2 < DISPATCH_WAVES; ++w2) {
                wbase[w2 * E + e2] = r;
                r += wcnt[w2 * E + e2];
            }
            run[e2] = r;
        }
        __syncthreads();
        if (valid) d.perm[wbase[wave * E + e] + rank] = (int32_t)i;
        __syncthreads();
    }
}

int launch_dispatch(const int32_t *ids, int64_t T, int K, int E, int BM, const Dispatch &d, hipStream_t st) {
    if (E <= 0 || E > 256) return -6;
    const size_t smem = sizeof(int) * ((size_t)E * 5 + 2 * (size_t)DISPATCH_WAVES * E);
    hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(DISPATCH_THREADS), smem, st, ids, T * K, E, BM, d);
    return hip_check_launch();
}

// ---------------------------------------------------------------- combine
// moe[t][n] = (float)( sum_k (double)(z[t*K+k][n] * w[t][k]) ), slot order;
// out = res + moe.
__global__ void __launch_bounds__(256) k_combine(const float *__restrict__ z, const float *__restrict__ w,
                                                 const float *res, float *out, int64_t T, int K, int D) {
    const int64_t total = T * (int64_t)D;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = idx / D;
        const int n = (int)(idx - t * D);
        double s = 0.0;
        for (int k = 0; k < K; ++k) {
            const float prod = z[(t * K + k) * D + n] * w[t * K + k];
            s = s + (double)prod;
        }
        const float moe = (float)s;
        out[idx] = res ? res[idx] + moe : moe;
    }
}

int launch_combine(const float *z, const float *w, const float *res, float *out, int64_t T, int K, int D,
                   hipStream_t st) {
    if (T <= 0) return 0;
    const int64_t total = T * (int64_t)D;
    const int64_t blocks = (total + 255) / 256 < 8192 ? (total + 255) / 256 : 8192;
    hipLaunchKernelGGL(k_combine, dim3((unsigned)blocks), dim3(256), 0, st, z, w, res, out, T, K, D);
    return hip_check_launch();
}

}  // namespace mimoe
