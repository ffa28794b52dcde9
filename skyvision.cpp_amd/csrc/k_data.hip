// k_data.hip - seeded synthetic data and k-quant weight quantizers.
//
// fill_normal: counter-based splitmix64 + Box-Muller with fixed polynomial
// log / sincos in fp64, so value i of (seed, stream) is a pure function and
// matches the CPU generator bit for bit (same operations, no contraction).
//
// quantize_q4_K / quantize_q6_K: ggml's quantize_row_q4_K_ref and
// quantize_row_q6_K_ref (ported by the reference in convert/q4k.py:27-127 and
// convert/q6k.py:103-193), one lane per sub-block; the per-sub-block search
// runs the reference's loops in the reference's order, so the bytes equal the
// CPU restatement's.
#include "common.hpp"
#include "launch.hpp"
#include "norm.hpp"

namespace mimoe {

// ---------------------------------------------------------------- RNG
__device__ inline uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

__device__ inline double poly_log(double x) {
    const uint64_t bits = __builtin_bit_cast(uint64_t, x);
    int e = (int)((bits >> 52) & 0x7ff) - 1022;
    double m = __builtin_bit_cast(double, (bits & 0x000FFFFFFFFFFFFFULL) | 0x3FE0000000000000ULL);
    if (m < 0.70710678118654752440) {
        m = m * 2.0;
        e = e - 1;
    }
    const double s = (m - 1.0) / (m + 1.0);
    const double z = s * s;
    double p = 1.0 / 25.0;
    p = p * z + 1.0 / 23.0;
    p = p * z + 1.0 / 21.0;
    p = p * z + 1.0 / 19.0;
    p = p * z + 1.0 / 17.0;
    p = p * z + 1.0 / 15.0;
    p = p * z + 1.0 / 13.0;
    p = p * z + 1.0 / 11.0;
    p = p * z + 1.0 / 9.0;
    p = p * z + 1.0 / 7.0;
    p = p * z + 1.0 / 5.0;
    p = p * z + 1.0 / 3.0;
    p = p * z + 1.0;
    const double ln2_hi = 6.93147180369123816490e-01;
    const double ln2_lo = 1.90821492927058770002e-10;
    const double de = (double)e;
    return de * ln2_hi + (2.0 * s * p + de * ln2_lo);
}

__device__ inline void poly_sincos_2pi(double u, double &s_out, double &c_out) {
    const double u4 = u * 4.0;
    const double q = floor(u4);
    const double f = u4 - q;
    const double a = f * 1.57079632679489661923;
    const double z = a * a;
    double sp = -1.0 / 25852016738884976640000.0;
    sp = sp * z + 1.0 / 51090942171709440000.0;
    sp = sp * z - 1.0 / 121645100408832000.0;
    sp = sp * z + 1.0 / 355687428096000.0;
    sp = sp * z - 1.0 / 1307674368000.0;
    sp = sp * z + 1.0 / 6227020800.0;
    sp = sp * z - 1.0 / 39916800.0;
    sp = sp * z + 1.0 / 362880.0;
    sp = sp * z - 1.0 / 5040.0;
    sp = sp * z + 1.0 / 120.0;
    sp = sp * z - 1.0 / 6.0;
    sp = sp * z + 1.0;
    const double sn = a * sp;
    double cp = 1.0 / 1124000727777607680000.0;
    cp = cp * z - 1.0 / 2432902008176640000.0;
    cp = cp * z + 1.0 / 6402373705728000.0;
    cp = cp * z - 1.0 / 20922789888000.0;
    cp = cp * z + 1.0 / 87178291200.0;
    cp = cp * z - 1.0 / 479001600.0;
    cp = cp * z + 1.0 / 3628800.0;
    cp = cp * z - 1.0 / 40320.0;
    cp = cp * z + 1.0 / 720.0;
    cp = cp * z - 1.0 / 24.0;
    cp = cp * z + 1.0 / 2.0;
    const double cs = 1.0 - z * cp;
    const int qi = (int)q;
    if (qi == 0) { s_out = sn; c_out = cs; }
    else if (qi == 1) { s_out = cs; c_out = -sn; }
    else if (qi == 2) { s_out = -sn; c_out = -cs; }
    else { s_out = -cs; c_out = sn; }
}

__global__ void __launch_bounds__(256) k_fill_normal(float *__restrict__ out, int64_t n, uint64_t seed,
                                                     uint64_t stream, double mean, double sd) {
    const uint64_t key = splitmix64(seed ^ splitmix64(stream + 0x1234567ULL));
    // each thread produces one Box-Muller pair (values 2j and 2j+1)
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; 2 * j < n;
         j += (int64_t)gridDim.x * blockDim.x) {
        const uint64_t r1 = splitmix64(key + (uint64_t)(2 * j) * 0xD1B54A32D192ED03ULL);
        const uint64_t r2 = splitmix64(key + (uint64_t)(2 * j + 1) * 0xD1B54A32D192ED03ULL);
        const double u1 = ((double)(r1 >> 11) + 0.5) * (1.0 / 9007199254740992.0);
        const double u2 = (double)(r2 >> 11) * (1.0 / 9007199254740992.0);
        const double r = sqrt(-2.0 * poly_log(u1));
        double s, c;
        poly_sincos_2pi(u2, s, c);
        out[2 * j] = (float)(mean + sd * (r * c));
        if (2 * j + 1 < n) out[2 * j + 1] = (float)(mean + sd * (r * s));
    }
}

// ---------------------------------------------------------------- Q4_K
// make_qkx2_quants(n=32, nmax=15, rmin=-1, rdelta=0.1, nstep=20, use_mad=false)
__device__ inline float make_qkx2_quants32(const float *x, const float *weights, uint8_t *L,
                                           float &the_min) {
    const int n = 32, nmax = 15;
    const float rmin = -1.f, rdelta = 0.1f;
    const int nstep = 20;
    float min = x[0];
    float max = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        float w = weights[i];
        sum_w += w;
        sum_x += w * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        the_min = -min;
        return 0.f;
    }
    float iscale = nmax / (max - min);
    float scale = 1 / iscale;
    float best_error = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * (x[i] - min));
        L[i] = (uint8_t)imax(0, imin(nmax, l));
        float diff = scale * L[i] + min - x[i];
        diff = diff * diff;
        float w = weights[i];
        best_error += w * diff;
    }
    uint8_t Laux[32];
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * (x[i] - min));
            l = imax(0, imin(nmax, l));
            Laux[i] = (uint8_t)l;
            float w = weights[i];
            sum_l += w * l;
            sum_l2 += w * l * l;
            sum_xl += w * l * x[i];
        }
        float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float cur_error = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * Laux[i] + this_min - x[i];
                diff = diff * diff;
                float w = weights[i];
                cur_error += w * diff;
            }
            if (cur_error < best_error) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_error = cur_error;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    the_min = -min;
    return scale;
}

// one thread per 32-value sub-block; 8 consecutive lanes form one super-block
__global__ void __launch_bounds__(256) k_quantize_q4_K(const float *__restrict__ src, uint8_t *__restrict__ dst,
                                                       int64_t nblocks) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t blk = gid >> 3;
    const int j = (int)(gid & 7);
    const bool active = blk < nblocks;
    const int64_t bclamp = active ? blk : 0;
    const float *x = src + bclamp * QK + 32 * j;

    float xv[32], wv[32];
    uint8_t L[32];
    float sum_x2 = 0;
    for (int l = 0; l < 32; ++l) {
        xv[l] = x[l];
        sum_x2 += xv[l] * xv[l];
    }
    const float av_x = sqrtf(sum_x2 / 32);
    for (int l = 0; l < 32; ++l) wv[l] = av_x + fabsf(xv[l]);
    float mn;
    const float sc = make_qkx2_quants32(xv, wv, L, mn);

    // block maxima over the 8 sub-blocks (max is order independent)
    float max_scale = fmaxf(0.f, sc), max_min = fmaxf(0.f, mn);
    for (int o = 1; o < 8; o <<= 1) {
        max_scale = fmaxf(max_scale, __shfl_xor(max_scale, o, 64));
        max_min = fmaxf(max_min, __shfl_xor(max_min, o, 64));
    }
    // reference: `if (scale > max_scale) max_scale = scale` starting at 0
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    int ls = (uint8_t)nearest_int(inv_scale * sc);
    int lm = (uint8_t)nearest_int(inv_min * mn);
    ls = imin(63, ls);
    lm = imin(63, lm);

    const uint32_t dbits = f32_to_fp16_bits(max_scale / 63.f);
    const uint32_t mbits = f32_to_fp16_bits(max_min / 63.f);

    // requantize against the 6-bit quantized scale/min
    const float d = fp16_bits_to_f32(dbits) * ls;
    if (d) {
        const float dm = fp16_bits_to_f32(mbits) * lm;
        for (int ii = 0; ii < 32; ++ii) {
            int l = nearest_int((xv[ii] + dm) / d);
            l = imax(0, imin(15, l));
            L[ii] = (uint8_t)l;
        }
    }

    // pack scales: gather the 8 (ls, lm) pairs of the block
    const int lane = threadIdx.x & 63;
    const int base = lane & ~7;
    int lsv[8], lmv[8];
    for (int q = 0; q < 8; ++q) {
        lsv[q] = __shfl(ls, base + q, 64);
        lmv[q] = __shfl(lm, base + q, 64);
    }
    // qs: byte 32c+l = L[64c+l] | L[64c+32+l] << 4 -> sub-blocks 2c (low) and 2c+1 (high)
    const int partner = lane ^ 1;
    uint8_t *out = dst + bclamp * Q4K_BYTES;
    for (int l = 0; l < 32; l += 4) {
        uint32_t mine = (uint32_t)L[l] | ((uint32_t)L[l + 1] << 8) | ((uint32_t)L[l + 2] << 16) |
                        ((uint32_t)L[l + 3] << 24);
        uint32_t other = __shfl(mine, partner, 64);
        if (!(j & 1)) {
            const uint32_t v = (mine & 0x0F0F0F0Fu) | ((other & 0x0F0F0F0Fu) << 4);
            if (active) *(uint32_t *)(out + 16 + 32 * (j >> 1) + l) = v;
        }
    }
    if (active && j == 0) {
        uint8_t s12[12];
        for (int q = 0; q < 4; ++q) {
            s12[q] = (uint8_t)lsv[q];
            s12[q + 4] = (uint8_t)lmv[q];
        }
        for (int q = 4; q < 8; ++q) {
            s12[q + 4] = (uint8_t)((lsv[q] & 0xF) | ((lmv[q] & 0xF) << 4));
            s12[q - 4] |= (uint8_t)((lsv[q] >> 4) << 6);
            s12[q - 0] |= (uint8_t)((lmv[q] >> 4) << 6);
        }
        *(uint32_t *)(out + 0) = dbits | (mbits << 16);
        for (int q = 0; q < 12; q += 4)
            *(uint32_t *)(out + 4 + q) = (uint32_t)s12[q] | ((uint32_t)s12[q + 1] << 8) |
                                         ((uint32_t)s12[q + 2] << 16) | ((uint32_t)s12[q + 3] << 24);
    }
}

// ---------------------------------------------------------------- Q6_K
// make_qx_quants(n=16, nmax=32, rmse_type=1, qw=NULL)
__device__ inline float make_qx_quants16(const float *x, int8_t *L) {
    const int n = 16, nmax = 32;
    float max = 0;
    float amax = 0;
    for (int i = 0; i < n; ++i) {
        float ax = fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            max = x[i];
        }
    }
    if (amax < 1e-15f) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.f;
    }
    float iscale = -nmax / max;
    float sumlx = 0;
    float suml2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = imax(-nmax, imin(nmax - 1, l));
        L[i] = (int8_t)(l + nmax);
        float w = x[i] * x[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    float scale = suml2 ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -(nmax + 0.1f * is) / max;
        sumlx = suml2 = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * x[i]);
            l = imax(-nmax, imin(nmax - 1, l));
            float w = x[i] * x[i];
            sumlx += w * x[i] * l;
            suml2 += w * l * l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) {
                int l = nearest_int(iscale * x[i]);
                L[i] = (int8_t)(nmax + imax(-nmax, imin(nmax - 1, l)));
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

// one thread per 16-value sub-block; 16 consecutive lanes form one super-block
__global__ void __launch_bounds__(256) k_quantize_q6_K(const float *__restrict__ src, uint8_t *__restrict__ dst,
                                                       int64_t nblocks) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t blk = gid >> 4;
    const int ib = (int)(gid & 15);
    const bool active = blk < nblocks;
    const int64_t bclamp = active ? blk : 0;
    const float *x = src + bclamp * QK + 16 * ib;
    const int lane = threadIdx.x & 63;
    const int base = lane & ~15;

    float xv[16];
    int8_t L[16];
    for (int i = 0; i < 16; ++i) xv[i] = x[i];
    const float scale = make_qx_quants16(xv, L);

    // first sub-block with the largest |scale| (reference: strict '>')
    AmaxIdx a{fabsf(scale), ib, scale};
    a = wave_amax_idx(a, 16);
    const float max_abs_scale = a.ax;
    const float max_scale = a.val;
    uint8_t *out = dst + bclamp * Q6K_BYTES;

    if (max_abs_scale < 1e-15f) {
        // all-zero block (memset + d = fp16(0))
        if (active) {
            for (int q = ib; q < Q6K_BYTES; q += 16) out[q] = 0;
        }
        return;
    }
    const float iscale = -128.f / max_scale;
    const uint32_t dbits = f32_to_fp16_bits(1 / iscale);
    const int sc = imin(127, nearest_int(iscale * scale));
    const float d = fp16_bits_to_f32(dbits) * (int8_t)sc;
    if (d) {
        for (int ii = 0; ii < 16; ++ii) {
            int l = nearest_int(xv[ii] / d);
            l = imax(-32, imin(31, l));
            L[ii] = (int8_t)(l + 32);
        }
    }
    // pack.  Element e = 128*h + 32*qq + l (qq quarter 0..3, l 0..31) lives in
    // sub-block ib = e/16 = 8h + 2qq + l/16.  ql[64h + l] holds q1|q3<<4 and
    // ql[64h + 32 + l] holds q2|q4<<4; qh[32h + l] holds the 2-bit highs of
    // the four quarters.  Lane (h, qq, l16) owns l in 16*l16 .. +16.
    const int h = ib >> 3;
    const int qq = (ib >> 1) & 3;
    const int l16 = ib & 1;
    // gather the 16 values of the partner lanes holding the other quarters
    // for the same (h, l16): lanes base + 8h + 2*q' + l16
    uint32_t lw[4];
    for (int w = 0; w < 4; ++w)
        lw[w] = (uint32_t)(uint8_t)L[4 * w] | ((uint32_t)(uint8_t)L[4 * w + 1] << 8) |
                ((uint32_t)(uint8_t)L[4 * w + 2] << 16) | ((uint32_t)(uint8_t)L[4 * w + 3] << 24);
    uint32_t quart[4][4];
    for (int q2 = 0; q2 < 4; ++q2)
        for (int w = 0; w < 4; ++w) quart[q2][w] = __shfl(lw[w], base + 8 * h + 2 * q2 + l16, 64);
    if (active && qq == 0) {
        // this lane writes ql/qh bytes for l in 16*l16 .. +16 of half h
        for (int w = 0; w < 4; ++w) {
            const uint32_t q1 = quart[0][w], q2v = quart[1][w], q3 = quart[2][w], q4 = quart[3][w];
            const uint32_t qla = (q1 & 0x0F0F0F0Fu) | ((q3 & 0x0F0F0F0Fu) << 4);
            const uint32_t qlb = (q2v & 0x0F0F0F0Fu) | ((q4 & 0x0F0F0F0Fu) << 4);
            const uint32_t qhv = ((q1 >> 4) & 0x03030303u) | (((q2v >> 4) & 0x03030303u) << 2) |
                                 (((q3 >> 4) & 0x03030303u) << 4) | (((q4 >> 4) & 0x03030303u) << 6);
            const int l = 16 * l16 + 4 * w;
            // Q6_K blocks are 210 bytes: only 2-byte alignment is guaranteed
            uint8_t *pa = out + 64 * h + l;
            uint8_t *pb = out + 64 * h + 32 + l;
            uint8_t *ph = out + 128 + 32 * h + l;
            for (int b = 0; b < 4; ++b) {
                pa[b] = (uint8_t)(qla >> (8 * b));
                pb[b] = (uint8_t)(qlb >> (8 * b));
                ph[b] = (uint8_t)(qhv >> (8 * b));
            }
        }
    }
    if (active) out[192 + ib] = (uint8_t)(int8_t)sc;
    if (active && ib == 0) {
        out[208] = (uint8_t)(dbits & 0xff);
        out[209] = (uint8_t)(dbits >> 8);
    }
}

// ---------------------------------------------------------------- launchers
// y[t] = norm(x[t]) (norm.hpp): one 256-thread work-group per row of D <=
// 4096; thread i holds the float4 pieces at 1024 k + 4 i (coalesced), sums in
// fp64 over its pieces in k order, then a fixed LDS tree (128, 64, .. 1) over
// the threads; LayerNorm's second sum reuses the held values.  y may equal x
// (every value is in registers before the first store).

__device__ inline double norm_block_sum(double v, double *red) {
    red[threadIdx.x] = v;
    __syncthreads();
    for (int o = NORM_T / 2; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + o];
        __syncthreads();
    }
    const double r = red[0];
    __syncthreads();   // red is reused
    return r;
}

__global__ void __launch_bounds__(NORM_T) k_norm_rows(const float *x, int D, NormParams p, float *y) {
    __shared__ double red[NORM_T];
    const int64_t t = blockIdx.x;
    const float *xr = x + t * D;
    float *yr = y + t * D;
    const bool vec = D % 4 == 0 && ((uintptr_t)xr & 15) == 0 && ((uintptr_t)yr & 15) == 0;
    float v[NORM_PIECES][4];
#pragma unroll
    for (int k = 0; k < NORM_PIECES; ++k) {
        const int i = 1024 * k + 4 * (int)threadIdx.x;
        if (vec && i < D) {
            const float4 a = *(const float4 *)(xr + i);
            v[k][0] = a.x; v[k][1] = a.y; v[k][2] = a.z; v[k][3] = a.w;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) v[k][j] = i + j < D ? xr[i + j] : 0.f;
        }
    }
    float m = 0.f, sc;
    double acc = 0.0;
    if (p.kind == NORM_RMS) {
#pragma unroll
        for (int k = 0; k < NORM_PIECES; ++k)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = acc + (double)(v[k][j] * v[k][j]);   // zeros past D add 0
        const float ms = (float)(norm_block_sum(acc, red) / (double)D);
        sc = 1.0f / sqrtf(ms + p.eps);
    } else {
#pragma unroll
        for (int k = 0; k < NORM_PIECES; ++k)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = acc + (double)v[k][j];
        m = (float)(norm_block_sum(acc, red) / (double)D);
        double acc2 = 0.0;
#pragma unroll
        for (int k = 0; k < NORM_PIECES; ++k)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (1024 * k + 4 * (int)threadIdx.x + j < D) {
                    const float d = v[k][j] - m;
                    acc2 = acc2 + (double)(d * d);
                }
        const float var = (float)(norm_block_sum(acc2, red) / (double)D);
        sc = 1.0f / sqrtf(var + p.eps);
    }
#pragma unroll
    for (int k = 0; k < NORM_PIECES; ++k) {
        const int i = 1024 * k + 4 * (int)threadIdx.x;
        if (i >= D) continue;
        float o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = norm_apply(p, v[k][j], i + j, m, sc);
        if (vec) {
            *(float4 *)(yr + i) = make_float4(o[0], o[1], o[2], o[3]);
        } else {
            for (int j = 0; j < 4; ++j)
                if (i + j < D) yr[i + j] = o[j];
        }
    }
}

int launch_norm(const NormParams &p, const float *x, int64_t T, int D, float *y, hipStream_t st) {
    if (T <= 0) return 0;
    if (T > 0x7fffffff || D <= 0 || D > 4096 || (p.kind != NORM_RMS && p.kind != NORM_LAYER)) return -6;
    hipLaunchKernelGGL(k_norm_rows, dim3((unsigned)T), dim3(NORM_T), 0, st, x, D, p, y);
    return hip_check_launch();
}

int launch_rmsnorm(const float *x, int64_t T, int D, float eps, float *y, hipStream_t st) {
    NormParams p;
    p.kind = NORM_RMS;
    p.eps = eps;
    return launch_norm(p, x, T, D, y, st);
}

int launch_fill_normal(float *out, int64_t n, uint64_t seed, uint64_t stream, float mean, float sd,
                       hipStream_t st) {
    if (n <= 0) return 0;
    const int64_t pairs = (n + 1) / 2;
    const int64_t blocks = min((int64_t)65536, (pairs + 255) / 256);
    hipLaunchKernelGGL(k_fill_normal, dim3((unsigned)blocks), dim3(256), 0, st, out, n, seed, stream,
                       (double)mean, (double)sd);
    return hip_check_launch();
}

int launch_quantize(int type, const float *src, void *dst, int64_t nblocks, hipStream_t st) {
    if (nblocks <= 0) return 0;
    if (type == 12) {
        const int64_t threads = nblocks * 8;
        hipLaunchKernelGGL(k_quantize_q4_K, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, src,
                           (uint8_t *)dst, nblocks);
    } else {
        const int64_t threads = nblocks * 16;
        hipLaunchKernelGGL(k_quantize_q6_K, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, src,
                           (uint8_t *)dst, nblocks);
    }
    return hip_check_launch();
}

// Q4_K tables in the grouped GEMMs' tiled order: for every matrix (mat
// bytes) and every 32-row group of its rows (rb bytes each), block b of the
// group's rows as 32 x 144 contiguous bytes, then block b + 1.  One thread
// per 16-byte piece of dst: coalesced stores, 16-byte gathers from the rows.
__global__ void __launch_bounds__(256) k_tile_q4k(const uint4 *__restrict__ src, uint4 *__restrict__ dst,
                                                   int64_t pieces, int64_t mat, int64_t rb) {
    const int64_t group = 32 * rb;
    for (int64_t p = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; p < pieces;
         p += (int64_t)gridDim.x * blockDim.x) {
        const int64_t o = 16 * p, e = o / mat, in_mat = o - e * mat, t = in_mat / group;
        const int64_t in_group = in_mat - t * group, b = in_group / (32 * Q4K_BYTES);
        const int64_t in_block = in_group - b * (32 * Q4K_BYTES), r = in_block / Q4K_BYTES;
        const int64_t j = in_block - r * Q4K_BYTES;
        dst[p] = src[(e * mat + (32 * t + r) * rb + Q4K_BYTES * b + j) / 16];
    }
}

// Q6_K tables in the down GEMM's tiled order: per matrix, 32-row group and
// block b, 9216 bytes = 8 code chunks of 1 KB and one scale chunk of 1 KB,
// 16 bytes per lane L (row 32 t + L % 32 of the group, half g2 = L / 32).
// Code chunk 4 h + m holds the lane's merged 6-bit codes (one per byte) of
// stage h, dword m of its 16-byte ql / qh runs:
//   a = ql[64 h + 16 g2 + 4 m ..], b = ql[64 h + 32 + 16 g2 + 4 m ..],
//   c = qh[32 h + 16 g2 + 4 m ..]  (dwords)
//   {a lo | (c << 4 & 0x30..), a hi | (c & 0x30..), b lo | (c << 2 & 0x30..),
//    b hi | (c >> 2 & 0x30..)}  (lo = & 0x0F.., hi = >> 4 & 0x0F..)
// - the codes the GEMM's Q6_K operand builder forms from the rows; the scale
// chunk holds fp16(d * scales[8 h + 2 j + g2] + 0) at half 4 h + j.  One thread
// per 16-byte piece; bytes read one at a time (blocks are 2-byte aligned).
__device__ inline uint32_t rd_u32_bytes(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

__global__ void __launch_bounds__(256) k_tile_q6k(const uint8_t *__restrict__ src, uint4 *__restrict__ dst,
                                                   int64_t pieces, int64_t src_mat, int64_t rb, int64_t ntile,
                                                   int nb) {
    for (int64_t p = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; p < pieces;
         p += (int64_t)gridDim.x * blockDim.x) {
        const int64_t tb = p / 576;   // (matrix, group, block), 9 chunks x 64 lanes each
        const int q = (int)(p - tb * 576), c = q >> 6, L = q & 63, g2 = L >> 5;
        const int b = (int)(tb % nb);
        const int64_t mt = tb / nb, t = mt % ntile, e = mt / ntile;
        const uint8_t *blk = src + e * src_mat + (32 * t + (L & 31)) * rb + (int64_t)Q6K_BYTES * b;
        uint4 o;
        if (c < 8) {
            const int h = c >> 2, m = c & 3;
            const uint32_t a = rd_u32_bytes(blk + 64 * h + 16 * g2 + 4 * m);
            const uint32_t bb = rd_u32_bytes(blk + 64 * h + 32 + 16 * g2 + 4 * m);
            const uint32_t qh = rd_u32_bytes(blk + 128 + 32 * h + 16 * g2 + 4 * m);
            o.x = (a & 0x0F0F0F0Fu) | ((qh << 4) & 0x30303030u);
            o.y = ((a >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u);
            o.z = (bb & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u);
            o.w = ((bb >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u);
        } else {
            const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(blk[208] | (blk[209] << 8)));
            uint32_t hv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int h = i >> 2, j = i & 3;
                // (+ 0: a zero scale gives +0 whatever d's sign, as the GEMM's
                // own conversion of d * scale does)
                const _Float16 v = (_Float16)(d * (float)(int)(int8_t)blk[192 + 8 * h + 2 * j + g2] + 0.0f);
                hv[i] = (uint32_t)__builtin_bit_cast(uint16_t, v);
            }
            o.x = hv[0] | (hv[1] << 16);
            o.y = hv[2] | (hv[3] << 16);
            o.z = hv[4] | (hv[5] << 16);
            o.w = hv[6] | (hv[7] << 16);
        }
        dst[p] = o;
    }
}

int launch_tile_q6k(const void *src, void *dst, int64_t n_mat, int64_t rows, int64_t rb, hipStream_t st) {
    const int nb = (int)(rb / Q6K_BYTES);
    const int64_t ntile = rows / 32, pieces = n_mat * ntile * nb * 576;
    if (pieces <= 0) return 0;
    const int64_t blocks = min((int64_t)65536, (pieces + 255) / 256);
    hipLaunchKernelGGL(k_tile_q6k, dim3((unsigned)blocks), dim3(256), 0, st, (const uint8_t *)src, (uint4 *)dst,
                       pieces, rows * rb, rb, ntile, nb);
    return hip_check_launch();
}

int launch_tile_q4k(const void *src, void *dst, int64_t n_mat, int64_t rows, int64_t rb, hipStream_t st) {
    const int64_t pieces = n_mat * rows * rb / 16;
    if (pieces <= 0) return 0;
    const int64_t blocks = min((int64_t)65536, (pieces + 255) / 256);
    hipLaunchKernelGGL(k_tile_q4k, dim3((unsigned)blocks), dim3(256), 0, st, (const uint4 *)src, (uint4 *)dst, pieces,
                       rows * rb, rb);
    return hip_check_launch();
}

}  // namespace mimoe
