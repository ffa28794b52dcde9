/*
 * moe_oracle.c - CPU oracle for the routed MoE FFN layer (test infrastructure
 * only; see moe_oracle.h for scope and the reference call sites it restates).
 *
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off -fopenmp).  Contraction
 * is off so every fp32/fp64 expression rounds exactly as written; the GPU
 * kernels that must agree bit for bit (RNG, quantizers, router, Q8_K) are
 * written with the same operation order and contraction disabled.
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK_K ORC_QK_K
#define GROUP_MAX_EPS 1e-15f

int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

static int nthr(int n) { return n > 0 ? n : orc_max_threads(); }

/* ------------------------------------------------------------------------ */
/* fp16 (IEEE binary16, round to nearest even) - what GGML_FP32_TO_FP16 does */
/* ------------------------------------------------------------------------ */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint64_t d2u(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
static inline double u2d(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }

float orc_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        /* subnormal: value = man * 2^-24 */
        float v = (float)man * u2f(0x33800000u); /* 2^-24, exact */
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7f800000u | (man << 13));
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t orc_fp32_to_fp16(float f) {
    const uint32_t x = f2u(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                       /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  /* rounds to inf */
    if (ax < 0x38800000u) {                        /* below fp16 normal range */
        if (ax < 0x33000000u) return (uint16_t)sign;            /* < 2^-25 -> 0 */
        /* subnormal: round(ax_value / 2^-24) to nearest even */
        const uint32_t e = ax >> 23;               /* biased fp32 exponent */
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - e;           /* 14..24 */
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    /* normal */
    uint32_t e = (ax >> 23) - 112u;
    uint32_t m = ax & 0x7fffffu;
    uint32_t q = (e << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

/* ggml nearest_int: round half to even via the 1.5*2^23 magic constant */
int orc_nearest_int(float fval) {
    float val = fval + 12582912.f;
    int i;
    memcpy(&i, &val, sizeof(int));
    return (i & 0x007fffff) - 0x00400000;
}

#define MAX(a, b) ((a) > (b) ? (a) : (b))
#define MIN(a, b) ((a) < (b) ? (a) : (b))

/* ------------------------------------------------------------------------ */
/* Q4_K quantizer: ggml make_qkx2_quants + quantize_row_q4_K_ref            */
/* (ported in convert/q4k.py:27-127; same algorithm)                        */
/* ------------------------------------------------------------------------ */
static float make_qkx2_quants(int n, int nmax, const float *x, const float *weights,
                              uint8_t *L, float *the_min, uint8_t *Laux,
                              float rmin, float rdelta, int nstep, int fixed_span) {
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
        *the_min = -min;
        return 0.f;
    }
    float iscale = nmax / (max - min);
    float scale = 1 / iscale;
    float best_error = 0;
    for (int i = 0; i < n; ++i) {
        int l = orc_nearest_int(iscale * (x[i] - min));
        L[i] = (uint8_t)MAX(0, MIN(nmax, l));
        float diff = scale * L[i] + min - x[i];
        diff = diff * diff;
        float w = weights[i];
        best_error += w * diff;
    }
    if (nstep < 1) {
        *the_min = -min;
        return scale;
    }
    /* ggml: the search span max - min follows the best min found so far;
     * fixed_span = 1 keeps the initial span (convert/q4k.py:43, port only) */
    const float span0 = max - min;
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (fixed_span ? span0 : max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = orc_nearest_int(iscale * (x[i] - min));
            l = MAX(0, MIN(nmax, l));
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
    *the_min = -min;
    return scale;
}

/* 6-bit scale/min unpack: convert/q4k.py:107-110 */
static inline void get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4);
    }
}

void orc_quantize_row_q4_K(const float *x, void *vy, int64_t k) { orc_quantize_row_q4_K_port(x, vy, k, 0); }

void orc_quantize_row_q4_K_port(const float *x, void *vy, int64_t k, int port) {
    orc_block_q4_K *y = (orc_block_q4_K *)vy;
    const int64_t nb = k / QK_K;
    uint8_t L[QK_K];
    uint8_t Laux[32];
    float weights[32];
    float mins[QK_K / 32];
    float scales[QK_K / 32];

    for (int64_t i = 0; i < nb; i++) {
        float max_scale = 0;
        float max_min = 0;
        for (int j = 0; j < QK_K / 32; ++j) {
            float sum_x2 = 0;
            for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
            float av_x = sqrtf(sum_x2 / 32);
            for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(x[32 * j + l]);
            scales[j] = make_qkx2_quants(32, 15, x + 32 * j, weights, L + 32 * j, &mins[j],
                                         Laux, -1.f, 0.1f, 20, port & ORC_PORT_FIXED_SPAN);
            float scale = scales[j];
            if (scale > max_scale) max_scale = scale;
            float min = mins[j];
            if (min > max_min) max_min = min;
        }

        float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
        float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
        for (int j = 0; j < QK_K / 32; ++j) {
            uint8_t ls = (uint8_t)orc_nearest_int(inv_scale * scales[j]);
            uint8_t lm = (uint8_t)orc_nearest_int(inv_min * mins[j]);
            ls = MIN(63, ls);
            lm = MIN(63, lm);
            if (j < 4) {
                y[i].scales[j] = ls;
                y[i].scales[j + 4] = lm;
            } else {
                y[i].scales[j + 4] = (ls & 0xF) | ((lm & 0xF) << 4);
                y[i].scales[j - 4] |= ((ls >> 4) << 6);
                y[i].scales[j - 0] |= ((lm >> 4) << 6);
            }
        }
        y[i].d = orc_fp32_to_fp16(max_scale / 63.f);
        y[i].dmin = orc_fp32_to_fp16(max_min / 63.f);

        uint8_t sc, m;
        for (int j = 0; j < QK_K / 32; ++j) {
            get_scale_min_k4(j, y[i].scales, &sc, &m);
            const float d = orc_fp16_to_fp32(y[i].d) * sc;
            if (!d) {   /* ggml keeps the search's codes; the port writes 0 */
                if (port & ORC_PORT_ZERO_L) memset(L + 32 * j, 0, 32);
                continue;
            }
            const float dm = orc_fp16_to_fp32(y[i].dmin) * m;
            for (int ii = 0; ii < 32; ++ii) {
                int l = orc_nearest_int((x[32 * j + ii] + dm) / d);
                l = MAX(0, MIN(15, l));
                L[32 * j + ii] = (uint8_t)l;
            }
        }

        uint8_t *q = y[i].qs;
        for (int j = 0; j < QK_K; j += 64) {
            for (int l = 0; l < 32; ++l) q[l] = L[j + l] | (L[j + l + 32] << 4);
            q += 32;
        }
        x += QK_K;
    }
}

void orc_dequantize_row_q4_K(const void *vx, float *y, int64_t k) {
    const orc_block_q4_K *x = (const orc_block_q4_K *)vx;
    const int64_t nb = k / QK_K;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t *q = x[i].qs;
        const float d = orc_fp16_to_fp32(x[i].d);
        const float min = orc_fp16_to_fp32(x[i].dmin);
        int is = 0;
        uint8_t sc, m;
        for (int j = 0; j < QK_K; j += 64) {
            get_scale_min_k4(is + 0, x[i].scales, &sc, &m);
            const float d1 = d * sc;
            const float m1 = min * m;
            get_scale_min_k4(is + 1, x[i].scales, &sc, &m);
            const float d2 = d * sc;
            const float m2 = min * m;
            for (int l = 0; l < 32; ++l) *y++ = d1 * (q[l] & 0xF) - m1;
            for (int l = 0; l < 32; ++l) *y++ = d2 * (q[l] >> 4) - m2;
            q += 32;
            is += 2;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Q6_K quantizer: ggml make_qx_quants(rmse_type=1) + quantize_row_q6_K_ref */
/* (ported in convert/q6k.py:103-193)                                        */
/* ------------------------------------------------------------------------ */
static float make_qx_quants_rmse1(int n, int nmax, const float *x, int8_t *L) {
    float max = 0;
    float amax = 0;
    for (int i = 0; i < n; ++i) {
        float ax = fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            max = x[i];
        }
    }
    if (amax < GROUP_MAX_EPS) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.f;
    }
    float iscale = -nmax / max;
    float sumlx = 0;
    float suml2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = orc_nearest_int(iscale * x[i]);
        l = MAX(-nmax, MIN(nmax - 1, l));
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
            int l = orc_nearest_int(iscale * x[i]);
            l = MAX(-nmax, MIN(nmax - 1, l));
            float w = x[i] * x[i];
            sumlx += w * x[i] * l;
            suml2 += w * l * l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) {
                int l = orc_nearest_int(iscale * x[i]);
                L[i] = (int8_t)(nmax + MAX(-nmax, MIN(nmax - 1, l)));
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

void orc_quantize_row_q6_K(const float *x, void *vy, int64_t k, int port) {
    const int requant_fp32_d = port & ORC_PORT_FP32_D;
    orc_block_q6_K *y = (orc_block_q6_K *)vy;
    const int64_t nb = k / QK_K;
    int8_t L[QK_K];
    float scales[QK_K / 16];

    for (int64_t i = 0; i < nb; i++) {
        float max_scale = 0;
        float max_abs_scale = 0;
        for (int ib = 0; ib < QK_K / 16; ++ib) {
            const float scale = make_qx_quants_rmse1(16, 32, x + 16 * ib, L + 16 * ib);
            scales[ib] = scale;
            const float abs_scale = fabsf(scale);
            if (abs_scale > max_abs_scale) {
                max_abs_scale = abs_scale;
                max_scale = scale;
            }
        }
        if (max_abs_scale < GROUP_MAX_EPS) {
            memset(&y[i], 0, sizeof(orc_block_q6_K));
            y[i].d = orc_fp32_to_fp16(0.f);
            x += QK_K;
            continue;
        }
        float iscale = -128.f / max_scale;
        const float d32 = 1 / iscale;
        y[i].d = orc_fp32_to_fp16(d32);
        for (int ib = 0; ib < QK_K / 16; ++ib) {
            y[i].scales[ib] = (int8_t)MIN(127, orc_nearest_int(iscale * scales[ib]));
        }
        for (int j = 0; j < QK_K / 16; ++j) {
            float d = (requant_fp32_d ? d32 : orc_fp16_to_fp32(y[i].d)) * y[i].scales[j];
            if (!d) {   /* ggml keeps the search's codes; the port writes 0 (value -32) */
                if (port & ORC_PORT_ZERO_L) memset(L + 16 * j, 0, 16);
                continue;
            }
            for (int ii = 0; ii < 16; ++ii) {
                int l = orc_nearest_int(x[16 * j + ii] / d);
                l = MAX(-32, MIN(31, l));
                L[16 * j + ii] = (int8_t)(l + 32);
            }
        }
        uint8_t *ql = y[i].ql;
        uint8_t *qh = y[i].qh;
        for (int j = 0; j < QK_K; j += 128) {
            for (int l = 0; l < 32; ++l) {
                const uint8_t q1 = L[j + l + 0] & 0xF;
                const uint8_t q2 = L[j + l + 32] & 0xF;
                const uint8_t q3 = L[j + l + 64] & 0xF;
                const uint8_t q4 = L[j + l + 96] & 0xF;
                ql[l + 0] = q1 | (q3 << 4);
                ql[l + 32] = q2 | (q4 << 4);
                qh[l] = (uint8_t)((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) |
                                  ((L[j + l + 64] >> 4) << 4) | ((L[j + l + 96] >> 4) << 6));
            }
            ql += 64;
            qh += 32;
        }
        x += QK_K;
    }
}

/* closed form: scripts/test_q6k.py:41-62 */
void orc_dequantize_row_q6_K(const void *vx, float *y, int64_t k) {
    const orc_block_q6_K *x = (const orc_block_q6_K *)vx;
    const int64_t nb = k / QK_K;
    for (int64_t i = 0; i < nb; i++) {
        const float d = orc_fp16_to_fp32(x[i].d);
        const uint8_t *ql = x[i].ql;
        const uint8_t *qh = x[i].qh;
        const int8_t *sc = x[i].scales;
        for (int n = 0; n < QK_K; n += 128) {
            for (int l = 0; l < 32; ++l) {
                int is = l / 16;
                const int8_t q1 = (int8_t)((ql[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int8_t q2 = (int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int8_t q3 = (int8_t)((ql[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int8_t q4 = (int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[l + 0] = d * sc[is + 0] * q1;
                y[l + 32] = d * sc[is + 2] * q2;
                y[l + 64] = d * sc[is + 4] * q3;
                y[l + 96] = d * sc[is + 6] * q4;
            }
            y += 128;
            ql += 64;
            qh += 32;
            sc += 8;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Q8_K: ggml quantize_row_q8_K_ref (activations for the k-quant dots)      */
/* ------------------------------------------------------------------------ */
void orc_quantize_row_q8_K(const float *x, void *vy, int64_t k) {
    orc_block_q8_K *y = (orc_block_q8_K *)vy;
    const int64_t nb = k / QK_K;
    for (int64_t i = 0; i < nb; i++) {
        float max = 0;
        float amax = 0;
        for (int j = 0; j < QK_K; ++j) {
            float ax = fabsf(x[j]);
            if (ax > amax) {
                amax = ax;
                max = x[j];
            }
        }
        if (!amax) {
            y[i].d = 0;
            memset(y[i].qs, 0, QK_K);
            memset(y[i].bsums, 0, sizeof(y[i].bsums));
            x += QK_K;
            continue;
        }
        const float iscale = -127.f / max;
        for (int j = 0; j < QK_K; ++j) {
            int v = orc_nearest_int(iscale * x[j]);
            y[i].qs[j] = (int8_t)MIN(127, v);
        }
        for (int j = 0; j < QK_K / 16; ++j) {
            int sum = 0;
            for (int ii = 0; ii < 16; ++ii) sum += y[i].qs[j * 16 + ii];
            y[i].bsums[j] = (int16_t)sum;
        }
        y[i].d = 1 / iscale;
        x += QK_K;
    }
}

void orc_dequantize_row_q8_K(const void *vx, float *y, int64_t k) {
    const orc_block_q8_K *x = (const orc_block_q8_K *)vx;
    const int64_t nb = k / QK_K;
    for (int64_t i = 0; i < nb; i++)
        for (int j = 0; j < QK_K; ++j) *y++ = x[i].d * x[i].qs[j];
}

/* ------------------------------------------------------------------------ */
/* 32-value block formats (ggml ggml-quants.c, the _ref quantizers and the  */
/* dequantizers; [ggml-ext]: ggml is not in the reference tree).  Q8_0 is    */
/* also the activation format the Q4_0 / Q5_0 / Q8_0 dots take (ggml-cpu    */
/* vec_dot_type).  ggml's x86 SIMD quantize_row_q8_0 rounds half to even     */
/* with id = 127 / amax; the portable _ref form restated here uses          */
/* id = 1 / fp32(amax / 127) and roundf (half away from zero): the two can   */
/* differ by one code on values at a rounding boundary.                      */
/* ------------------------------------------------------------------------ */
void orc_quantize_row_q4_0(const float *x, void *vy, int64_t k) {
    orc_block_q4_0 *y = (orc_block_q4_0 *)vy;
    const int64_t nb = k / ORC_QK32;
    for (int64_t i = 0; i < nb; i++) {
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < ORC_QK32; j++) {
            const float v = x[i * ORC_QK32 + j];
            if (amax < fabsf(v)) {
                amax = fabsf(v);
                max = v;
            }
        }
        const float d = max / -8;
        const float id = d ? 1.0f / d : 0.0f;
        y[i].d = orc_fp32_to_fp16(d);
        for (int j = 0; j < ORC_QK32 / 2; ++j) {
            const float x0 = x[i * ORC_QK32 + j] * id;
            const float x1 = x[i * ORC_QK32 + ORC_QK32 / 2 + j] * id;
            const uint8_t xi0 = (uint8_t)MIN(15, (int8_t)(x0 + 8.5f));
            const uint8_t xi1 = (uint8_t)MIN(15, (int8_t)(x1 + 8.5f));
            y[i].qs[j] = (uint8_t)(xi0 | (xi1 << 4));
        }
    }
}

void orc_quantize_row_q5_0(const float *x, void *vy, int64_t k) {
    orc_block_q5_0 *y = (orc_block_q5_0 *)vy;
    const int64_t nb = k / ORC_QK32;
    for (int64_t i = 0; i < nb; i++) {
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < ORC_QK32; j++) {
            const float v = x[i * ORC_QK32 + j];
            if (amax < fabsf(v)) {
                amax = fabsf(v);
                max = v;
            }
        }
        const float d = max / -16;
        const float id = d ? 1.0f / d : 0.0f;
        y[i].d = orc_fp32_to_fp16(d);
        uint32_t qh = 0;
        for (int j = 0; j < ORC_QK32 / 2; ++j) {
            const float x0 = x[i * ORC_QK32 + j] * id;
            const float x1 = x[i * ORC_QK32 + ORC_QK32 / 2 + j] * id;
            const uint8_t xi0 = (uint8_t)MIN(31, (int8_t)(x0 + 16.5f));
            const uint8_t xi1 = (uint8_t)MIN(31, (int8_t)(x1 + 16.5f));
            y[i].qs[j] = (uint8_t)((xi0 & 0x0F) | ((xi1 & 0x0F) << 4));
            qh |= ((uint32_t)(xi0 & 0x10u) >> 4) << j;
            qh |= ((uint32_t)(xi1 & 0x10u) >> 4) << (j + ORC_QK32 / 2);
        }
        memcpy(y[i].qh, &qh, sizeof(qh));
    }
}

void orc_quantize_row_q8_0(const float *x, void *vy, int64_t k) {
    orc_block_q8_0 *y = (orc_block_q8_0 *)vy;
    const int64_t nb = k / ORC_QK32;
    for (int64_t i = 0; i < nb; i++) {
        float amax = 0.0f;
        for (int j = 0; j < ORC_QK32; j++) amax = MAX(amax, fabsf(x[i * ORC_QK32 + j]));
        const float d = amax / ((1 << 7) - 1);
        const float id = d ? 1.0f / d : 0.0f;
        y[i].d = orc_fp32_to_fp16(d);
        for (int j = 0; j < ORC_QK32; ++j) y[i].qs[j] = (int8_t)roundf(x[i * ORC_QK32 + j] * id);
    }
}

void orc_dequantize_row_q4_0(const void *vx, float *y, int64_t k) {
    const orc_block_q4_0 *x = (const orc_block_q4_0 *)vx;
    for (int64_t i = 0; i < k / ORC_QK32; i++) {
        const float d = orc_fp16_to_fp32(x[i].d);
        for (int j = 0; j < ORC_QK32 / 2; ++j) {
            y[i * ORC_QK32 + j] = ((x[i].qs[j] & 0x0F) - 8) * d;
            y[i * ORC_QK32 + j + ORC_QK32 / 2] = ((x[i].qs[j] >> 4) - 8) * d;
        }
    }
}

void orc_dequantize_row_q5_0(const void *vx, float *y, int64_t k) {
    const orc_block_q5_0 *x = (const orc_block_q5_0 *)vx;
    for (int64_t i = 0; i < k / ORC_QK32; i++) {
        const float d = orc_fp16_to_fp32(x[i].d);
        uint32_t qh;
        memcpy(&qh, x[i].qh, sizeof(qh));
        for (int j = 0; j < ORC_QK32 / 2; ++j) {
            const uint8_t xh_0 = (uint8_t)(((qh >> j) << 4) & 0x10);
            const uint8_t xh_1 = (uint8_t)((qh >> (j + 12)) & 0x10);
            y[i * ORC_QK32 + j] = (((x[i].qs[j] & 0x0F) | xh_0) - 16) * d;
            y[i * ORC_QK32 + j + ORC_QK32 / 2] = (((x[i].qs[j] >> 4) | xh_1) - 16) * d;
        }
    }
}

void orc_dequantize_row_q8_0(const void *vx, float *y, int64_t k) {
    const orc_block_q8_0 *x = (const orc_block_q8_0 *)vx;
    for (int64_t i = 0; i < k / ORC_QK32; i++) {
        const float d = orc_fp16_to_fp32(x[i].d);
        for (int j = 0; j < ORC_QK32; ++j) y[i * ORC_QK32 + j] = x[i].qs[j] * d;
    }
}

/* ggml_vec_dot_q4_0_q8_0 / q5_0_q8_0 / q8_0_q8_0 (generic): per block an
 * exact integer sum, then sumf += that sum scaled by the two fp16 scales in
 * each function's own expression order */
float orc_vec_dot_q4_0_q8_0(int n, const void *vx, const void *vy) {
    const orc_block_q4_0 *x = (const orc_block_q4_0 *)vx;
    const orc_block_q8_0 *y = (const orc_block_q8_0 *)vy;
    float sumf = 0;
    for (int ib = 0; ib < n / ORC_QK32; ++ib) {
        int sumi0 = 0, sumi1 = 0;
        for (int j = 0; j < ORC_QK32 / 2; ++j) {
            const int v0 = (x[ib].qs[j] & 0x0F) - 8;
            const int v1 = (x[ib].qs[j] >> 4) - 8;
            sumi0 += v0 * y[ib].qs[j];
            sumi1 += v1 * y[ib].qs[j + ORC_QK32 / 2];
        }
        const int sumi = sumi0 + sumi1;
        sumf += sumi * orc_fp16_to_fp32(x[ib].d) * orc_fp16_to_fp32(y[ib].d);
    }
    return sumf;
}

float orc_vec_dot_q5_0_q8_0(int n, const void *vx, const void *vy) {
    const orc_block_q5_0 *x = (const orc_block_q5_0 *)vx;
    const orc_block_q8_0 *y = (const orc_block_q8_0 *)vy;
    float sumf = 0;
    for (int ib = 0; ib < n / ORC_QK32; ++ib) {
        uint32_t qh;
        memcpy(&qh, x[ib].qh, sizeof(qh));
        int sumi0 = 0, sumi1 = 0;
        for (int j = 0; j < ORC_QK32 / 2; ++j) {
            const uint8_t xh_0 = (uint8_t)(((qh & (1u << j)) >> j) << 4);
            const uint8_t xh_1 = (uint8_t)((qh & (1u << (j + 16))) >> (j + 12));
            const int32_t x0 = (int8_t)(((x[ib].qs[j] & 0x0F) | xh_0) - 16);
            const int32_t x1 = (int8_t)(((x[ib].qs[j] >> 4) | xh_1) - 16);
            sumi0 += x0 * y[ib].qs[j];
            sumi1 += x1 * y[ib].qs[j + ORC_QK32 / 2];
        }
        const int sumi = sumi0 + sumi1;
        sumf += (orc_fp16_to_fp32(x[ib].d) * orc_fp16_to_fp32(y[ib].d)) * sumi;
    }
    return sumf;
}

float orc_vec_dot_q8_0_q8_0(int n, const void *vx, const void *vy) {
    const orc_block_q8_0 *x = (const orc_block_q8_0 *)vx;
    const orc_block_q8_0 *y = (const orc_block_q8_0 *)vy;
    float sumf = 0;
    for (int ib = 0; ib < n / ORC_QK32; ++ib) {
        int sumi = 0;
        for (int j = 0; j < ORC_QK32; j++) sumi += x[ib].qs[j] * y[ib].qs[j];
        sumf += sumi * (orc_fp16_to_fp32(x[ib].d) * orc_fp16_to_fp32(y[ib].d));
    }
    return sumf;
}

float orc_vec_dot_f16(int n, const uint16_t *x, const uint16_t *y) {
    double sumf = 0.0;
    for (int i = 0; i < n; ++i) sumf += (double)(orc_fp16_to_fp32(x[i]) * orc_fp16_to_fp32(y[i]));
    return (float)sumf;
}

size_t orc_row_size(int type, int64_t k) {
    switch (type) {
    case ORC_TYPE_F32: return (size_t)k * 4;
    case ORC_TYPE_F16: return (size_t)k * 2;
    case ORC_TYPE_Q4_K: return (size_t)(k / QK_K) * sizeof(orc_block_q4_K);
    case ORC_TYPE_Q6_K: return (size_t)(k / QK_K) * sizeof(orc_block_q6_K);
    case ORC_TYPE_Q8_K: return (size_t)(k / QK_K) * sizeof(orc_block_q8_K);
    case ORC_TYPE_Q4_0: return (size_t)(k / ORC_QK32) * sizeof(orc_block_q4_0);
    case ORC_TYPE_Q5_0: return (size_t)(k / ORC_QK32) * sizeof(orc_block_q5_0);
    case ORC_TYPE_Q8_0: return (size_t)(k / ORC_QK32) * sizeof(orc_block_q8_0);
    default: return 0;
    }
}

void orc_quantize_rows(int type, const float *x, void *y, int64_t nrows, int64_t k, int nthreads) {
    const size_t rs = orc_row_size(type, k);
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t r = 0; r < nrows; r++) {
        const float *xr = x + r * k;
        void *yr = (char *)y + (size_t)r * rs;
        if (type == ORC_TYPE_Q4_K) orc_quantize_row_q4_K(xr, yr, k);
        else if (type == ORC_TYPE_Q6_K) orc_quantize_row_q6_K(xr, yr, k, 0);
        else if (type == ORC_TYPE_Q8_K) orc_quantize_row_q8_K(xr, yr, k);
        else if (type == ORC_TYPE_Q4_0) orc_quantize_row_q4_0(xr, yr, k);
        else if (type == ORC_TYPE_Q5_0) orc_quantize_row_q5_0(xr, yr, k);
        else if (type == ORC_TYPE_Q8_0) orc_quantize_row_q8_0(xr, yr, k);
        else if (type == ORC_TYPE_F16) {
            uint16_t *h = (uint16_t *)yr;
            for (int64_t i = 0; i < k; i++) h[i] = orc_fp32_to_fp16(xr[i]);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* k-quant x Q8_K dot products: ggml_vec_dot_q{4,6}_K_q8_K (generic form).  */
/* The integer part of each super-block is exact; the fp32 scaling follows  */
/* the generic 8-lane accumulation order.                                   */
/* ------------------------------------------------------------------------ */
float orc_vec_dot_q4_K_q8_K(int n, const void *vx, const void *vy) {
    const orc_block_q4_K *x = (const orc_block_q4_K *)vx;
    const orc_block_q8_K *y = (const orc_block_q8_K *)vy;
    const int nb = n / QK_K;
    int8_t aux8[QK_K];
    int16_t aux16[8];
    float sums[8];
    int32_t aux32[8];
    memset(sums, 0, sizeof(sums));
    float sumf = 0;
    for (int i = 0; i < nb; ++i) {
        const uint8_t *q4 = x[i].qs;
        const int8_t *q8 = y[i].qs;
        memset(aux32, 0, sizeof(aux32));
        int8_t *a = aux8;
        for (int j = 0; j < QK_K / 64; ++j) {
            for (int l = 0; l < 32; ++l) a[l] = (int8_t)(q4[l] & 0xF);
            a += 32;
            for (int l = 0; l < 32; ++l) a[l] = (int8_t)(q4[l] >> 4);
            a += 32;
            q4 += 32;
        }
        uint8_t scales[8], mins[8];
        for (int j = 0; j < 8; ++j) get_scale_min_k4(j, x[i].scales, &scales[j], &mins[j]);
        int sumi = 0;
        for (int j = 0; j < QK_K / 16; ++j) sumi += y[i].bsums[j] * mins[j / 2];
        a = aux8;
        int is = 0;
        for (int j = 0; j < QK_K / 32; ++j) {
            int32_t scale = scales[is++];
            for (int r = 0; r < 4; ++r) {
                for (int l = 0; l < 8; ++l) aux16[l] = (int16_t)(q8[l] * a[l]);
                for (int l = 0; l < 8; ++l) aux32[l] += scale * aux16[l];
                q8 += 8;
                a += 8;
            }
        }
        const float d = orc_fp16_to_fp32(x[i].d) * y[i].d;
        for (int l = 0; l < 8; ++l) sums[l] += d * aux32[l];
        const float dmin = orc_fp16_to_fp32(x[i].dmin) * y[i].d;
        sumf -= dmin * sumi;
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

float orc_vec_dot_q6_K_q8_K(int n, const void *vx, const void *vy) {
    const orc_block_q6_K *x = (const orc_block_q6_K *)vx;
    const orc_block_q8_K *y = (const orc_block_q8_K *)vy;
    const int nb = n / QK_K;
    int8_t aux8[QK_K];
    int16_t aux16[8];
    float sums[8];
    int32_t aux32[8];
    memset(sums, 0, sizeof(sums));
    float sumf = 0;
    for (int i = 0; i < nb; ++i) {
        const uint8_t *q4 = x[i].ql;
        const uint8_t *qh = x[i].qh;
        const int8_t *q8 = y[i].qs;
        memset(aux32, 0, sizeof(aux32));
        int8_t *a = aux8;
        for (int j = 0; j < QK_K; j += 128) {
            for (int l = 0; l < 32; ++l) {
                a[l + 0] = (int8_t)((q4[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                a[l + 32] = (int8_t)((q4[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                a[l + 64] = (int8_t)((q4[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                a[l + 96] = (int8_t)((q4[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            }
            a += 128;
            q4 += 64;
            qh += 32;
        }
        a = aux8;
        int is = 0;
        for (int j = 0; j < QK_K / 16; ++j) {
            int scale = x[i].scales[is++];
            for (int r = 0; r < 2; ++r) {
                for (int l = 0; l < 8; ++l) aux16[l] = (int16_t)(q8[l] * a[l]);
                for (int l = 0; l < 8; ++l) aux32[l] += scale * aux16[l];
                q8 += 8;
                a += 8;
            }
        }
        const float d = orc_fp16_to_fp32(x[i].d) * y[i].d;
        for (int l = 0; l < 8; ++l) sums[l] += d * aux32[l];
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

/* ------------------------------------------------------------------------ */
/* The same two dots on AVX-512 (BW + VNNI), bit for bit the scalar forms    */
/* above: the generic order keeps eight int32 sums aux32[l], l = position   */
/* mod 8, each an exact integer, then one fp32 product-and-add per l and    */
/* block.  Here a sub-block's weight codes times its scale become int16      */
/* (|a * sc| <= 15 * 63 / 32 * 128, exact), the Q8_K codes int16, both       */
/* permuted so that each int32 lane pairs positions k and k + 8 (the same    */
/* class), and vpdpwssd accumulates the pairs: lane i holds class i mod 8.   */
/* Integer sums do not depend on their order, so aux32 is the scalar one,   */
/* and the fp32 steps are the scalar steps.  Used by the CPU baseline when  */
/* the host has AVX-512 VNNI (orc_set_simd); the scalar forms stay the      */
/* checker's definition.                                                    */
/* ------------------------------------------------------------------------ */
#if defined(__x86_64__)
#include <immintrin.h>
#define ORC_AVX512 __attribute__((target("avx512f,avx512bw,avx512vnni")))

/* int16 order [0, 8, 1, 9, .., 7, 15, 16, 24, 17, 25, .., 23, 31] */
ORC_AVX512 static inline __m512i orc_pair_perm(void) {
    return _mm512_set_epi16(31, 23, 30, 22, 29, 21, 28, 20, 27, 19, 26, 18, 25, 17, 24, 16,
                            15, 7, 14, 6, 13, 5, 12, 4, 11, 3, 10, 2, 9, 1, 8, 0);
}

/* acc += (codes x scale-vector) . (q8 codes), 32 positions, both int16-widened */
ORC_AVX512 static inline __m512i orc_dot32(__m512i acc, __m256i a8, int is_signed_a, __m512i scv,
                                            const int8_t *q8, __m512i perm) {
    const __m512i a16 = is_signed_a ? _mm512_cvtepi8_epi16(a8) : _mm512_cvtepu8_epi16(a8);
    const __m512i as = _mm512_permutexvar_epi16(perm, _mm512_mullo_epi16(a16, scv));
    const __m512i x16 = _mm512_permutexvar_epi16(perm, _mm512_cvtepi8_epi16(_mm256_loadu_si256((const __m256i *)q8)));
    return _mm512_dpwssd_epi32(acc, as, x16);
}

/* aux32[l] = lane l + lane l + 8 */
ORC_AVX512 static inline void orc_fold8(__m512i acc, int32_t aux32[8]) {
    const __m256i lo = _mm512_castsi512_si256(acc), hi = _mm512_extracti64x4_epi64(acc, 1);
    _mm256_storeu_si256((__m256i *)aux32, _mm256_add_epi32(lo, hi));
}

ORC_AVX512 static float orc_vec_dot_q4_K_q8_K_avx512(int n, const void *vx, const void *vy) {
    const orc_block_q4_K *x = (const orc_block_q4_K *)vx;
    const orc_block_q8_K *y = (const orc_block_q8_K *)vy;
    const int nb = n / QK_K;
    const __m512i perm = orc_pair_perm();
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    float sums[8];
    int32_t aux32[8];
    memset(sums, 0, sizeof(sums));
    float sumf = 0;
    for (int i = 0; i < nb; ++i) {
        uint8_t scales[8], mins[8];
        for (int j = 0; j < 8; ++j) get_scale_min_k4(j, x[i].scales, &scales[j], &mins[j]);
        int sumi = 0;
        for (int j = 0; j < QK_K / 16; ++j) sumi += y[i].bsums[j] * mins[j / 2];
        __m512i acc = _mm512_setzero_si512();
        for (int c = 0; c < QK_K / 64; ++c) {
            /* sub-block 2c: low nibbles of qs[32c ..], 2c + 1: high nibbles */
            const __m256i q = _mm256_loadu_si256((const __m256i *)(x[i].qs + 32 * c));
            const __m256i lo = _mm256_and_si256(q, m4);
            const __m256i hi = _mm256_and_si256(_mm256_srli_epi16(q, 4), m4);
            acc = orc_dot32(acc, lo, 0, _mm512_set1_epi16((short)scales[2 * c]), y[i].qs + 64 * c, perm);
            acc = orc_dot32(acc, hi, 0, _mm512_set1_epi16((short)scales[2 * c + 1]), y[i].qs + 64 * c + 32, perm);
        }
        orc_fold8(acc, aux32);
        const float d = orc_fp16_to_fp32(x[i].d) * y[i].d;
        for (int l = 0; l < 8; ++l) sums[l] += d * aux32[l];
        const float dmin = orc_fp16_to_fp32(x[i].dmin) * y[i].d;
        sumf -= dmin * sumi;
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

ORC_AVX512 static float orc_vec_dot_q6_K_q8_K_avx512(int n, const void *vx, const void *vy) {
    const orc_block_q6_K *x = (const orc_block_q6_K *)vx;
    const orc_block_q8_K *y = (const orc_block_q8_K *)vy;
    const int nb = n / QK_K;
    const __m512i perm = orc_pair_perm();
    const __m256i m4 = _mm256_set1_epi8(0x0F), m3 = _mm256_set1_epi8(3), c32 = _mm256_set1_epi8(32);
    float sums[8];
    int32_t aux32[8];
    memset(sums, 0, sizeof(sums));
    float sumf = 0;
    for (int i = 0; i < nb; ++i) {
        __m512i acc = _mm512_setzero_si512();
        for (int h = 0; h < 2; ++h) {   /* 128 values: ql[64 h ..], qh[32 h ..] */
            const __m256i ql0 = _mm256_loadu_si256((const __m256i *)(x[i].ql + 64 * h));
            const __m256i ql1 = _mm256_loadu_si256((const __m256i *)(x[i].ql + 64 * h + 32));
            const __m256i qh = _mm256_loadu_si256((const __m256i *)(x[i].qh + 32 * h));
            __m256i a[4];
            a[0] = _mm256_or_si256(_mm256_and_si256(ql0, m4), _mm256_slli_epi16(_mm256_and_si256(qh, m3), 4));
            a[1] = _mm256_or_si256(_mm256_and_si256(ql1, m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qh, 2), m3), 4));
            a[2] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(ql0, 4), m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qh, 4), m3), 4));
            a[3] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(ql1, 4), m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qh, 6), m3), 4));
            for (int r = 0; r < 4; ++r) {
                /* values 128 h + 32 r .. + 31: scales 8 h + 2 r (first 16), + 1 (last 16) */
                const __m256i as = _mm256_sub_epi8(a[r], c32);
                const int j = 8 * h + 2 * r;
                const __m512i scv = _mm512_mask_blend_epi16(0xFFFF0000u, _mm512_set1_epi16(x[i].scales[j]),
                                                            _mm512_set1_epi16(x[i].scales[j + 1]));
                acc = orc_dot32(acc, as, 1, scv, y[i].qs + 128 * h + 32 * r, perm);
            }
        }
        orc_fold8(acc, aux32);
        const float d = orc_fp16_to_fp32(x[i].d) * y[i].d;
        for (int l = 0; l < 8; ++l) sums[l] += d * aux32[l];
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

static int orc_simd_on = 0;

int orc_set_simd(int on) {
    __builtin_cpu_init();
    const int have = __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
                     __builtin_cpu_supports("avx512vnni");
    orc_simd_on = on && have;
    return orc_simd_on;
}
#else
static int orc_simd_on = 0;
int orc_set_simd(int on) { (void)on; return 0; }
#endif

/* the dot the mul_mat_id below uses: scalar, or the AVX-512 form when on */
static float orc_dot_kq(int type, int n, const void *x, const void *y) {
#if defined(__x86_64__)
    if (orc_simd_on)
        return type == ORC_TYPE_Q4_K ? orc_vec_dot_q4_K_q8_K_avx512(n, x, y) : orc_vec_dot_q6_K_q8_K_avx512(n, x, y);
#endif
    return type == ORC_TYPE_Q4_K ? orc_vec_dot_q4_K_q8_K(n, x, y) : orc_vec_dot_q6_K_q8_K(n, x, y);
}

float orc_vec_dot_kq_simd(int type, int n, const void *x, const void *y) {
#if defined(__x86_64__)
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
        __builtin_cpu_supports("avx512vnni"))
        return type == ORC_TYPE_Q4_K ? orc_vec_dot_q4_K_q8_K_avx512(n, x, y) : orc_vec_dot_q6_K_q8_K_avx512(n, x, y);
#endif
    return type == ORC_TYPE_Q4_K ? orc_vec_dot_q4_K_q8_K(n, x, y) : orc_vec_dot_q6_K_q8_K(n, x, y);
}

/* ------------------------------------------------------------------------ */
/* seeded synthetic data                                                    */
/* ------------------------------------------------------------------------ */
static inline uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

uint64_t orc_rng_u64(uint64_t seed, uint64_t stream, uint64_t i) {
    const uint64_t key = splitmix64(seed ^ splitmix64(stream + 0x1234567ULL));
    return splitmix64(key + i * 0xD1B54A32D192ED03ULL);
}

/* log(x) for normal x > 0: x = m * 2^e with m in [sqrt(1/2), sqrt(2)),
 * log(m) = 2 atanh(s), s = (m-1)/(m+1), |s| <= 0.1716, series to s^25. */
double orc_poly_log(double x) {
    uint64_t bits = d2u(x);
    int e = (int)((bits >> 52) & 0x7ff) - 1022;
    double m = u2d((bits & 0x000FFFFFFFFFFFFFULL) | 0x3FE0000000000000ULL); /* [0.5, 1) */
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

/* sin and cos of 2*pi*u for u in [0, 1): quadrant from 4u (exact), then
 * Taylor series on [0, pi/2) to degree 23 / 22. */
void orc_poly_sincos_2pi(double u, double *s_out, double *c_out) {
    const double u4 = u * 4.0;
    const double q = floor(u4);
    const double f = u4 - q;
    const double a = f * 1.57079632679489661923;
    const double z = a * a;
    double sp = -1.0 / 25852016738884976640000.0;      /* -1/23! */
    sp = sp * z + 1.0 / 51090942171709440000.0;        /* 1/21! */
    sp = sp * z - 1.0 / 121645100408832000.0;          /* 1/19! */
    sp = sp * z + 1.0 / 355687428096000.0;             /* 1/17! */
    sp = sp * z - 1.0 / 1307674368000.0;               /* 1/15! */
    sp = sp * z + 1.0 / 6227020800.0;                  /* 1/13! */
    sp = sp * z - 1.0 / 39916800.0;                    /* 1/11! */
    sp = sp * z + 1.0 / 362880.0;                      /* 1/9!  */
    sp = sp * z - 1.0 / 5040.0;                        /* 1/7!  */
    sp = sp * z + 1.0 / 120.0;                         /* 1/5!  */
    sp = sp * z - 1.0 / 6.0;                           /* 1/3!  */
    sp = sp * z + 1.0;
    const double sn = a * sp;
    double cp = 1.0 / 1124000727777607680000.0;        /* 1/22! */
    cp = cp * z - 1.0 / 2432902008176640000.0;         /* 1/20! */
    cp = cp * z + 1.0 / 6402373705728000.0;            /* 1/18! */
    cp = cp * z - 1.0 / 20922789888000.0;              /* 1/16! */
    cp = cp * z + 1.0 / 87178291200.0;                 /* 1/14! */
    cp = cp * z - 1.0 / 479001600.0;                   /* 1/12! */
    cp = cp * z + 1.0 / 3628800.0;                     /* 1/10! */
    cp = cp * z - 1.0 / 40320.0;                       /* 1/8!  */
    cp = cp * z + 1.0 / 720.0;                         /* 1/6!  */
    cp = cp * z - 1.0 / 24.0;                          /* 1/4!  */
    cp = cp * z + 1.0 / 2.0;                           /* 1/2!  */
    const double cs = 1.0 - z * cp;
    const int qi = (int)q;
    if (qi == 0) { *s_out = sn; *c_out = cs; }
    else if (qi == 1) { *s_out = cs; *c_out = -sn; }
    else if (qi == 2) { *s_out = -sn; *c_out = -cs; }
    else { *s_out = -cs; *c_out = sn; }
}

/* value i of a normal stream: pair j = i/2 uses draws 2j, 2j+1; even i takes
 * the cosine branch, odd i the sine branch. */
static inline float normal_at(uint64_t seed, uint64_t stream, uint64_t i, double mean, double sd) {
    const uint64_t j = i >> 1;
    const uint64_t r1 = orc_rng_u64(seed, stream, 2 * j);
    const uint64_t r2 = orc_rng_u64(seed, stream, 2 * j + 1);
    const double u1 = ((double)(r1 >> 11) + 0.5) * (1.0 / 9007199254740992.0);
    const double u2 = (double)(r2 >> 11) * (1.0 / 9007199254740992.0);
    const double r = sqrt(-2.0 * orc_poly_log(u1));
    double s, c;
    orc_poly_sincos_2pi(u2, &s, &c);
    const double z = (i & 1) ? r * s : r * c;
    return (float)(mean + sd * z);
}

void orc_fill_normal(float *out, int64_t n, uint64_t seed, uint64_t stream,
                     float mean, float stddev, int nthreads) {
    const double m = (double)mean, sd = (double)stddev;
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t i = 0; i < n; i++) out[i] = normal_at(seed, stream, (uint64_t)i, m, sd);
}

/* ------------------------------------------------------------------------ */
/* router / gating / dispatch                                               */
/* ------------------------------------------------------------------------ */
void orc_router_logits(const float *W, const float *b, const float *x,
                       int64_t T, int D, int E, float *logits, int nthreads) {
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t t = 0; t < T; t++) {
        const float *xt = x + t * (int64_t)D;
        for (int e = 0; e < E; e++) {
            const float *we = W + (int64_t)e * D;
            double acc = 0.0;
            for (int c0 = 0; c0 < D; c0 += 64) {
                /* inside a 64-wide chunk: d = c0 + 16*g + s, s outer, g inner */
                double part = 0.0;
                for (int s = 0; s < 16; s++)
                    for (int g = 0; g < 4; g++) {
                        const int d = c0 + 16 * g + s;
                        if (d < D) part += (double)we[d] * (double)xt[d];
                    }
                acc += part;
            }
            float v = (float)acc;
            if (b) v = v + b[e];
            logits[t * E + e] = v;
        }
    }
}

void orc_top_k(const float *logits, int64_t T, int E, int K, int32_t *sel) {
    for (int64_t t = 0; t < T; t++) {
        const float *l = logits + t * E;
        int32_t *s = sel + t * K;
        /* repeated selection: the largest not yet taken; strict > keeps the
         * lower id on ties */
        for (int k = 0; k < K; k++) {
            int best = -1;
            for (int e = 0; e < E; e++) {
                int taken = 0;
                for (int j = 0; j < k; j++) if (s[j] == e) { taken = 1; break; }
                if (taken) continue;
                if (best < 0 || l[e] > l[best]) best = e;
            }
            s[k] = best;
        }
    }
}

void orc_softmax_selected(const float *logits, const int32_t *sel,
                          int64_t T, int E, int K, float *w) {
    for (int64_t t = 0; t < T; t++) {
        float v[512];
        for (int k = 0; k < K; k++) v[k] = logits[t * E + sel[t * K + k]];
        float max = -INFINITY;
        for (int k = 0; k < K; k++) max = MAX(max, v[k]);
        double sum = 0.0;
        for (int k = 0; k < K; k++) {
            float val = expf(v[k] - max);
            sum += (double)val;
            v[k] = val;
        }
        sum = 1.0 / sum;
        const float s = (float)sum;
        for (int k = 0; k < K; k++) w[t * K + k] = v[k] * s;
    }
}

/* Router gating variants (kind 0: top-k on logits + softmax over the K;
 * kind 1: nemotronomni_model.cpp:344-354 - s = sigmoid(logit), top-k on
 * s + sel_bias, w = s / (sum s + eps) * scaling; kind 2:
 * diffusiongemma_model.cpp:923-932 - p = soft_max over all E logits, top-k
 * on p, w = p / sum_K p); expert_scale multiplies the weights
 * (diffusiongemma_model.cpp:932-936).  The sigmoid and the exponentials of
 * kind 2 are evaluated in double and rounded once to float (the restatement's
 * choice, so rankings do not depend on a float exp's last bit; ggml's
 * ggml_sigmoid / soft_max use float exp); weight sums are double sums in slot
 * order, rounded to float (kind 1 then adds eps); kind 2's full softmax is
 * ggml's: max, e = fl32(exp(l - max)) with the difference in float, the sum of
 * the e in double in expert order, p = e * fl32(1 / sum).  Ties rank the lower
 * id first (strict > in the repeated selection). */
static float orc_sigmoid(float x) { return (float)(1.0 / (1.0 + exp(-(double)x))); }

void orc_route_gated(const float *logits, int64_t T, int E, int K, int kind, const float *sel_bias,
                     const float *expert_scale, float scaling, float eps, int32_t *sel, float *w) {
    for (int64_t t = 0; t < T; t++) {
        const float *l = logits + t * E;
        int32_t *s = sel + t * K;
        float score[1024];
        if (kind == 2) {
            float mx = -INFINITY;
            for (int e = 0; e < E; e++) mx = MAX(mx, l[e]);
            double sum = 0.0;
            for (int e = 0; e < E; e++) {
                score[e] = (float)exp((double)(l[e] - mx));
                sum += (double)score[e];
            }
            const float inv = (float)(1.0 / sum);
            for (int e = 0; e < E; e++) score[e] = score[e] * inv;
        } else {
            for (int e = 0; e < E; e++)
                score[e] = kind == 1 ? orc_sigmoid(l[e]) + (sel_bias ? sel_bias[e] : 0.f) : l[e];
        }
        for (int k = 0; k < K; k++) {
            int best = -1;
            for (int e = 0; e < E; e++) {
                int taken = 0;
                for (int j = 0; j < k; j++) if (s[j] == e) { taken = 1; break; }
                if (taken) continue;
                if (best < 0 || score[e] > score[best]) best = e;
            }
            s[k] = best;
        }
        if (kind == 1) {
            float sv[512];
            double sum = 0.0;
            for (int k = 0; k < K; k++) {
                sv[k] = orc_sigmoid(l[s[k]]);
                sum += (double)sv[k];
            }
            for (int k = 0; k < K; k++) w[t * K + k] = sv[k] / ((float)sum + eps) * scaling;
        } else if (kind == 2) {
            double sum = 0.0;
            for (int k = 0; k < K; k++) sum += (double)score[s[k]];
            const float fs = (float)sum;
            for (int k = 0; k < K; k++) w[t * K + k] = score[s[k]] / fs;
        } else {
            orc_softmax_selected(logits + t * E, s, 1, E, K, w + t * K);
        }
        if (expert_scale)
            for (int k = 0; k < K; k++) w[t * K + k] = w[t * K + k] * expert_scale[s[k]];
    }
}

void orc_dispatch(const int32_t *sel, int64_t T, int K, int E,
                  int32_t *counts, int32_t *offsets, int32_t *perm) {
    for (int e = 0; e < E; e++) counts[e] = 0;
    for (int64_t i = 0; i < T * K; i++) counts[sel[i]]++;
    offsets[0] = 0;
    for (int e = 0; e < E; e++) offsets[e + 1] = offsets[e] + counts[e];
    int32_t *cur = (int32_t *)malloc(sizeof(int32_t) * (size_t)(E > 0 ? E : 1));
    for (int e = 0; e < E; e++) cur[e] = offsets[e];
    for (int64_t t = 0; t < T; t++)
        for (int k = 0; k < K; k++) {
            const int e = sel[t * K + k];
            perm[cur[e]++] = (int32_t)(t * K + k);
        }
    free(cur);
}

/* ------------------------------------------------------------------------ */
/* ggml_mul_mat_id                                                          */
/* ------------------------------------------------------------------------ */
static void dequant_row_any(int type, const void *row, float *out, int64_t k) {
    if (type == ORC_TYPE_Q4_K) orc_dequantize_row_q4_K(row, out, k);
    else if (type == ORC_TYPE_Q6_K) orc_dequantize_row_q6_K(row, out, k);
    else if (type == ORC_TYPE_F32) memcpy(out, row, sizeof(float) * (size_t)k);
    else if (type == ORC_TYPE_Q4_0) orc_dequantize_row_q4_0(row, out, k);
    else if (type == ORC_TYPE_Q5_0) orc_dequantize_row_q5_0(row, out, k);
    else if (type == ORC_TYPE_Q8_0) orc_dequantize_row_q8_0(row, out, k);
    else if (type == ORC_TYPE_F16) {
        const uint16_t *h = (const uint16_t *)row;
        for (int64_t i = 0; i < k; i++) out[i] = orc_fp16_to_fp32(h[i]);
    }
}

int orc_mul_mat_id(int type, const void *as, int64_t Kin, int64_t N, int E,
                   const float *b, int ne11, const int32_t *ids, int n_used,
                   int64_t T, float *dst, int exact, int nthreads) {
    if (!as || !b || !ids || !dst || Kin <= 0 || N <= 0 || E <= 0 || n_used <= 0 || T < 0)
        return -1;
    if (ne11 != 1 && ne11 != n_used) return -1;
    const int kq = (type == ORC_TYPE_Q4_K || type == ORC_TYPE_Q6_K);
    const int b32 = (type == ORC_TYPE_Q4_0 || type == ORC_TYPE_Q5_0 || type == ORC_TYPE_Q8_0);
    const int f16 = type == ORC_TYPE_F16;
    if (kq && (Kin % QK_K)) return -1;
    if (b32 && (Kin % ORC_QK32)) return -1;
    if (!kq && !b32 && type != ORC_TYPE_F32 && !f16) return -1;
    for (int64_t i = 0; i < T * n_used; i++)
        if (ids[i] < 0 || ids[i] >= E) return -1;
    if (T == 0) return 0;

    const size_t rs = orc_row_size(type, Kin);
    const int64_t nbrows = T * ne11;

    /* activations in the weight type's vec_dot_type: Q8_K rows (k-quants),
     * Q8_0 rows (32-value formats), fp16 rows (F16), or fp32/fp64 as given */
    orc_block_q8_K *bq = NULL;
    orc_block_q8_0 *bq0 = NULL;
    uint16_t *bh = NULL;
    if (kq && !exact) {
        bq = (orc_block_q8_K *)malloc(sizeof(orc_block_q8_K) * (size_t)(Kin / QK_K) * (size_t)nbrows);
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
        for (int64_t r = 0; r < nbrows; r++)
            orc_quantize_row_q8_K(b + r * Kin, bq + r * (Kin / QK_K), Kin);
    }
    if (b32 && !exact) {
        bq0 = (orc_block_q8_0 *)malloc(sizeof(orc_block_q8_0) * (size_t)(Kin / ORC_QK32) * (size_t)nbrows);
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
        for (int64_t r = 0; r < nbrows; r++)
            orc_quantize_row_q8_0(b + r * Kin, bq0 + r * (Kin / ORC_QK32), Kin);
    }
    if (f16 && !exact) {
        bh = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)Kin * (size_t)nbrows);
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
        for (int64_t r = 0; r < nbrows; r++)
            for (int64_t q = 0; q < Kin; q++) bh[r * Kin + q] = orc_fp32_to_fp16(b[r * Kin + q]);
    }

    /* group (t, k) rows per expert, tokens outer / slots inner */
    int32_t *counts = (int32_t *)calloc((size_t)E, sizeof(int32_t));
    int32_t *offs = (int32_t *)malloc(sizeof(int32_t) * (size_t)(E + 1));
    int32_t *perm = (int32_t *)malloc(sizeof(int32_t) * (size_t)(T * n_used));
    orc_dispatch(ids, T, n_used, E, counts, offs, perm);

    /* work items: (expert, chunk of 16 weight rows) */
    const int64_t RCH = 16;
    const int64_t nch = (N + RCH - 1) / RCH;
#pragma omp parallel num_threads(nthr(nthreads))
    {
        float *wrow = (float *)malloc(sizeof(float) * (size_t)Kin);
#pragma omp for schedule(dynamic, 1) collapse(2)
        for (int e = 0; e < E; e++) {
            for (int64_t c = 0; c < nch; c++) {
                const int32_t n_rows = counts[e];
                if (n_rows == 0) continue;
                const char *We = (const char *)as + (size_t)e * (size_t)N * rs;
                for (int64_t n = c * RCH; n < MIN(N, (c + 1) * RCH); n++) {
                    const char *wr = We + (size_t)n * rs;
                    if (exact || type == ORC_TYPE_F32) dequant_row_any(type, wr, wrow, Kin);
                    for (int32_t i = 0; i < n_rows; i++) {
                        const int32_t p = perm[offs[e] + i];
                        const int64_t t = p / n_used;
                        const int k = p % n_used;
                        const int64_t brow = t * ne11 + (ne11 == 1 ? 0 : k);
                        float v;
                        if (exact) {
                            const float *bb = b + brow * Kin;
                            double acc = 0.0;
                            for (int64_t q = 0; q < Kin; q++) acc += (double)wrow[q] * (double)bb[q];
                            v = (float)acc;
                        } else if (kq) {
                            const void *yb = bq + brow * (Kin / QK_K);
                            v = orc_dot_kq(type, (int)Kin, wr, yb);
                        } else if (b32) {
                            const void *yb = bq0 + brow * (Kin / ORC_QK32);
                            v = type == ORC_TYPE_Q8_0   ? orc_vec_dot_q8_0_q8_0((int)Kin, wr, yb)
                                : type == ORC_TYPE_Q5_0 ? orc_vec_dot_q5_0_q8_0((int)Kin, wr, yb)
                                                        : orc_vec_dot_q4_0_q8_0((int)Kin, wr, yb);
                        } else if (f16) {
                            v = orc_vec_dot_f16((int)Kin, (const uint16_t *)wr, bh + brow * Kin);
                        } else {
                            const float *bb = b + brow * Kin;
                            float acc = 0.f;
                            for (int64_t q = 0; q < Kin; q++) acc += wrow[q] * bb[q];
                            v = acc;
                        }
                        dst[(t * n_used + k) * N + n] = v;
                    }
                }
            }
        }
        free(wrow);
    }
    free(counts);
    free(offs);
    free(perm);
    free(bq);
    free(bq0);
    free(bh);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* GLU variants (ggml_vec_{swiglu,geglu_erf,geglu}_f32 element formulas)    */
/* ------------------------------------------------------------------------ */
#define SQRT_2_INV 0.70710678118654752440084436210484f
#define SQRT_2_OVER_PI 0.79788456080286535587989211986876f
#define GELU_COEF_A 0.044715f

float orc_act_pair(int act, float a, float b) {
    switch (act) {
    case ORC_ACT_SILU: return (a / (1.0f + expf(-a))) * b;
    case ORC_ACT_GELU_ERF_GP1: {
        const float g1 = b + 1.0f;                                  /* ggml_add(g, one_fill) */
        return 0.5f * a * (1.0f + erff(a * SQRT_2_INV)) * g1;
    }
    case ORC_ACT_GELU_TANH:
        return 0.5f * a * (1.0f + tanhf(SQRT_2_OVER_PI * a * (1.0f + GELU_COEF_A * a * a))) * b;
    case ORC_ACT_GELU_ERF: return 0.5f * a * (1.0f + erff(a * SQRT_2_INV)) * b;
    case ORC_ACT_RELU_SQR: {                                        /* ggml_sqr(ggml_relu(u)) */
        const float r = a > 0.f ? a : 0.f;
        return r * r;
    }
    default: return 0.f;
    }
}

static double act_pair_f64(int act, double a, double b) {
    switch (act) {
    case ORC_ACT_SILU: return a / (1.0 + exp(-a)) * b;
    case ORC_ACT_GELU_ERF_GP1: return 0.5 * a * (1.0 + erf(a * 0.70710678118654752440)) * (b + 1.0);
    case ORC_ACT_GELU_TANH:
        return 0.5 * a * (1.0 + tanh(0.79788456080286535588 * a * (1.0 + 0.044715 * a * a))) * b;
    case ORC_ACT_GELU_ERF: return 0.5 * a * (1.0 + erf(a * 0.70710678118654752440)) * b;
    case ORC_ACT_RELU_SQR: return a > 0.0 ? a * a : 0.0;
    default: return 0.0;
    }
}

/* ------------------------------------------------------------------------ */
/* whole layer                                                              */
/* ------------------------------------------------------------------------ */
/* act rows from the gate (and up) products: gated pairs, or one product */
static void orc_act_rows(int act, int fused, int64_t rows, int I, const float *gu, const float *up, float *out,
                         int exact, int nthreads) {
    const int gated = ORC_ACT_GATED(act);
    const int64_t Ng = gated && fused ? 2 * (int64_t)I : I;
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        for (int i = 0; i < I; i++) {
            float a, bb = 0.f;
            if (!gated) {
                a = gu[r * Ng + i];
            } else if (fused) {
                a = gu[r * Ng + i];
                bb = gu[r * Ng + I + i];
            } else {
                a = gu[r * I + i];
                bb = up[r * I + i];
            }
            out[r * I + i] = exact ? (float)act_pair_f64(act, a, bb) : orc_act_pair(act, a, bb);
        }
    }
}

/* the shared expert of every token: sh[t] = down(act(gate x, up x)) [* sigmoid
 * (gate_inp . x)], each product a mul_mat with Q8_K activations (ggml
 * vec_dot_type) - here mul_mat_id over one expert; the scalar gate row is a
 * router row of one expert (the router's fixed fp64 order) whose sigmoid is
 * evaluated in double and rounded once */
static int orc_shared_expert(const orc_layer *L, const float *x, int64_t T, float *sh, int exact, int nthreads) {
    const int D = L->D, I = L->sh_I;
    const int gated = ORC_ACT_GATED(L->sh_act);
    int32_t *z0 = (int32_t *)calloc((size_t)T, sizeof(int32_t));
    float *g = (float *)malloc(sizeof(float) * (size_t)(T * I));
    float *u = gated ? (float *)malloc(sizeof(float) * (size_t)(T * I)) : NULL;
    float *a = (float *)malloc(sizeof(float) * (size_t)(T * I));
    int rc = orc_mul_mat_id(L->sh_type, L->sh_gate, D, I, 1, x, 1, z0, 1, T, g, exact, nthreads);
    if (!rc && gated) rc = orc_mul_mat_id(L->sh_type, L->sh_up, D, I, 1, x, 1, z0, 1, T, u, exact, nthreads);
    if (!rc) {
        orc_act_rows(L->sh_act, 0, T, I, g, u, a, exact, nthreads);
        rc = orc_mul_mat_id(L->sh_down_type, L->sh_down, I, D, 1, a, 1, z0, 1, T, sh, exact, nthreads);
    }
    if (!rc && L->sh_gate_inp) {
        float *lg = (float *)malloc(sizeof(float) * (size_t)T);
        orc_router_logits(L->sh_gate_inp, NULL, x, T, D, 1, lg, nthreads);
        for (int64_t t = 0; t < T; t++) {
            const float s = orc_sigmoid(lg[t]);
            for (int n = 0; n < D; n++) sh[t * D + n] = sh[t * D + n] * s;   /* ggml_mul(sd, gate_row) */
        }
        free(lg);
    }
    free(z0); free(g); free(u); free(a);
    return rc;
}

int orc_moe_forward(const orc_layer *L, const float *x, int64_t T,
                    const float *res, float *out, orc_debug *dbg,
                    const int32_t *sel_in, const int32_t *down_sel_in, const float *w_in,
                    int exact, int nthreads) {
    if (!L || !x || !out || T < 0) return -1;
    const int D = L->D, E = L->E, K = L->K, I = L->I;
    const int gated = ORC_ACT_GATED(L->act);
    if (D <= 0 || E <= 0 || K <= 0 || K > E || I <= 0) return -1;
    if (!L->gate || !L->down || (gated && !L->fused_gate_up && !L->up)) return -1;
    if (!gated && L->fused_gate_up) return -1;
    if ((!sel_in || !w_in) && !L->router_w) return -1;
    if (L->gating < 0 || L->gating > 2) return -1;
    if (L->sh_I < 0 || (L->sh_I > 0 && (!L->sh_gate || !L->sh_down || (ORC_ACT_GATED(L->sh_act) && !L->sh_up))))
        return -1;
    if (T == 0) return 0;

    float *logits = (float *)malloc(sizeof(float) * (size_t)(T * E));
    int32_t *sel = (int32_t *)malloc(sizeof(int32_t) * (size_t)(T * K));
    int32_t *dsel = (int32_t *)malloc(sizeof(int32_t) * (size_t)(T * K));
    float *w = (float *)malloc(sizeof(float) * (size_t)(T * K));
    if (sel_in && w_in) {
        memcpy(sel, sel_in, sizeof(int32_t) * (size_t)(T * K));
        memcpy(w, w_in, sizeof(float) * (size_t)(T * K));
        memset(logits, 0, sizeof(float) * (size_t)(T * E));
    } else {
        orc_router_logits(L->router_w, L->router_b, x, T, D, E, logits, nthreads);
        orc_route_gated(logits, T, E, K, L->gating, L->sel_bias, L->expert_scale,
                        L->routed_scaling != 0.f ? L->routed_scaling : 1.f, L->gate_eps, sel, w);
    }
    memcpy(dsel, down_sel_in ? down_sel_in : sel, sizeof(int32_t) * (size_t)(T * K));

    const int64_t Ng = gated && L->fused_gate_up ? 2 * (int64_t)I : I;
    float *gu = (float *)malloc(sizeof(float) * (size_t)(T * K * Ng));
    float *up = gated && !L->fused_gate_up ? (float *)malloc(sizeof(float) * (size_t)(T * K * I)) : NULL;
    float *act = (float *)malloc(sizeof(float) * (size_t)(T * K * I));
    float *ff = (float *)malloc(sizeof(float) * (size_t)(T * K * D));
    float *sh = L->sh_I > 0 ? (float *)malloc(sizeof(float) * (size_t)(T * D)) : NULL;
    int rc = 0;

    rc |= orc_mul_mat_id(L->gate_type, L->gate, D, Ng, E, x, 1, sel, K, T, gu, exact, nthreads);
    if (up) rc |= orc_mul_mat_id(L->gate_type, L->up, D, I, E, x, 1, sel, K, T, up, exact, nthreads);
    if (rc) goto done;
    orc_act_rows(L->act, L->fused_gate_up, T * K, I, gu, up, act, exact, nthreads);
    rc |= orc_mul_mat_id(L->down_type, L->down, I, D, E, act, K, dsel, K, T, ff, exact, nthreads);
    if (rc) goto done;
    if (sh) rc |= orc_shared_expert(L, x, T, sh, exact, nthreads);
    if (rc) goto done;

    /* ggml_mul(ff3, w) -> permute/cont -> sum_rows (fp64 accumulation, slot
     * order), + the shared expert (ggml_add(routed, sh)), -> add res */
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t t = 0; t < T; t++) {
        for (int n = 0; n < D; n++) {
            double sum = 0.0;
            for (int k = 0; k < K; k++) {
                if (exact) sum += (double)ff[(t * K + k) * D + n] * (double)w[t * K + k];
                else {
                    const float prod = ff[(t * K + k) * D + n] * w[t * K + k];
                    sum += (double)prod;
                }
            }
            float moe;
            if (sh && exact) moe = (float)(sum + (double)sh[t * D + n]);
            else if (sh) moe = (float)sum + sh[t * D + n];
            else moe = (float)sum;
            out[t * D + n] = res ? res[t * D + n] + moe : moe;
        }
    }

    if (dbg) {
        if (dbg->logits) memcpy(dbg->logits, logits, sizeof(float) * (size_t)(T * E));
        if (dbg->sel) memcpy(dbg->sel, sel, sizeof(int32_t) * (size_t)(T * K));
        if (dbg->w) memcpy(dbg->w, w, sizeof(float) * (size_t)(T * K));
        if (dbg->counts || dbg->offsets || dbg->perm) {
            int32_t *c = (int32_t *)malloc(sizeof(int32_t) * (size_t)E);
            int32_t *o = (int32_t *)malloc(sizeof(int32_t) * (size_t)(E + 1));
            int32_t *p = (int32_t *)malloc(sizeof(int32_t) * (size_t)(T * K));
            orc_dispatch(sel, T, K, E, c, o, p);
            if (dbg->counts) memcpy(dbg->counts, c, sizeof(int32_t) * (size_t)E);
            if (dbg->offsets) memcpy(dbg->offsets, o, sizeof(int32_t) * (size_t)(E + 1));
            if (dbg->perm) memcpy(dbg->perm, p, sizeof(int32_t) * (size_t)(T * K));
            free(c); free(o); free(p);
        }
        if (dbg->act) memcpy(dbg->act, act, sizeof(float) * (size_t)(T * K * I));
        if (dbg->ff) memcpy(dbg->ff, ff, sizeof(float) * (size_t)(T * K * D));
        if (dbg->sh && sh) memcpy(dbg->sh, sh, sizeof(float) * (size_t)(T * D));
    }

done:
    free(logits); free(sel); free(dsel); free(w); free(gu); free(up); free(act); free(ff); free(sh);
    return rc ? -1 : 0;
}
