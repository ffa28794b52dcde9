// k_decode.hip - the whole MoE block for one token in one kernel.
//
// Reference block (one decode step): router mul_mat(+bias) -> top_k ->
// get_rows -> soft_max -> mul_mat_id gate/up -> GLU -> mul_mat_id down ->
// mul(w) -> sum_rows (-> add residual)
//   moondream3: src/models/moondream/moondream.cpp:509-544 (+ residual :547)
//   qwen3omni : src/models/qwen3omni/qwen3omni_model.cpp:759-780
//
// A single-token step reads ~29 MB of expert weights and does almost no
// arithmetic, so its time is the HBM stream plus whatever serial latency
// sits in front of it.  The separate-kernel chain pays a launch gap per
// stage; here every stage lives in one grid of one work-group per CU, and
// the stages meet at two hand-offs:
//
//   A  units a < E: router row a (one wave, fp64 fixed order) and, for
//      a < D/256, Q8_K of x block a.  WG a runs unit a.
//   -- logits --
//   B  every WG ranks the E logits itself (no extra barrier for top-k).
//      Units u < K I / P: P (h, g) row pairs of the selected experts' gate/up
//      rows, DMA'd into LDS (buffer_load ... lds, 1 KB per wave instruction);
//      integer Q4_K x Q8_K dots, GLU, fp32 activations written through.  WG
//      u runs unit u, then DMAs its share of the down rows (they stream
//      while the activations are handed over) and unpacks them into a
//      dot-ready form.
//   -- activations --
//   C  per WG: Q8_K of each slot's activations, down dots from the
//      LDS-resident rows of its columns, weighted combine in slot order
//      (fp64, ggml's sum_rows of the weighted rows) and residual add.
//
// Numerics are the GEMV path's: exact integer dots per 32-value piece,
// fp32 block scaling, act_pair for the GLU, the shared Q8_K and softmax
// code.  Routing is exact: the rank form below selects the same experts in
// the same order as the stable descending argsort of ggml_top_k.
//
// Synchronization.  Values one WG hands to another are written with relaxed
// agent-scope atomic stores (global_store ... sc1) and read with loads that
// carry the same agent-coherent cache policy as agent-scope atomic loads
// (buffer_load ... sc1: the instruction a relaxed agent-scope atomic load
// compiles to), issued only after the poll that saw the producer's completion
// word: every hand-off read is a coherent read at agent scope, whatever an
// XCD's L2 held before.  (Agent-scope acquire / release fences would add a
// whole-L2 invalidate / write-back per work-group and hand-off.)  Each unit
// publishes a 64-bit completion word tagged with the launch epoch (the
// logit itself for an A unit; a B unit's word follows its activation
// stores); consumers poll the words (one coalesced wave load per try).  An
// A unit's logit is stored only after its Q8_K of x is out, so ready logits
// imply ready x.  The epoch is per WG (read at start, stored +1 at the end),
// so all epochs agree at every launch, with no atomics and no reset, and a
// captured graph replays correctly.
//
// No co-residency is assumed: a WG that has not seen a unit complete after
// DecArgs::rescue_polls tries computes the unit itself and publishes it
// again (the same bits).  So a WG only ever waits on a running WG, and the
// kernel cannot deadlock when other work holds some CUs: the plain launch is
// safe anywhere, the cooperative launch is optional.  Waits are bounded all
// the same; a WG whose waits give up writes NaN and sets an error word.
#include "act.hpp"
#include "common.hpp"
#include "kq_dot.hpp"
#include "launch.hpp"
#include "wave_ops.hpp"

namespace mimoe {

typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int DEC_WAVES = 8;
constexpr int DEC_THREADS = DEC_WAVES * 64;
constexpr int DEC_GU_SEG = 9;       // 1 KB DMA segments per wave of gate/up rows
constexpr int DEC_WREG = DEC_LIMIT_UNPACKED_BYTES;   // LDS per wave: gate/up rows, then its slot's unpacked down rows
constexpr int DEC_DN_SEG = 7;       // 1 KB DMA segments per slot of down rows
constexpr int DEC_KMAX = 8;         // slots: one wave each in the down phase
constexpr int DEC_PMAX = 64;        // (h, g) row pairs per WG
constexpr int DEC_CMAX = 64;        // down columns per WG
constexpr unsigned DEC_SPIN_LIMIT = 1u << 20;

// ---------------------------------------------------------------- tagged words
__device__ inline void tw_store(uint64_t *p, uint32_t tag, uint32_t v) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint64_t tw_load(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_dev4(void *base, uint32_t off, uint32_t v) {
    __hip_atomic_store((uint32_t *)((uint8_t *)base + off), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One tagged word: true once it carries `tag` (value in v), false after
// `limit` further tries.
__device__ inline bool tw_wait1(const uint64_t *p, uint32_t tag, unsigned limit, uint32_t &v) {
    uint64_t w = tw_load(p);
    unsigned n = 0;
    while ((uint32_t)(w >> 32) != tag) {
        if (n++ >= limit) return false;
        __builtin_amdgcn_s_sleep(1);
        w = tw_load(p);
    }
    v = (uint32_t)w;
    return true;
}

// workgroup barrier that does not wait for outstanding global loads / DMA
__device__ inline void dec_lds_barrier() { lds_barrier(); }

// True when no thread of the WG saw a unit missing: one ballot per wave, one
// LDS word per wave, one barrier.  (A caller that goes on polling calls
// dec_missing first, whose barriers separate the rounds.)
__device__ inline bool dec_none_missing(int *s_wmiss, bool miss) {
    const bool any = __ballot(miss) != 0;
    if ((threadIdx.x & 63) == 0) s_wmiss[threadIdx.x >> 6] = any;
    dec_lds_barrier();
    int m = 0;
#pragma unroll
    for (int w = 0; w < DEC_WAVES; ++w) m |= s_wmiss[w];
    return m == 0;
}

// Units still missing after a WG's poll: each polling thread appends the (up
// to two) units it did not see complete to an LDS list; returns the list's
// length (uniform).  Three LDS-only barriers.
__device__ inline int dec_missing(int *s_n, int *s_list, int u0, int u1, bool miss0, bool miss1) {
    dec_lds_barrier();   // earlier readers of the list are done
    if (threadIdx.x == 0) *s_n = 0;
    dec_lds_barrier();
    if (miss0) s_list[atomicAdd(s_n, 1)] = u0;
    if (miss1) s_list[atomicAdd(s_n, 1)] = u1;
    dec_lds_barrier();
    return __builtin_amdgcn_readfirstlane(*s_n);
}

// Hand-off reads: 16 / 4 bytes at byte offset off of a buffer of nbytes,
// loaded with the agent-coherent cache policy (sc1) of agent-scope atomic loads
constexpr int CPOL_SC1 = 16;
__device__ inline __amdgpu_buffer_rsrc_t co_rsrc(const void *p, uint32_t nbytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)nbytes, 0x00020000);
}
__device__ inline u32x4 co_ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, CPOL_SC1);
}
__device__ inline uint32_t co_ld4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, CPOL_SC1);
}

// reinterpret a 32-bit value (passed by value: this toolchain's
// __builtin_bit_cast of an ext-vector element reads element 0)
__device__ inline float as_float(uint32_t u) { return __builtin_bit_cast(float, u); }

// ---------------------------------------------------------------- phase A
// logit of expert e: the router's fixed fp64 order (64-wide chunk c: sum over
// s = 0..15, g = 0..3 of W[64c+16g+s] * x[64c+16g+s]; chunk partials added in
// chunk order from 0.0; fl32; + bias in fp32).  Lane c owns chunk c.  The
// row's loads are issued first (dec_row_issue) so that they stream while the
// WG normalizes x (mi_moe_forward_norm); x then comes from the staged normed
// row sxn in LDS (chunk c's float4 q at slot ax_slot(c, q): 16 lanes reading
// chunks c .. c + 15 hit 16 different slots), else from global memory.
__device__ inline int ax_slot(int c, int q) { return 16 * c + ((q + c) & 15); }
__device__ inline void dec_row_issue(const DecArgs &g, int e, int lane, float4_t (&w)[16]) {
    const int D = g.D;
    if (64 * lane + 64 <= D) {
        const float *wr = g.rw + (int64_t)e * D + 64 * lane;
#pragma unroll
        for (int q = 0; q < 16; ++q) w[q] = *(const float4_t *)(wr + 4 * q);
    } else {
#pragma unroll
        for (int q = 0; q < 16; ++q) w[q] = float4_t{0.f, 0.f, 0.f, 0.f};
    }
}
__device__ inline float dec_row_finish(const DecArgs &g, int e, int lane, const float4_t (&w)[16],
                                       const float4_t *sxn) {
    const int D = g.D;
    const int nch = D >> 6;   // D is a multiple of 256
    double part = 0.0;
    if (lane < nch) {
        float xv[64], wv[64];
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const float4_t a = sxn ? sxn[ax_slot(lane, q)] : *(const float4_t *)(g.x + 64 * lane + 4 * q);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                xv[4 * q + j] = a[j];
                wv[4 * q + j] = w[q][j];
            }
        }
#pragma unroll
        for (int s = 0; s < 16; ++s)
#pragma unroll
            for (int q = 0; q < 4; ++q) part = fma((double)wv[16 * q + s], (double)xv[16 * q + s], part);
    }
    // chunk partials added left to right (lane reads, no LDS round trips)
    const uint64_t pb = __builtin_bit_cast(uint64_t, part);
    const uint32_t plo = (uint32_t)pb, phi = (uint32_t)(pb >> 32);
    double acc = 0.0;
    for (int c = 0; c < nch; ++c) {
        const uint64_t v = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)phi, c) << 32) |
                           (uint32_t)__builtin_amdgcn_readlane((int)plo, c);
        acc = acc + __builtin_bit_cast(double, v);
    }
    float v = (float)acc;
    if (g.rb) v = v + g.rb[e];
    return v;
}

// Q8_K of x block b (natural order, ggml block_q8_K fields split), written
// through for the other WGs; x from the staged normed row when there is one
__device__ inline void dec_q8k_x(const DecArgs &g, int b, int lane, const float4_t *sxn) {
    const float4_t xv = sxn ? sxn[ax_slot(4 * b + (lane >> 4), lane & 15)] : *(const float4_t *)(g.x + b * QK + 4 * lane);
    const float v[4] = {xv[0], xv[1], xv[2], xv[3]};
    int q[4];
    const float d = q8k_wave(v, lane, q);
    st_dev4(g.xq, b * QK + 4 * lane, pack_i8x4(q));
    if (lane == 0) st_dev4(g.xd, 4u * b, __builtin_bit_cast(uint32_t, d));
    // block sums 2j and 2j+1 (lanes 8j and 8j+4) as one 32-bit word
    const int s = q8k_bsum16(q);
    const int s_hi = __shfl_down(s, 4, 64);
    if ((lane & 7) == 0)
        st_dev4(g.xbs, 2u * (b * 16 + (lane >> 2)),
                (uint32_t)(uint16_t)(int16_t)s | ((uint32_t)(uint16_t)(int16_t)s_hi << 16));
}

// Sum of the NORM_T partials held by threads T0 .. T0 + NORM_T - 1 of the WG
// (v of the others is ignored), paired as k_norm_rows pairs them: red[t] +=
// red[t + o] for o = NORM_T / 2 .. 1 (two levels through LDS, the rest by lane
// shifts in one wave; fp64 addition is commutative, so the bits agree).
// Every thread gets the sum; LDS-only barriers (loads in flight stay so).
template <int T0>
__device__ inline double dec_sum_norm(double v, double *red, double *s_sum) {
    const int t = (int)threadIdx.x - T0;
    if (t >= 0 && t < NORM_T) red[t] = v;
    dec_lds_barrier();
    if (t >= 0 && t < NORM_T / 2) red[t] = red[t] + red[t + NORM_T / 2];
    dec_lds_barrier();
    if (t >= 0 && t < NORM_T / 4) {
        double r = red[t] + red[t + NORM_T / 4];   // one wave: lanes t < 64
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const uint64_t rb = __builtin_bit_cast(uint64_t, r);
            const uint64_t nb = ((uint64_t)(uint32_t)__shfl_down((int)(rb >> 32), o, 64) << 32) |
                                (uint32_t)__shfl_down((int)(uint32_t)rb, o, 64);
            r = r + __builtin_bit_cast(double, nb);
        }
        if (t == 0) *s_sum = r;
    }
    dec_lds_barrier();
    return *s_sum;
}

// The norm of x (mi_moe_forward_norm) inside the kernel: threads DEC_NORM_T0
// .. + NORM_T - 1 load x, compute the statistics in k_norm_rows' order and
// stage the normed row (norm_apply: the same roundings) into sxn; every
// thread of the WG takes part in the barriers.  Bit for bit the row mi_norm
// writes.
constexpr int DEC_NORM_T0 = 256;   // waves 4-7: wave 0 has its router row loads in flight
__device__ inline void dec_norm_stage(const DecArgs &g, float4_t *sxn, double *red, double *s_sum) {
    const NormParams &p = g.norm;
    const int D = g.D, t = (int)threadIdx.x - DEC_NORM_T0;
    const bool on = t >= 0 && t < NORM_T;
    float v[NORM_PIECES][4];
#pragma unroll
    for (int k = 0; k < NORM_PIECES; ++k) {
        const int i = 1024 * k + 4 * t;
        if (on && i < D) {
            const float4_t a = *(const float4_t *)(g.x + i);
#pragma unroll
            for (int j = 0; j < 4; ++j) v[k][j] = a[j];
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) v[k][j] = 0.f;
        }
    }
    float m = 0.f, sc;
    double acc = 0.0;
    if (p.kind == NORM_RMS) {
#pragma unroll
        for (int k = 0; k < NORM_PIECES; ++k)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = acc + (double)(v[k][j] * v[k][j]);
        const float ms = (float)(dec_sum_norm<DEC_NORM_T0>(acc, red, s_sum) / (double)D);
        sc = 1.0f / sqrtf(ms + p.eps);
    } else {
#pragma unroll
        for (int k = 0; k < NORM_PIECES; ++k)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = acc + (double)v[k][j];
        m = (float)(dec_sum_norm<DEC_NORM_T0>(acc, red, s_sum) / (double)D);
        double acc2 = 0.0;
#pragma unroll
        for (int k = 0; k < NORM_PIECES; ++k)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (1024 * k + 4 * t + j < D) {
                    const float d = v[k][j] - m;
                    acc2 = acc2 + (double)(d * d);
                }
        const float var = (float)(dec_sum_norm<DEC_NORM_T0>(acc2, red, s_sum) / (double)D);
        sc = 1.0f / sqrtf(var + p.eps);
    }
#pragma unroll
    for (int k = 0; k < NORM_PIECES; ++k) {
        const int i = 1024 * k + 4 * t;
        if (on && i < D) {
            float4_t o;
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = norm_apply(p, v[k][j], i + j, m, sc);
            sxn[ax_slot(i >> 6, (i & 63) >> 2)] = o;
        }
    }
    dec_lds_barrier();
}

// ---------------------------------------------------------------- dots
// One lane's 32-value piece sl of a Q4_K block held in LDS against the
// matching Q8_K activation piece in registers (ggml_vec_dot_q4_K_q8_K
// restricted to sub-blocks 2c, 2c+1, c = sl/2, values 16*(sl%2)..+16 of each).
struct Q4X {
    u32x4 xa, xb;    // activation codes of the low / high nibble halves
    int bsa, bsb;    // their 16-value block sums
    float dx;
};
// (written by other WGs: coherent loads; D values, D / 16 block sums, D / 256 scales)
__device__ inline Q4X dec_q4x_load(const int8_t *xq, const int16_t *xbs, const float *xd, int D, int b, int sl) {
    const int c = sl >> 1, l0 = 16 * (sl & 1);
    const auto rq = co_rsrc(xq, (uint32_t)D), rb = co_rsrc(xbs, (uint32_t)(D / 8)), rd = co_rsrc(xd, (uint32_t)(D / 64));
    Q4X x;
    const uint32_t blk = (uint32_t)(b * QK);
    x.xa = co_ld16(rq, blk + 64 * c + l0);
    x.xb = co_ld16(rq, blk + 64 * c + 32 + l0);
    // block sums 4c + (sl & 1) and 4c + 2 + (sl & 1): the low or high half of two dwords
    const uint32_t wa = co_ld4(rb, 2u * (uint32_t)(b * 16 + 4 * c));
    const uint32_t wb = co_ld4(rb, 2u * (uint32_t)(b * 16 + 4 * c + 2));
    const uint32_t sh = 16u * (uint32_t)(sl & 1);
    x.bsa = (int)(int16_t)(uint16_t)(wa >> sh);
    x.bsb = (int)(int16_t)(uint16_t)(wb >> sh);
    x.dx = __builtin_bit_cast(float, co_ld4(rd, 4u * (uint32_t)b));
    return x;
}
__device__ inline float dec_q4_piece(const uint8_t *blk, int sl, const Q4X &x) {
    const u32x4 h = *(const u32x4 *)blk;
    const u32x4 q = *(const u32x4 *)(blk + 16 + 16 * sl);
    const float d = h2f((uint16_t)(h[0] & 0xffff)), dmin = h2f((uint16_t)(h[0] >> 16));
    const int c = sl >> 1;
    int scA, mA, scB, mB;
    scale_min_k4_reg(2 * c, h[1], h[2], h[3], scA, mA);
    scale_min_k4_reg(2 * c + 1, h[1], h[2], h[3], scB, mB);
    int sa = 0, sb = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        sa = __builtin_amdgcn_sdot4((int)(q[i] & 0x0F0F0F0Fu), (int)x.xa[i], sa, false);
        sb = __builtin_amdgcn_sdot4((int)((q[i] >> 4) & 0x0F0F0F0Fu), (int)x.xb[i], sb, false);
    }
    const int isum = scA * sa + scB * sb;
    const int msum = mA * x.bsa + mB * x.bsb;
    return (d * x.dx) * (float)isum - (dmin * x.dx) * (float)msum;
}

// N dwords from byte offset off (2-byte aligned) of an LDS region, reading
// only the aligned dwords that intersect the range
template <int N>
__device__ inline void lds_words(const uint8_t *region, uint32_t off, uint32_t (&out)[N]) {
    const uint32_t mis = off & 3u;
    const uint32_t *w = (const uint32_t *)(region + (off & ~3u));
    uint32_t a[N + 1];
#pragma unroll
    for (int i = 0; i <= N; ++i) a[i] = w[i];
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = __builtin_amdgcn_alignbyte(a[i + 1], a[i], mis);
}

// ---------------------------------------------------------------- down rows, unpacked
// Phase C reads its slot's down rows in a dot-ready form that the wave builds
// from the raw GGUF rows while it waits for the activations: per row c the I
// weights as int8 (Q4_K: q in 0..15, Q6_K: q - 32); per (row, block b, lane
// slot j < 8) one word with the scales and mins of 16-value groups j and
// j + 8 (s_j | s_{j+8} << 8 | m_j << 16 | m_{j+8} << 24; Q4_K: the 6-bit
// scale and min of the group's sub-block, Q6_K: its int8 scale and min 0);
// per (row, block) the float pair (d, dmin) (Q6_K: dmin 0).  A block then
// contributes (d dx) sum_g s_g dot_g - (dmin dx) sum_g m_g bsum_g, the
// integer form of ggml_vec_dot_q4_K_q8_K / ggml_vec_dot_q6_K_q8_K.
// Rows are DN_PAD bytes apart beyond their I weights, so the eight rows one
// instruction touches start in different LDS banks.
constexpr int DN_PAD = 16;
struct DnLayout {
    uint32_t row, sc, dm;   // row stride; byte offsets of the scale words and (d, dmin) pairs
};
__device__ inline DnLayout dn_layout(int C, int I) {
    DnLayout L;
    L.row = (uint32_t)(I + DN_PAD);
    L.sc = (uint32_t)C * L.row;
    L.dm = L.sc + (uint32_t)(C * (I / QK) * 32);
    return L;
}

// unpack half h of block b of row c (raw row bytes at dn + c*rbd + b*BB)
__device__ inline void dn_unpack_q4(const uint8_t *dn, uint8_t *un, const DnLayout &L, int I, int NBI,
                                    uint32_t rbd, int c, int b, int h) {
    const uint8_t *raw = dn + c * rbd + b * Q4K_BYTES;     // 16-byte aligned (Q4_K rows)
    const u32x4 hdr = *(const u32x4 *)raw;
    int8_t *w = (int8_t *)un + c * L.row + b * QK;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        // qs bytes 64h + 16t .. +16 = sub-block pair jj = 2h + t/2, positions l0 = 16 (t % 2) ..
        const u32x4 qv = *(const u32x4 *)(raw + 16 + 64 * h + 16 * t);
        const int jj = 2 * h + (t >> 1), l0 = 16 * (t & 1);
        u32x4 lo, hi;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            lo[e] = qv[e] & 0x0F0F0F0Fu;
            hi[e] = (qv[e] >> 4) & 0x0F0F0F0Fu;
        }
        *(u32x4 *)(w + 64 * jj + l0) = lo;        // values 64 jj + l0 ..
        *(u32x4 *)(w + 64 * jj + 32 + l0) = hi;   // values 64 jj + 32 + l0 ..
    }
    // scale words 4h .. 4h + 3: groups j and j + 8 lie in sub-blocks j/2 and j/2 + 4
    uint32_t *sw = (uint32_t *)(un + L.sc) + (c * NBI + b) * 8 + 4 * h;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        int sa, ma, sb, mb;
        scale_min_k4_reg(2 * h + i, hdr[1], hdr[2], hdr[3], sa, ma);
        scale_min_k4_reg(2 * h + i + 4, hdr[1], hdr[2], hdr[3], sb, mb);
        const uint32_t word = (uint32_t)sa | ((uint32_t)sb << 8) | ((uint32_t)ma << 16) | ((uint32_t)mb << 24);
        sw[2 * i] = word;
        sw[2 * i + 1] = word;
    }
    if (h == 0) {
        float *dm = (float *)(un + L.dm) + 2 * (c * NBI + b);
        dm[0] = h2f((uint16_t)(hdr[0] & 0xffff));
        dm[1] = h2f((uint16_t)(hdr[0] >> 16));
    }
}

__device__ inline void dn_unpack_q6(const uint8_t *dn, uint8_t *un, const DnLayout &L, int I, int NBI,
                                    uint32_t boff, int c, int b, int h) {
    // block at byte boff of the raw region (2-byte aligned)
    uint32_t ql[16], qh[8];
    lds_words<16>(dn, boff + 64 * h, ql);        // ql[64h .. 64h + 64)
    lds_words<8>(dn, boff + 128 + 32 * h, qh);   // qh[32h .. 32h + 32)
    int8_t *w = (int8_t *)un + c * L.row + b * QK + 128 * h;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
        // values 32 qq + l, l < 32: low / high nibble of ql[l] or ql[l + 32]
        // and bits 2 qq .. 2 qq + 1 of qh[l] (ggml dequantize_row_q6_K)
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            u32x4 out;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int wi = 4 * half + e;   // word of l = 4 wi .. 4 wi + 3
                const uint32_t lw = (qq & 1) ? ql[8 + wi] : ql[wi];
                const uint32_t lo = (qq >> 1) ? ((lw >> 4) & 0x0F0F0F0Fu) : (lw & 0x0F0F0F0Fu);
                const uint32_t hi2 = ((qh[wi] >> (2 * qq)) << 4) & 0x30303030u;
                // 6-bit q -> q - 32 as a signed byte: q ^ 0x20 is its 6-bit two's
                // complement; copy bit 5 into bits 6-7 (0x20 * 6 = 0xC0, no carries)
                const uint32_t x6 = (lo | hi2) ^ 0x20202020u;
                out[e] = x6 | ((x6 & 0x20202020u) * 6u);
            }
            *(u32x4 *)(w + 32 * qq + 16 * half) = out;
        }
    }
    // scale words 4h .. 4h + 3: int8 scales of groups j and j + 8
    uint32_t scw[4];
    lds_words<4>(dn, boff + 192, scw);
    uint32_t *sw = (uint32_t *)(un + L.sc) + (c * NBI + b) * 8 + 4 * h;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t s0 = (scw[h] >> (8 * i)) & 0xffu;
        const uint32_t s1 = (scw[h + 2] >> (8 * i)) & 0xffu;
        sw[i] = s0 | (s1 << 8);
    }
    if (h == 0) {
        uint32_t dw[1];
        lds_words<1>(dn, boff + 208, dw);
        float *dm = (float *)(un + L.dm) + 2 * (c * NBI + b);
        dm[0] = h2f((uint16_t)(dw[0] & 0xffff));
        dm[1] = 0.f;
    }
}

// copy a byte range of one expert matrix into LDS: DEC segments of 1 KB, lane
// l moving 16 bytes.  The resource covers exactly the 16-aligned span of the
// range, so segments past it read zeros without touching memory and the
// number of DMA instructions per wave is a compile-time constant.
template <int NSEG>
__device__ inline void dec_dma(const uint8_t *base16, uint32_t span, uint8_t *lds, int lane) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base16), (short)0, (int)span, 0x00020000);
#pragma unroll
    for (int s = 0; s < NSEG; ++s)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t *)(lds + 1024 * s), 16, 1024 * s + 16 * lane, 0, 0,
                                                 0);
}

// rows [row0, row0 + nrows) of expert e of m: 16-aligned base, byte shift of
// the first row, span in bytes (multiple of 16)
struct DecChunk {
    const uint8_t *base16;
    uint32_t shift, span;
};
__device__ inline DecChunk dec_chunk(const ExpertMat &m, int e, int64_t row0, int nrows, bool on) {
    DecChunk c;
    const uint8_t *p = m.data + (int64_t)e * m.mat_bytes + row0 * m.row_bytes;
    const uintptr_t a = (uintptr_t)p;
    c.base16 = (const uint8_t *)(a & ~(uintptr_t)15);
    c.shift = (uint32_t)(a & 15);
    const uint32_t len = on ? (uint32_t)(nrows * m.row_bytes) : 0u;
    c.span = on ? (c.shift + len + 15u) & ~15u : 0u;
    return c;
}

// ---------------------------------------------------------------- kernel
constexpr int DEC_RSTEPS = 16;   // row steps per wave in the gate/up phase (R / RPS)

// NBI = I / 256: blocks per down row (compile time, so the per-slot Q8_K and
// the down reductions unroll)
template <int DT, int NBI>
__global__ void __launch_bounds__(DEC_THREADS) k_decode1(DecArgs g) {
    __shared__ __attribute__((aligned(1024))) uint8_t s_gu[DEC_WAVES][DEC_WREG];
    __shared__ __attribute__((aligned(1024))) uint8_t s_dn[DEC_KMAX][DEC_DN_SEG * 1024];
    __shared__ float s_logit[256];
    __shared__ int s_sel[DEC_KMAX];
    __shared__ float s_val[DEC_KMAX], s_w[DEC_KMAX];
    __shared__ float s_hg[2 * DEC_PMAX];
    __shared__ float s_z[DEC_KMAX * DEC_CMAX];
    __shared__ int s_list[DEC_MAX_GRID];   // units still missing after a poll
    __shared__ int s_fail, s_nmiss, s_wmiss[DEC_WAVES];
    __shared__ double s_red[NORM_T], s_nsum;   // norm of x

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wg = blockIdx.x, G = gridDim.x;
    const int D = g.D, E = g.E, K = g.K, I = g.I;
    const int NB = D / QK;
    // this launch's epoch (see the header comment)
    const uint32_t tag = __hip_atomic_load(g.epoch + wg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    bool ok = true;
    if (tid == 0) s_fail = 0;
    // residual of this WG's output columns, loaded now (off the kernel's tail)
    const int C = g.C, n0 = wg * C;
    const bool do_c = n0 < D;
    const float resv = (do_c && tid < C && g.res) ? g.res[n0 + tid] : 0.f;

    // ---- A: router row wg (wave 0) and Q8_K of x block wg (wave 1); the
    // logit is published only once this WG's Q8_K of x is out.  With a norm of
    // x, every WG first normalizes x into LDS (s_dn: phase B parks down rows
    // there later) while wave 0's row loads stream.
    float4_t wrow[16];
    if (wave == 0 && wg < E) dec_row_issue(g, wg, lane, wrow);
    const float4_t *sxn = nullptr;
    if (g.norm.kind != NORM_NONE) {
        dec_norm_stage(g, (float4_t *)&s_dn[0][0], s_red, &s_nsum);
        sxn = (const float4_t *)&s_dn[0][0];
    }
    float logit = 0.f;
    if (wave == 0 && wg < E) logit = dec_row_finish(g, wg, lane, wrow, sxn);
    else if (wave == 1 && wg < NB) dec_q8k_x(g, wg, lane, sxn);
    vm_drain();
    dec_lds_barrier();
    if (wave == 0 && lane == 0 && wg < E) tw_store(g.tw + DEC_TW_LOGIT + wg, tag, __builtin_bit_cast(uint32_t, logit));

    // ---- every logit (and so every Q8_K block of x); an A unit still missing
    // after g.rescue_polls tries is computed here and stored again (same bits):
    // no WG waits on a WG that is not running
    unsigned spins = 0;
    for (;;) {
        bool have = true;
        if (tid < E) {
            uint32_t v;
            have = tw_wait1(g.tw + DEC_TW_LOGIT + tid, tag, g.rescue_polls, v);
            if (have) s_logit[tid] = as_float(v);
        }
        if (dec_none_missing(s_wmiss, !have)) break;
        const int nmiss = dec_missing(&s_nmiss, s_list, tid, -1, !have, false);
        spins += g.rescue_polls + 1;
        if (spins > DEC_SPIN_LIMIT) {
            ok = false;
            break;
        }
        for (int m = wave; m < nmiss; m += DEC_WAVES) {
            const int a = __builtin_amdgcn_readfirstlane(s_list[m]);
            if (a < NB) dec_q8k_x(g, a, lane, sxn);
            float4_t wr[16];
            dec_row_issue(g, a, lane, wr);
            const float lv = dec_row_finish(g, a, lane, wr, sxn);
            vm_drain();   // the x block is out before the logit
            if (lane == 0) tw_store(g.tw + DEC_TW_LOGIT + a, tag, __builtin_bit_cast(uint32_t, lv));
        }
    }

    // ---- B: routing (every WG), DMA of its gate/up and down rows
    if (tid < DEC_KMAX) s_sel[tid] = tid < K ? tid : 0;
    dec_lds_barrier();
    // this lane's activation piece: row group of LPR = 8*NB lanes, block bq,
    // piece sl (every logit is in, so the Q8_K of x is too)
    const int LPR = 8 * NB, RPS = 64 / LPR;
    const int rr = lane / LPR, bq = (lane % LPR) >> 3, sl = lane & 7;
    const Q4X xg = dec_q4x_load(g.xq, g.xbs, g.xd, D, bq, sl);
    {
        // rank of expert e = #{i : l_i > l_e} + #{i < e : l_i == l_e}; the K
        // lowest ranks in rank order are ggml_top_k's stable descending pick.
        // 8, 4 or 2 lanes per expert (E <= 64, 128, 256), each comparing a
        // share of the logits
        const int tpe = E <= DEC_THREADS / 8 ? 8 : E <= DEC_THREADS / 4 ? 4 : 2;
        const int e = tid / tpe, j = tid % tpe;
        int cnt = 0;
        float ve = 0.f;
        if (e < E) {
            ve = s_logit[e];
#pragma unroll 8
            for (int i = j; i < E; i += tpe) {
                const float vi = s_logit[i];
                cnt += (int)(vi > ve) | ((int)(vi == ve) & (int)(i < e));
            }
        }
        cnt += dpp_i<0xB1>(cnt);
        if (tpe >= 4) cnt += dpp_i<0x4E>(cnt);
        if (tpe >= 8) cnt += dpp_i<0x141>(cnt);
        if (e < E && j == 0 && cnt < K) {
            s_sel[cnt] = e;
            s_val[cnt] = ve;
        }
    }
    dec_lds_barrier();

    const int64_t pairs = (int64_t)K * I;
    const int P = g.P, R = P / 4;
    const int UB = (int)(pairs / P);          // gate/up units of P (h, g) row pairs
    const int64_t q0 = (int64_t)wg * P;
    const bool do_b = q0 < pairs;
    uint32_t dn_shift = 0;
    // DMA of unit u's gate/up rows into s_gu (wave v: rows v % 4 of the h
    // (v < 4) or g half)
    auto b_issue = [&](int u, bool on) {
        const int64_t q = (int64_t)u * P;
        const int kb = on ? (int)(q / I) : 0, ib = on ? (int)(q % I) : 0;
        int eb = __builtin_amdgcn_readfirstlane(s_sel[kb]);
        eb = eb < 0 ? 0 : (eb >= E ? E - 1 : eb);
        const bool hpart = wave < 4;
        const ExpertMat &m = (hpart || g.fused) ? g.gate : g.up;
        const int64_t row0 = (int64_t)ib + (wave & 3) * R + ((!hpart && g.fused) ? I : 0);
        const DecChunk c = dec_chunk(m, eb, row0, R, on);
        dec_dma<DEC_GU_SEG>(c.base16, c.span, s_gu[wave], lane);
    };
    // gate/up dots of the unit in s_gu: wave v owns R consecutive rows (h for
    // v < 4, g for v >= 4); every row's piece first, then the lane-group sums
    // of all rows together (independent exchanges overlap instead of queueing
    // one row at a time)
    auto b_dots = [&]() {
        const int64_t rb = (int64_t)NB * Q4K_BYTES;   // Q4_K tables are 16-byte aligned: no shift
        float acc[DEC_RSTEPS];
#pragma unroll
        for (int j = 0; j < DEC_RSTEPS; ++j) {
            acc[j] = 0.f;
            const int r = j * RPS + rr;
            if (j * RPS < R && r < R) acc[j] = dec_q4_piece(s_gu[wave] + r * rb + bq * Q4K_BYTES, sl, xg);
        }
#pragma unroll
        for (int j = 0; j < DEC_RSTEPS; ++j) acc[j] += dpp_f<0xB1>(acc[j]);
#pragma unroll
        for (int j = 0; j < DEC_RSTEPS; ++j) acc[j] += dpp_f<0x4E>(acc[j]);
#pragma unroll
        for (int j = 0; j < DEC_RSTEPS; ++j) acc[j] += dpp_f<0x141>(acc[j]);
        if (LPR >= 16) {
#pragma unroll
            for (int j = 0; j < DEC_RSTEPS; ++j) acc[j] += dpp_f<0x140>(acc[j]);
        }
        if (LPR >= 32) {
#pragma unroll
            for (int j = 0; j < DEC_RSTEPS; ++j) acc[j] += __shfl_xor(acc[j], 16, 64);
        }
        if (LPR >= 64) {
#pragma unroll
            for (int j = 0; j < DEC_RSTEPS; ++j) acc[j] += __shfl_xor(acc[j], 32, 64);
        }
#pragma unroll
        for (int j = 0; j < DEC_RSTEPS; ++j) {
            const int r = j * RPS + rr;
            if (j * RPS < R && r < R && (lane % LPR) == 0) s_hg[(wave >> 2) * P + (wave & 3) * R + r] = acc[j];
        }
    };
    // GLU of the unit (after an LDS barrier), activations written through,
    // then the unit's completion word once wave 0's stores are out (P <= 64:
    // every store comes from wave 0)
    auto b_publish = [&](int u, bool owner) {
        const int64_t q = (int64_t)u * P;
        if (tid < P)
            st_dev4(g.actf, 4u * (uint32_t)(q + tid), __builtin_bit_cast(uint32_t, act_pair(g.act, s_hg[tid], s_hg[P + tid])));
        if (wave == 0) {
            vm_drain();
            if (lane == 0) tw_store(g.tw + DEC_TW_BDONE + u, tag, 1u);
        }
    };
    b_issue(wg, do_b);
    // down rows of slot k = wave: prefetched into registers now (the stream
    // overlaps the gate/up arithmetic), parked in LDS after it
    u32x4 dnv[DEC_DN_SEG];
    {
        const int k = wave < K ? wave : 0;
        int ed = __builtin_amdgcn_readfirstlane(s_sel[k]);
        ed = ed < 0 ? 0 : (ed >= E ? E - 1 : ed);
        const DecChunk c = dec_chunk(g.down, ed, n0, C, do_c && wave < K);
        dn_shift = c.shift;
        const __amdgpu_buffer_rsrc_t r =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(c.base16), (short)0, (int)c.span, 0x00020000);
#pragma unroll
        for (int s = 0; s < DEC_DN_SEG; ++s) dnv[s] = __builtin_amdgcn_raw_buffer_load_b128(r, 1024 * s + 16 * lane, 0, 0);
    }

    if (wave == 0) {
        const float myval = lane < K ? s_val[lane] : 0.f;
        const float myw = softmax_selected_wave(myval, K, lane);
        if (lane < K) s_w[lane] = myw;
        if (wg == 0 && lane < K) {
            g.sel[lane] = s_sel[lane];
            g.w[lane] = myw;
        }
    }
    if (wg == 0) {
        if (tid < E) g.logits[tid] = s_logit[tid];
        // single-token dispatch: one list entry per selected expert
        for (int e = tid; e < E; e += DEC_THREADS) {
            int cnt = 0, below = 0, slot = 0;
            for (int k = 0; k < K; ++k) {
                if (s_sel[k] == e) {
                    cnt++;
                    slot = k;
                }
                below += s_sel[k] < e;
            }
            g.counts[e] = cnt;
            g.offsets[e] = below;
            if (cnt) g.perm[below] = slot;
        }
        if (tid == 0) g.offsets[E] = K;
    }

    if (do_b) b_dots();
#pragma unroll
    for (int s = 0; s < DEC_DN_SEG; ++s) *(u32x4 *)(s_dn[wave] + 1024 * s + 16 * lane) = dnv[s];
    dec_lds_barrier();
    if (do_b) b_publish(wg, true);

    // while the other WGs finish: turn this wave's slot of down rows into the
    // dot-ready form (raw rows in s_dn[wave], result in s_gu[wave])
    const DnLayout UL = dn_layout(C, I);
    auto unpack = [&]() {
        if (do_c && wave < K) {
            const uint32_t rbd = (uint32_t)g.down.row_bytes;
            for (int u = lane; u < C * NBI * 2; u += 64) {
                const int c = u / (2 * NBI), rem = u % (2 * NBI), b = rem >> 1, h = rem & 1;
                if constexpr (DT == 12) dn_unpack_q4(s_dn[wave] + dn_shift, s_gu[wave], UL, I, NBI, rbd, c, b, h);
                else dn_unpack_q6(s_dn[wave], s_gu[wave], UL, I, NBI, dn_shift + c * rbd + b * Q6K_BYTES, c, b, h);
            }
        }
    };

    unpack();
    // ---- every gate/up unit: each thread polls one or two units' completion
    // words (no counters: the word lands right after the unit's activations,
    // measured 0.5 us per call faster than a two-level counter and release
    // word); a unit still missing after g.rescue_polls tries is computed here
    // (its rows pass through s_gu, so this WG's down rows are unpacked again
    // afterwards)
    for (;;) {
        const int u0 = tid, u1 = tid + DEC_THREADS;
        uint32_t v;
        const bool miss0 = u0 < UB && !tw_wait1(g.tw + DEC_TW_BDONE + u0, tag, g.rescue_polls, v);
        const bool miss1 = u1 < UB && !tw_wait1(g.tw + DEC_TW_BDONE + u1, tag, g.rescue_polls, v);
        if (dec_none_missing(s_wmiss, miss0 || miss1)) break;
        const int nmiss = dec_missing(&s_nmiss, s_list, u0, u1, miss0, miss1);
        spins += g.rescue_polls + 1;
        if (spins > DEC_SPIN_LIMIT) {
            ok = false;
            break;
        }
        for (int m = 0; m < nmiss; ++m) {
            const int u = __builtin_amdgcn_readfirstlane(s_list[m]);
            dec_lds_barrier();   // s_gu / s_hg readers of the previous unit are done
            b_issue(u, true);
            b_dots();
            dec_lds_barrier();
            b_publish(u, false);
        }
        dec_lds_barrier();
        unpack();
    }
    // the activations of slot k = wave (written by other WGs: coherent
    // loads), 16 lanes per 256-block, four blocks per pass
    constexpr int NPASS = (NBI + 3) / 4;
    float av[NPASS][16];
    if (do_c && wave < K) {
        const auto ra = co_rsrc(g.actf, (uint32_t)(4 * K * I));
        const int seg = lane & 15;
#pragma unroll
        for (int pp = 0; pp < NPASS; ++pp) {
            const int b = 4 * pp + (lane >> 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                u32x4 a4 = {0u, 0u, 0u, 0u};
                if (b < NBI) a4 = co_ld16(ra, 4u * (uint32_t)(wave * I + b * QK + 16 * seg + 4 * i));
#pragma unroll
                for (int e = 0; e < 4; ++e) av[pp][4 * i + e] = as_float(a4[e]);
            }
        }
    }

    // ---- C: Q8_K of slot k = wave's activations, down rows, weighted combine
    if (do_c && wave < K) {
        const int k = wave;
        // Q8_K of the I activations of slot k (ggml quantizes each mul_mat_id
        // source row on its own): codes / scales / block sums into s_dn[k],
        // whose raw rows are unpacked already
        int8_t *aq = (int8_t *)s_dn[k];
        float *ad = (float *)(s_dn[k] + 2048);
        int16_t *abs_ = (int16_t *)(s_dn[k] + 2048 + 64);
        // 16 lanes per block, four blocks per pass, from the polled values
#pragma unroll
        for (int pp = 0; pp < NPASS; ++pp) {
            const int b = 4 * pp + (lane >> 4), seg = lane & 15;
            int q[16], bsum;
            const float d = q8k_wave4x16(av[pp], lane, q, bsum);
            if (b < NBI) {
                u32x4 pk;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int qi[4] = {q[4 * i], q[4 * i + 1], q[4 * i + 2], q[4 * i + 3]};
                    pk[i] = pack_i8x4(qi);
                }
                *(u32x4 *)(aq + b * QK + 16 * seg) = pk;
                abs_[b * 16 + seg] = (int16_t)bsum;
                if (seg == 0) ad[b] = d;
            }
        }
        // lane (row c = c0 + lane / 8, j = lane % 8): groups j and j + 8 of every block
        const int j = lane & 7, rsub = lane >> 3;
        u32x4 x0[NBI], x1[NBI];
        int bs0[NBI], bs1[NBI];
        float dx[NBI];
#pragma unroll
        for (int b = 0; b < NBI; ++b) {
            x0[b] = *(const u32x4 *)(aq + b * QK + 16 * j);
            x1[b] = *(const u32x4 *)(aq + b * QK + 128 + 16 * j);
            bs0[b] = abs_[b * 16 + j];
            bs1[b] = abs_[b * 16 + 8 + j];
            dx[b] = ad[b];
        }
        const uint8_t *un = s_gu[k];
        for (int c0 = 0; c0 < C; c0 += 8) {
            const int c = c0 + rsub;
            float acc = 0.f;
            if (c < C) {
#pragma unroll
                for (int b = 0; b < NBI; ++b) {
                    const int8_t *wr = (const int8_t *)un + c * UL.row + b * QK;
                    const u32x4 w0 = *(const u32x4 *)(wr + 16 * j);
                    const u32x4 w1 = *(const u32x4 *)(wr + 128 + 16 * j);
                    const uint32_t sw = *((const uint32_t *)(un + UL.sc) + (c * NBI + b) * 8 + j);
                    const float2 dm = *((const float2 *)(un + UL.dm) + (c * NBI + b));
                    int d0 = 0, d1 = 0;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        d0 = __builtin_amdgcn_sdot4((int)w0[i], (int)x0[b][i], d0, false);
                        d1 = __builtin_amdgcn_sdot4((int)w1[i], (int)x1[b][i], d1, false);
                    }
                    const int s0 = (int)(int8_t)(sw & 0xff), s1 = (int)(int8_t)((sw >> 8) & 0xff);
                    const int m0 = (int)((sw >> 16) & 0xff), m1 = (int)(sw >> 24);
                    const int isum = s0 * d0 + s1 * d1;
                    const int msum = m0 * bs0[b] + m1 * bs1[b];
                    acc += (dm.x * dx[b]) * (float)isum - (dm.y * dx[b]) * (float)msum;
                }
            }
            acc += dpp_f<0xB1>(acc);
            acc += dpp_f<0x4E>(acc);
            acc += dpp_f<0x141>(acc);
            if (c < C && j == 0) s_z[k * C + c] = acc;
        }
    }
    if (!ok) s_fail = 1;
    dec_lds_barrier();
    const bool failed = s_fail != 0;
    if (do_c && tid < C) {
        double s = 0.0;
        for (int k = 0; k < K; ++k) s = s + (double)(s_z[k * C + tid] * s_w[k]);
        const float moe = (float)s;
        float v = g.res ? resv + moe : moe;
        if (failed) v = __builtin_nanf("");
        g.out[n0 + tid] = v;
    }
    if (tid == 0) {
        if (failed) __hip_atomic_fetch_add(g.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(g.epoch + wg, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ================================================================ batched decode
// k_decodeb: the MoE block for 2..16 tokens in one kernel (the separate-kernel
// chain pays seven launches of latency at these sizes).  Same numerics,
// hand-off rules (coherent stores and loads, epoch-tagged completion words)
// and rescue-by-recomputation as k_decode1; units belong to waves (global
// wave w of W runs units w, w + W, ...) except the C units, which belong to
// work-groups:
//
//   A  units u < E T: router row u % E for token u / E (the logit travels in
//      the completion word); units E T + t NB + b: Q8_K of x block b of token
//      t.
//   -- every WG: all A words; x's Q8_K staged in LDS; each token ranked by
//      one wave (the shared top-k / softmax code); the distinct selected
//      experts listed in first-use order of the flat (t, k) pairs --
//   B  units (d, q): gate/up rows 4 q .. 4 q + 3 (h and g) of distinct expert
//      d, dotted against every pair (t, k) that selected d; GLU; fp32
//      activations of those pairs written through.  The next unit's weight
//      bytes are loaded while the current unit computes.
//   -- per C unit: the B words of its token's K experts --
//   C  units (t, 64 columns), one WG each: Q8_K of the token's K activation
//      rows (wave k), then wave w dots columns 8 w .. 8 w + 7 of every slot's
//      down rows (the next slot's rows load during the current slot's dots)
//      and combines the slots in fp64 slot order with the residual.
//
// Word layout in tw2: A words [0, E T + T NB), B words from there, QB = I / 4
// per distinct expert.
constexpr int DECB_WAVES = 8;
constexpr int DECB_THREADS = DECB_WAVES * 64;
constexpr int DECB_NB_MAX = 8;     // D <= 2048
constexpr int DECB_NBI_MAX = 4;    // I <= 1024 (one Q8_K pass per activation row)
constexpr int DECB_COLS = 64;      // output columns per C unit (at most)
constexpr int DECB_PAIRS_MAX = DECB_T_MAX;   // pairs per distinct expert: a token picks an expert once

__device__ inline float decb_router_row(const float *rw, const float *rb, const float *x, int D, int e, int lane) {
    const int nch = (D + 63) >> 6;
    double part = 0.0;
    if (lane < nch) {
        const float *xr = x + 64 * lane;
        const float *wr = rw + (int64_t)e * D + 64 * lane;
        float xv[64], wv[64];
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const float4_t a = *(const float4_t *)(xr + 4 * q);
            const float4_t b = *(const float4_t *)(wr + 4 * q);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                xv[4 * q + j] = a[j];
                wv[4 * q + j] = b[j];
            }
        }
#pragma unroll
        for (int s = 0; s < 16; ++s)
#pragma unroll
            for (int q = 0; q < 4; ++q) part = fma((double)wv[16 * q + s], (double)xv[16 * q + s], part);
    }
    const uint64_t pb = __builtin_bit_cast(uint64_t, part);
    const uint32_t plo = (uint32_t)pb, phi = (uint32_t)(pb >> 32);
    double acc = 0.0;
    for (int c = 0; c < nch; ++c) {
        const uint64_t v = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)phi, c) << 32) |
                           (uint32_t)__builtin_amdgcn_readlane((int)plo, c);
        acc = acc + __builtin_bit_cast(double, v);
    }
    float v = (float)acc;
    if (rb) v = v + rb[e];
    return v;
}

// Q8_K of x block b of token t (natural order; codes, scale, block sums),
// written through
__device__ inline void decb_q8k_x(const DecArgs &g, int t, int b, int lane) {
    const int D = g.D, NB = D / QK;
    const float4_t xv = *(const float4_t *)(g.x + (int64_t)t * D + b * QK + 4 * lane);
    const float v[4] = {xv[0], xv[1], xv[2], xv[3]};
    int q[4];
    const float d = q8k_wave(v, lane, q);
    st_dev4(g.xq, (uint32_t)(t * D + b * QK + 4 * lane), pack_i8x4(q));
    if (lane == 0) st_dev4(g.xd, 4u * (uint32_t)(t * NB + b), __builtin_bit_cast(uint32_t, d));
    const int s = q8k_bsum16(q);
    const int s_hi = __shfl_down(s, 4, 64);
    if ((lane & 7) == 0)
        st_dev4(g.xbs, 2u * (uint32_t)(t * (D / 16) + b * 16 + (lane >> 2)),
                (uint32_t)(uint16_t)(int16_t)s | ((uint32_t)(uint16_t)(int16_t)s_hi << 16));
}

// A unit u (see above); the wave publishes it
__device__ inline void decb_unit_a(const DecArgs &g, uint32_t tag, int u, int lane) {
    const int E = g.E, T = g.T, NB = g.D / QK;
    if (u < E * T) {
        const int t = u / E, e = u - t * E;
        const float lv = decb_router_row(g.rw, g.rb, g.x + (int64_t)t * g.D, g.D, e, lane);
        if (lane == 0) tw_store(g.tw2 + u, tag, __builtin_bit_cast(uint32_t, lv));
    } else {
        const int v = u - E * T, t = v / NB, b = v - t * NB;
        decb_q8k_x(g, t, b, lane);
        vm_drain();   // the block is out before its word
        if (lane == 0) tw_store(g.tw2 + u, tag, 1u);
    }
}

// one B unit's weight bytes for the lane: NB blocks x (header, 16 qs bytes)
struct DecBW {
    u32x4 h[DECB_NB_MAX], q[DECB_NB_MAX];
};

template <int NB>
__device__ inline void decb_b_load(const DecArgs &g, int e, int q, int lane, DecBW &w) {
    const int rs = lane >> 3, sl = lane & 7;
    const int64_t row = 4 * (int64_t)q + (rs & 3);
    const bool hpart = rs < 4;
    const ExpertMat &m = (hpart || g.fused) ? g.gate : g.up;
    const int64_t wrow = row + ((!hpart && g.fused) ? g.I : 0);
    const uint8_t *rowp = m.data + (int64_t)e * m.mat_bytes + wrow * m.row_bytes;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        w.h[b] = *(const u32x4 *)(rowp + b * Q4K_BYTES);
        w.q[b] = *(const u32x4 *)(rowp + b * Q4K_BYTES + 16 + 16 * sl);
    }
}

// lane piece sl of a Q4_K block (header h, qs bytes qv) against x's Q8_K
// block in LDS (codes xq, block sums xbs, scale dx): ggml_vec_dot_q4_K_q8_K
// restricted to the lane's 32 values
__device__ inline float decb_q4_dot(const u32x4 &h, const u32x4 &qv, int sl, const int8_t *xq, const int16_t *xbs,
                                    float dx) {
    const float d = h2f((uint16_t)(h[0] & 0xffff)), dmin = h2f((uint16_t)(h[0] >> 16));
    const int c = sl >> 1, l0 = 16 * (sl & 1);
    int scA, mA, scB, mB;
    scale_min_k4_reg(2 * c, h[1], h[2], h[3], scA, mA);
    scale_min_k4_reg(2 * c + 1, h[1], h[2], h[3], scB, mB);
    const u32x4 xa = *(const u32x4 *)(xq + 64 * c + l0);
    const u32x4 xb = *(const u32x4 *)(xq + 64 * c + 32 + l0);
    int sa = 0, sb = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        sa = __builtin_amdgcn_sdot4((int)(qv[i] & 0x0F0F0F0Fu), (int)xa[i], sa, false);
        sb = __builtin_amdgcn_sdot4((int)((qv[i] >> 4) & 0x0F0F0F0Fu), (int)xb[i], sb, false);
    }
    const int bsa = xbs[4 * c + (sl & 1)], bsb = xbs[4 * c + 2 + (sl & 1)];
    return (d * dx) * (float)(scA * sa + scB * sb) - (dmin * dx) * (float)(mA * bsa + mB * bsb);
}

// 8-lane sum (lanes 8 r .. 8 r + 7), in every lane of the group
__device__ inline float decb_sum8(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    return v;
}

// Q8_K of x for all T tokens, in LDS (codes [T][D], scales [T][NB], block sums [T][D/16])
struct DecBX {
    int8_t *q;
    float *d;
    int16_t *bs;
};

// B unit (d, q) from the loaded weights w: every pair of expert d
template <int NB>
__device__ inline void decb_b_compute(const DecArgs &g, const DecBX &x, const int *s_dcnt, const int *s_dpair, int d,
                                      int q, int lane, const DecBW &w) {
    const int rs = lane >> 3, sl = lane & 7, D = g.D, I = g.I;
    const int n = s_dcnt[d];
    for (int j = 0; j < n; ++j) {
        const int p = s_dpair[d * DECB_PAIRS_MAX + j], t = p / g.K;
        float acc = 0.f;
#pragma unroll
        for (int b = 0; b < NB; ++b)
            acc += decb_q4_dot(w.h[b], w.q[b], sl, x.q + t * D + b * QK, x.bs + t * (D / 16) + b * 16, x.d[t * NB + b]);
        acc = decb_sum8(acc);
        const float other = __shfl_xor(acc, 32, 64);   // the g row of the same column
        if (rs < 4 && sl == 0)
            st_dev4(g.actf, 4u * (uint32_t)((int64_t)p * I + 4 * q + rs),
                    __builtin_bit_cast(uint32_t, act_pair(g.act, acc, other)));
    }
}

// one lane's raw down-row bytes of a C pass: NBI blocks
template <int DT> struct DecBDn;
template <> struct DecBDn<12> {
    u32x4 h[DECB_NBI_MAX], q[DECB_NBI_MAX];
};
template <> struct DecBDn<14> {
    uint32_t a[DECB_NBI_MAX][3], b[DECB_NBI_MAX][3], qh[DECB_NBI_MAX][3], s[DECB_NBI_MAX][3], dw[DECB_NBI_MAX];
    uint32_t mis[DECB_NBI_MAX];
};

// the three aligned dwords holding bytes [p, p + 8) of a 2-byte-aligned address
// (the third only when p is not dword aligned: no byte past the range is read)
__device__ inline void decb_raw8(const uint8_t *p, uint32_t (&w)[3]) {
    const uint32_t *a = (const uint32_t *)((uintptr_t)p & ~(uintptr_t)3);
    w[0] = a[0];
    w[1] = a[1];
    w[2] = ((uintptr_t)p & 3u) ? a[2] : 0u;
}
__device__ inline uint2 decb_al8(const uint32_t (&w)[3], uint32_t mis) {
    uint2 r;
    r.x = __builtin_amdgcn_alignbyte(w[1], w[0], mis);
    r.y = __builtin_amdgcn_alignbyte(w[2], w[1], mis);
    return r;
}

// row `row` of expert e's down matrix, lane piece sl of each block
template <int DT, int NBI>
__device__ inline void decb_dn_load(const ExpertMat &m, int e, int64_t row, int sl, DecBDn<DT> &r) {
    const uint8_t *rowp = m.data + (int64_t)e * m.mat_bytes + row * m.row_bytes;
#pragma unroll
    for (int b = 0; b < NBI; ++b) {
        if constexpr (DT == 12) {
            r.h[b] = *(const u32x4 *)(rowp + b * Q4K_BYTES);
            r.q[b] = *(const u32x4 *)(rowp + b * Q4K_BYTES + 16 + 16 * sl);
        } else {
            const uint8_t *blk = rowp + b * Q6K_BYTES;
            const int h = sl >> 2, l0 = 8 * (sl & 3);
            r.mis[b] = (uint32_t)((uintptr_t)blk & 3u);
            decb_raw8(blk + 64 * h + l0, r.a[b]);
            decb_raw8(blk + 64 * h + 32 + l0, r.b[b]);
            decb_raw8(blk + 128 + 32 * h + l0, r.qh[b]);
            decb_raw8(blk + 192 + 8 * h, r.s[b]);
            r.dw[b] = *(const uint16_t *)(blk + 208);   // d (2-byte aligned)
        }
    }
}

// the lane's share of one down row's dot with the slot's Q8_K (LDS: codes aq,
// scales ad, block sums abs_)
template <int DT, int NBI>
__device__ inline float decb_dn_dot(const DecBDn<DT> &r, int sl, const int8_t *aq, const float *ad,
                                    const int16_t *abs_) {
    float acc = 0.f;
#pragma unroll
    for (int b = 0; b < NBI; ++b) {
        if constexpr (DT == 12) {
            acc += decb_q4_dot(r.h[b], r.q[b], sl, aq + b * QK, abs_ + b * 16, ad[b]);
        } else {
            const uint32_t mis = r.mis[b];
            Q6Piece w;
            w.qla = decb_al8(r.a[b], mis);
            w.qlb = decb_al8(r.b[b], mis);
            w.qh = decb_al8(r.qh[b], mis);
            const uint2 s8 = decb_al8(r.s[b], mis);
            const int is = (8 * (sl & 3)) >> 4;
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) {
                const int idx = is + 2 * qq;
                const uint32_t word = (idx >> 2) ? s8.y : s8.x;
                w.sc[qq] = (int)(int8_t)(word >> (8 * (idx & 3)));
            }
            w.d = h2f((uint16_t)r.dw[b]);
            acc += dot_q6_piece(w, sl, aq + b * QK, ad[b]);
        }
    }
    return acc;
}


constexpr int DECB_LIST = 1024;   // missing units listed per rescue round

template <int DT, int NB, int NBI>
__global__ void __launch_bounds__(DECB_THREADS) k_decodeb(DecArgs g) {
    __shared__ __attribute__((aligned(16))) int8_t s_xq[DECB_T_MAX * DECB_NB_MAX * QK];
    __shared__ float s_xd[DECB_T_MAX * DECB_NB_MAX];
    __shared__ int16_t s_xbs[DECB_T_MAX * DECB_NB_MAX * 16];
    __shared__ float s_logit[DECB_T_MAX * 256];
    __shared__ int s_sel[DECB_T_MAX * DEC_KMAX], s_pd[DECB_T_MAX * DEC_KMAX];
    __shared__ float s_w[DECB_T_MAX * DEC_KMAX];
    __shared__ int s_first[256], s_dist[DECB_T_MAX * DEC_KMAX], s_dcnt[DECB_T_MAX * DEC_KMAX];
    __shared__ int s_eidx[256];
    __shared__ unsigned s_tmask[256];
    __shared__ int s_dpair[DECB_T_MAX * DEC_KMAX * DECB_PAIRS_MAX];
    __shared__ __attribute__((aligned(16))) int8_t s_aq[DEC_KMAX][DECB_NBI_MAX * QK];
    __shared__ float s_ad[DEC_KMAX][DECB_NBI_MAX];
    __shared__ int16_t s_abs[DEC_KMAX][DECB_NBI_MAX * 16];
    __shared__ float s_z[DEC_KMAX][DECB_COLS];
    __shared__ int s_list[DECB_LIST];
    __shared__ int s_nd, s_nmiss, s_fail, s_wmiss[DECB_WAVES];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wg = blockIdx.x, G = gridDim.x;
    const int gw = wg * DECB_WAVES + wave, NW = G * DECB_WAVES;
    const int D = g.D, E = g.E, K = g.K, I = g.I, T = g.T;
    const int UA = E * T + T * NB;       // A units (= words)
    const int QB = I / 4;                // B units per distinct expert
    const uint32_t tag = __hip_atomic_load(g.epoch + wg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    bool ok = true;
    unsigned spins = 0;
    if (tid == 0) s_fail = 0;
    const DecBX X = {s_xq, s_xd, s_xbs};

    // B unit ub = d QB + q, computed and published by the calling wave
    auto unit_b = [&](int ub) {
        const int d = ub / QB, q = ub - d * QB;
        DecBW w;
        decb_b_load<NB>(g, s_dist[d], q, lane, w);
        decb_b_compute<NB>(g, X, s_dcnt, s_dpair, d, q, lane, w);
        vm_drain();   // the activations are out before the word
        if (lane == 0) tw_store(g.tw2 + UA + ub, tag, 1u);
    };

    // Wait until the n words at tw2[word(i)], i < n, carry this launch's tag.
    // Each thread polls its share; after g.rescue_polls tries the missing
    // units are listed and computed by this WG's waves (rescue(u)), which
    // publish them, and the poll repeats.  False when the spin budget ran out.
    auto wait_words = [&](int n, auto word, auto rescue) -> bool {
        for (;;) {
            // one round = every word of the thread loaded at once (one
            // latency), repeated up to g.rescue_polls times while any is missing
            bool miss = true;
            for (unsigned r = 0; r <= g.rescue_polls && miss; ++r) {
                if (r) __builtin_amdgcn_s_sleep(1);
                miss = false;
#pragma unroll 4
                for (int i = tid; i < n; i += DECB_THREADS)
                    miss |= (uint32_t)(tw_load(g.tw2 + word(i)) >> 32) != tag;
            }
            if (dec_none_missing(s_wmiss, miss)) return true;
            dec_lds_barrier();   // earlier readers of the list are done
            if (tid == 0) s_nmiss = 0;
            dec_lds_barrier();
            for (int i = tid; i < n; i += DECB_THREADS) {
                const uint64_t wv = tw_load(g.tw2 + word(i));
                if ((uint32_t)(wv >> 32) != tag) {
                    const int at = atomicAdd(&s_nmiss, 1);
                    if (at < DECB_LIST) s_list[at] = word(i);
                }
            }
            dec_lds_barrier();
            const int nm = imin(__builtin_amdgcn_readfirstlane(s_nmiss), DECB_LIST);
            spins += g.rescue_polls + 1;
            if (spins > DEC_SPIN_LIMIT) return false;
            for (int m = wave; m < nm; m += DECB_WAVES) rescue(__builtin_amdgcn_readfirstlane(s_list[m]));
            dec_lds_barrier();
        }
    };


    // ---- A: router rows and Q8_K of x, by waves, dealt across the WGs first
    // (unit u to wave u / G of WG u % G): every CU takes about UA / G of them
    for (int u = wave * G + wg; u < UA; u += NW) decb_unit_a(g, tag, u, lane);

    // ---- every A word (the logits travel in them); missing units computed here
    ok = wait_words(UA, [&](int i) { return i; }, [&](int u) { decb_unit_a(g, tag, u, lane); });
    // the logits and x's Q8_K for every token (coherent loads: other WGs wrote
    // them): every load goes out at once (one memory round trip, not one per
    // array); the logits land in LDS now, the codes after the ranking
    constexpr int LG_PER = DECB_T_MAX * 256 / DECB_THREADS;                      // logit words per thread
    constexpr int XQ_PER = DECB_T_MAX * DECB_NB_MAX * QK / 16 / DECB_THREADS;   // 16-byte pieces per thread
    constexpr int XB_PER = (DECB_T_MAX * DECB_NB_MAX * 8 + DECB_THREADS - 1) / DECB_THREADS;   // block-sum words
    static_assert(DECB_T_MAX * DECB_NB_MAX <= DECB_THREADS, "one scale per thread");
    uint64_t lgv[LG_PER];
    u32x4 xqv[XQ_PER];
    uint32_t xbv[XB_PER];
    float xdv = 0.f;
    const int nxq = T * D / 16, nxb = T * (D / 16) / 2;
    {
#pragma unroll
        for (int j = 0; j < LG_PER; ++j) {
            const int i = tid + j * DECB_THREADS;
            if (i < E * T) lgv[j] = tw_load(g.tw2 + i);
        }
        const auto rq = co_rsrc(g.xq, (uint32_t)(T * D));
#pragma unroll
        for (int j = 0; j < XQ_PER; ++j) {
            const int i = tid + j * DECB_THREADS;
            if (i < nxq) xqv[j] = co_ld16(rq, 16u * (uint32_t)i);
        }
        const auto rd = co_rsrc(g.xd, (uint32_t)(4 * T * NB));
        if (tid < T * NB) xdv = as_float(co_ld4(rd, 4u * (uint32_t)tid));
        const auto rb = co_rsrc(g.xbs, (uint32_t)(2 * T * (D / 16)));
#pragma unroll
        for (int j = 0; j < XB_PER; ++j) {
            const int i = tid + j * DECB_THREADS;
            if (i < nxb) xbv[j] = co_ld4(rb, 4u * (uint32_t)i);
        }
    }
#pragma unroll
    for (int j = 0; j < LG_PER; ++j) {
        const int i = tid + j * DECB_THREADS;
        if (i < E * T) s_logit[i] = as_float((uint32_t)lgv[j]);
    }
    if (tid < T * NB) s_xd[tid] = xdv;
#pragma unroll
    for (int j = 0; j < XB_PER; ++j) {
        const int i = tid + j * DECB_THREADS;
        if (i < nxb) {
            s_xbs[2 * i] = (int16_t)(uint16_t)(xbv[j] & 0xffffu);
            s_xbs[2 * i + 1] = (int16_t)(uint16_t)(xbv[j] >> 16);
        }
    }
    for (int e = tid; e < E; e += DECB_THREADS) {
        s_first[e] = DECB_T_MAX * DEC_KMAX;
        s_tmask[e] = 0u;
    }
    dec_lds_barrier();
    // ---- ranking: token t by wave t % 8 (the shared top-k / softmax code)
    for (int t = wave; t < T; t += DECB_WAVES) {
        int mysel;
        float myw;
        topk_softmax_wave(s_logit + t * E, E, K, lane, mysel, myw, true);
        if (lane < K) {
            s_sel[t * K + lane] = mysel;
            s_w[t * K + lane] = myw;
            atomicMin(&s_first[mysel], t * K + lane);
            atomicOr(&s_tmask[mysel], 1u << t);
        }
    }
#pragma unroll
    for (int j = 0; j < XQ_PER; ++j) {
        const int i = tid + j * DECB_THREADS;
        if (i < nxq) *(u32x4 *)(s_xq + 16 * i) = xqv[j];
    }
    dec_lds_barrier();
    // distinct experts in first-use order of the flat pairs p = t K + k, and
    // each one's pairs in flat order (the same lists in every WG)
    const int NP = T * K;
    if (wave == 0) {
        int nd = 0;
        for (int p0 = 0; p0 < NP; p0 += 64) {
            const int p = p0 + lane;
            const bool first = p < NP && s_first[s_sel[p]] == p;
            const uint64_t m = __ballot(first);
            if (first) {
                const int d = nd + __popcll(m & ((1ull << lane) - 1ull));
                s_dist[d] = s_sel[p];
                s_eidx[s_sel[p]] = d;
            }
            nd += __popcll(m);
        }
        if (lane == 0) s_nd = nd;
    }
    dec_lds_barrier();
    const int ND = __builtin_amdgcn_readfirstlane(s_nd);
    // pair p = t K + k of expert e: the j-th of e's pairs, j = the tokens
    // before t that picked e (a token picks an expert once)
    for (int p = tid; p < NP; p += DECB_THREADS) {
        const int e = s_sel[p], t = p / K, d = s_eidx[e];
        const unsigned m = s_tmask[e];
        s_pd[p] = d;
        s_dpair[d * DECB_PAIRS_MAX + __popc(m & ((1u << t) - 1u))] = p;
        if ((m & ((1u << t) - 1u)) == 0u) s_dcnt[d] = __popc(m);
    }
    dec_lds_barrier();
    if (wg == 0) {
        // routing outputs: logits, ids, weights, and the dispatch of the T K
        // ids (stable counting sort)
        for (int i = tid; i < E * T; i += DECB_THREADS) g.logits[i] = s_logit[i];
        for (int p = tid; p < NP; p += DECB_THREADS) {
            g.sel[p] = s_sel[p];
            g.w[p] = s_w[p];
            const int e = s_sel[p];
            int below = 0, before = 0;
            for (int q2 = 0; q2 < NP; ++q2) {
                below += s_sel[q2] < e;
                before += (s_sel[q2] == e) & (q2 < p);
            }
            g.perm[below + before] = p;
        }
        for (int e = tid; e < E; e += DECB_THREADS) {
            int cnt = 0, below = 0;
            for (int q2 = 0; q2 < NP; ++q2) {
                cnt += s_sel[q2] == e;
                below += s_sel[q2] < e;
            }
            g.counts[e] = cnt;
            g.offsets[e] = below;
        }
        if (tid == 0) g.offsets[E] = NP;
    }

    // ---- B: (distinct expert, 4 row pairs) units by waves; the next unit's
    // weight bytes load while the current one computes
    const int UB = ND * QB;
    if (ok) {
        int u = gw;
        DecBW wc, wn;
        if (u < UB) decb_b_load<NB>(g, s_dist[u / QB], u % QB, lane, wc);
        for (; u < UB; u += NW) {
            const int un = u + NW;
            if (un < UB) decb_b_load<NB>(g, s_dist[un / QB], un % QB, lane, wn);
            const int d = u / QB, q = u - d * QB;
            decb_b_compute<NB>(g, X, s_dcnt, s_dpair, d, q, lane, wc);
            vm_drain();   // activations (and the next loads) are in
            if (lane == 0) tw_store(g.tw2 + UA + u, tag, 1u);
            wc = wn;
        }
    }

    // ---- C: (token, CC columns) units by WGs
    const int CC = g.C;                  // columns per C unit (a multiple of 8, <= 64)
    const int UCT = D / CC, UC = T * UCT;
    for (int cu = wg; cu < UC; cu += G) {
        const int t = cu / UCT, n0 = (cu - t * UCT) * CC;
        // wave k's down rows (slot k's expert, columns n0 ..): passes of 8
        // rows, the loads AH passes ahead of the dots, as deep as the
        // registers allow without spilling (Q6_K's raw bytes of a pass take 56
        // registers at I = 1024).  The expert is known since the ranking, so
        // the first AH passes go out before the wait for the B words below.
        constexpr int AH = DT == 12 ? (NBI <= 3 ? 2 : 1) : 0;
        const int npass = CC / 8;
        const int rs = lane >> 3, sl = lane & 7;
        const int e_dn = wave < K ? s_sel[t * K + wave] : 0;
        DecBDn<DT> rb[AH + 1];
        if (wave < K) {
#pragma unroll
            for (int a = 0; a < AH; ++a)
                if (a < npass) decb_dn_load<DT, NBI>(g.down, e_dn, n0 + 8 * a + rs, sl, rb[a]);
        }
        // the B words of the token's K experts
        if (ok)
            ok = wait_words(K * QB, [&](int i) { return UA + s_pd[t * K + i / QB] * QB + i % QB; },
                            [&](int w) { unit_b(w - UA); });
        // wave k: the Q8_K of slot k's I activations (coherent loads), then
        // its CC down rows' dots, CC / 8 rows per pass, the next pass loading
        if (wave < K) {
            const int k = wave, p = t * K + k;
            const auto ra = co_rsrc(g.actf + (int64_t)p * I, (uint32_t)(4 * I));
            const int b = lane >> 4, seg = lane & 15;
            float av[16];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                u32x4 a4 = {0u, 0u, 0u, 0u};
                if (b < NBI) a4 = co_ld16(ra, 4u * (uint32_t)(b * QK + 16 * seg + 4 * i));
#pragma unroll
                for (int e = 0; e < 4; ++e) av[4 * i + e] = as_float(a4[e]);
            }
            int qv[16], bsum;
            const float dq = q8k_wave4x16(av, lane, qv, bsum);
            if (b < NBI) {
                u32x4 pk;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int qi[4] = {qv[4 * i], qv[4 * i + 1], qv[4 * i + 2], qv[4 * i + 3]};
                    pk[i] = pack_i8x4(qi);
                }
                *(u32x4 *)(s_aq[k] + b * QK + 16 * seg) = pk;
                s_abs[k][b * 16 + seg] = (int16_t)bsum;
                if (seg == 0) s_ad[k][b] = dq;
            }
            wave_lds_sync();
            // a rolled loop (the buffers rotate by copies): unrolled, the
            // scheduler would hoist every pass's loads
#pragma unroll 1
            for (int ps = 0; ps < npass; ++ps) {
                if (ps + AH < npass) decb_dn_load<DT, NBI>(g.down, e_dn, n0 + 8 * (ps + AH) + rs, sl, rb[AH]);
                float z = decb_dn_dot<DT, NBI>(rb[0], sl, s_aq[k], s_ad[k], s_abs[k]);
                z = decb_sum8(z);
                if (sl == 0) s_z[k][8 * ps + rs] = z;
#pragma unroll
                for (int a = 0; a < AH; ++a) rb[a] = rb[a + 1];
            }
        }
        if (!ok) s_fail = 1;
        dec_lds_barrier();
        const bool failed = s_fail != 0;
        if (tid < CC) {
            double s = 0.0;
            for (int k = 0; k < K; ++k) s = s + (double)(s_z[k][tid] * s_w[t * K + k]);
            const int64_t o = (int64_t)t * D + n0 + tid;
            float v = g.res ? g.res[o] + (float)s : (float)s;
            if (failed) v = __builtin_nanf("");
            g.out[o] = v;
        }
        dec_lds_barrier();   // s_z / s_aq are rewritten by the next unit
    }
    if (!ok) s_fail = 1;
    dec_lds_barrier();
    if (tid == 0) {
        if (s_fail) __hip_atomic_fetch_add(g.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(g.epoch + wg, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int DT, int NB>
static const void *decodeb_fn2(int nbi) {
    switch (nbi) {
    case 1: return (const void *)k_decodeb<DT, NB, 1>;
    case 2: return (const void *)k_decodeb<DT, NB, 2>;
    case 3: return (const void *)k_decodeb<DT, NB, 3>;
    case 4: return (const void *)k_decodeb<DT, NB, 4>;
    default: return nullptr;
    }
}
template <int DT>
static const void *decodeb_fn(int nb, int nbi) {
    switch (nb) {
    case 1: return decodeb_fn2<DT, 1>(nbi);
    case 2: return decodeb_fn2<DT, 2>(nbi);
    case 4: return decodeb_fn2<DT, 4>(nbi);
    case 8: return decodeb_fn2<DT, 8>(nbi);
    default: return nullptr;
    }
}

int launch_decodeb(const DecArgs &g, int grid, hipStream_t st) {
    if (g.T < 2 || g.T > DECB_T_MAX || g.K > DEC_KMAX || g.E > 256 || grid <= 0 || grid > DEC_MAX_GRID) return -6;
    if (g.C <= 0 || g.C > DECB_COLS || g.C % 8 || g.D % g.C) return -6;
    const int nb = g.D / QK, nbi = g.I / QK;
    const void *fn = g.down.type == 12 ? decodeb_fn<12>(nb, nbi) : g.down.type == 14 ? decodeb_fn<14>(nb, nbi) : nullptr;
    if (!fn) return -3;
    void *args[] = {(void *)&g};
    const hipError_t e = hipLaunchKernel(fn, dim3(grid), dim3(DECB_THREADS), args, 0, st);
    if (e != hipSuccess) return record_hip_error(e);
    return hip_check_launch();
}

template <int DT>
static const void *decode1_fn(int nbi) {
    switch (nbi) {
    case 1: return (const void *)k_decode1<DT, 1>;
    case 2: return (const void *)k_decode1<DT, 2>;
    case 3: return (const void *)k_decode1<DT, 3>;
    case 4: return (const void *)k_decode1<DT, 4>;
    case 5: return (const void *)k_decode1<DT, 5>;
    case 6: return (const void *)k_decode1<DT, 6>;
    case 7: return (const void *)k_decode1<DT, 7>;
    case 8: return (const void *)k_decode1<DT, 8>;
    default: return nullptr;
    }
}

int launch_decode1(const DecArgs &g, int grid, hipStream_t st) {
    const int nbi = g.I / QK;
    const void *fn = g.down.type == 12 ? decode1_fn<12>(nbi) : g.down.type == 14 ? decode1_fn<14>(nbi) : nullptr;
    if (!fn) return -3;
    void *args[] = {(void *)&g};
    const hipError_t e = hipLaunchKernel(fn, dim3(grid), dim3(DEC_THREADS), args, 0, st);
    if (e != hipSuccess) return record_hip_error(e);
    return hip_check_launch();
}

int decode1_max_grid(int device, int *grid) {
    int cus = 0;
    hipError_t e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
    if (e != hipSuccess) return record_hip_error(e);
    int per = 1;
    for (int dt = 12; dt <= 14; dt += 2)
        for (int nbi = 1; nbi <= 8; ++nbi) {
            int p = 0;
            e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&p, dt == 12 ? decode1_fn<12>(nbi) : decode1_fn<14>(nbi),
                                                             DEC_THREADS, 0);
            if (e != hipSuccess) return record_hip_error(e);
            per = imin(per, p);
        }
    *grid = cus * per;   // one WG per CU
    if (*grid > DEC_MAX_GRID) *grid = 0;
    return 0;
}

}  // namespace mimoe
