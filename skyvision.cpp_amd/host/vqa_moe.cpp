// vqa_moe.cpp - vqa::moe on the libmimoe C ABI (see vqa_moe.hpp).
//
// Reference: src/core/engine/moe_compute.cpp:33-151 (the builders) and its
// MOE_COMPUTE_TEST_MAIN self-test (:154-230), mirrored below under
// VQA_MOE_SELFTEST with the same hand-computed known answer.
#include "vqa_moe.hpp"

#include <algorithm>
#include <cstring>

namespace vqa {
namespace moe {

namespace {

int32_t mi_act_of(UnaryOp act) {
    switch (act) {
    case UnaryOp::SILU: return MI_ACT_SILU;
    case UnaryOp::GELU: return MI_ACT_GELU_TANH;
    case UnaryOp::GELU_ERF: return MI_ACT_GELU_ERF;
    }
    return -1;
}

mi_tensor as_mi(const Tensor *t) {
    mi_tensor m{};
    m.data = t->data;
    m.type = t->type;
    for (int i = 0; i < 4; ++i) {
        m.ne[i] = t->ne[i];
        m.nb[i] = t->nb[i];
    }
    return m;
}

// bytes of a row of n values (mi_row_size covers the expert-table types)
size_t row_bytes(int type, int64_t n) {
    if (n <= 0) return 0;
    if (type == MI_TYPE_I32) return 4 * (size_t)n;
    return mi_row_size(type, n);
}

// rows of ne0 values stored back to back, planes back to back
bool contiguous(const Tensor *t) {
    const size_t row = row_bytes(t->type, t->ne[0]);
    return row > 0 && t->nb[1] == row && t->nb[2] == row * (size_t)t->ne[1] &&
           t->nb[3] == t->nb[2] * (size_t)t->ne[2];
}

size_t bytes_of(const Tensor *t) { return t->nb[3] * (size_t)t->ne[3]; }

}  // namespace

// ------------------------------------------------------------------ Session
Session::Session(int device) {
    if (fail(mi_moe_ctx_create(&ctx_, device))) return;
    fail(mi_stream_create(&stream_));
}

Session::~Session() {
    if (stream_) (void)mi_stream_synchronize(stream_);
    for (Tensor *t : owned_) {
        (void)mi_dev_free(t->data);
        delete t;
    }
    if (stream_) (void)mi_stream_destroy(stream_);
    if (ctx_) mi_moe_ctx_destroy(ctx_);
}

int Session::fail(int rc) {
    if (rc && !status_) status_ = rc;
    return rc;
}

Tensor *Session::new_tensor(int type, int64_t ne0, int64_t ne1, int64_t ne2) {
    const size_t row = row_bytes(type, ne0);
    if (!row || ne1 <= 0 || ne2 <= 0) {
        fail(MI_MOE_ERR_SHAPE);
        return nullptr;
    }
    Tensor *t = new Tensor;
    t->type = type;
    t->ne[0] = ne0; t->ne[1] = ne1; t->ne[2] = ne2; t->ne[3] = 1;
    t->nb[0] = type == MI_TYPE_F32 || type == MI_TYPE_I32 ? 4 : type == MI_TYPE_F16 ? 2 : row / (size_t)(ne0 / 256);
    t->nb[1] = row;
    t->nb[2] = row * (size_t)ne1;
    t->nb[3] = t->nb[2] * (size_t)ne2;
    if (fail(mi_dev_malloc(&t->data, bytes_of(t)))) {
        delete t;
        return nullptr;
    }
    owned_.push_back(t);
    return t;
}

int Session::set(Tensor *t, const void *host, size_t bytes) {
    if (!t || !host) return fail(MI_MOE_ERR_NULL);
    if (bytes > bytes_of(t)) return fail(MI_MOE_ERR_SHAPE);
    if (int rc = fail(mi_stream_synchronize(stream_))) return rc;
    return fail(mi_memcpy_h2d(t->data, host, bytes));
}

int Session::get(const Tensor *t, void *host, size_t bytes) {
    if (!t || !host) return fail(MI_MOE_ERR_NULL);
    if (bytes > bytes_of(t)) return fail(MI_MOE_ERR_SHAPE);
    if (int rc = fail(mi_stream_synchronize(stream_))) return rc;
    return fail(mi_memcpy_d2h(host, t->data, bytes));
}

int Session::compute() {
    if (status_) return status_;
    return fail(mi_stream_synchronize(stream_));
}

int Session::ensure(int64_t T, int32_t D, int32_t I, int32_t E, int32_t K) {
    if (T <= cap_T_ && D <= cap_D_ && I <= cap_I_ && E <= cap_E_ && K <= cap_K_) return 0;
    // the workspace is replaced: nothing queued may still use it
    if (int rc = fail(mi_stream_synchronize(stream_))) return rc;
    cap_T_ = std::max(cap_T_, T);
    cap_D_ = std::max(cap_D_, D);
    cap_I_ = std::max(cap_I_, I);
    cap_E_ = std::max(cap_E_, E);
    cap_K_ = std::max(cap_K_, K);
    return fail(mi_moe_ctx_reserve(ctx_, cap_T_, cap_D_, cap_I_, cap_E_, cap_K_));
}

// ------------------------------------------------------------------ v3 table form
Tensor *build_expert_ffn_table_res(Session &s, Tensor *x, Tensor *res, Tensor *gate_table, Tensor *up_table,
                                   Tensor *down_table, Tensor *gate_up_ids, Tensor *down_ids, Tensor *w,
                                   UnaryOp act) {
    // moe_compute.cpp:102-122, in order
    if (!s.ctx() || !x || !res || !w) return nullptr;
    if (!gate_table || !up_table || !down_table || !gate_up_ids || !down_ids) return nullptr;
    if (w->type != MI_TYPE_F32) return nullptr;
    const int64_t K = w->ne[0];
    const int64_t T = x->ne[1];
    if (K <= 0 || w->ne[1] != T || w->ne[2] != 1 || w->ne[3] != 1) return nullptr;
    if (res->ne[0] != x->ne[0] || res->ne[1] != T) return nullptr;
    if (gate_up_ids->type != MI_TYPE_I32 || down_ids->type != MI_TYPE_I32) return nullptr;
    if (gate_up_ids->ne[0] != K || down_ids->ne[0] != K) return nullptr;
    if (gate_up_ids->ne[1] != T || down_ids->ne[1] != T) return nullptr;
    if (gate_table->type != up_table->type || gate_table->ne[0] != up_table->ne[0] ||
        gate_table->ne[1] != up_table->ne[1] || gate_table->nb[1] != up_table->nb[1])
        return nullptr;
    if (gate_table->ne[0] != x->ne[0]) return nullptr;
    if (up_table->ne[0] != x->ne[0]) return nullptr;
    if (down_table->ne[0] != gate_table->ne[1]) return nullptr;
    if (down_table->ne[1] != x->ne[0]) return nullptr;
    // this build: F32 contiguous activations, one slot count for the tables
    if (x->type != MI_TYPE_F32 || res->type != MI_TYPE_F32) return nullptr;
    if (!contiguous(x) || !contiguous(res) || !contiguous(w) || !contiguous(gate_up_ids) || !contiguous(down_ids))
        return nullptr;
    if (up_table->ne[2] != gate_table->ne[2] || down_table->ne[2] != gate_table->ne[2]) return nullptr;
    if (T <= 0 || x->ne[0] > INT32_MAX || gate_table->ne[1] > INT32_MAX || gate_table->ne[2] > INT32_MAX ||
        K > INT32_MAX)
        return nullptr;
    const int32_t D = (int32_t)x->ne[0], I = (int32_t)gate_table->ne[1], E = (int32_t)gate_table->ne[2];

    Tensor *out = s.new_tensor(MI_TYPE_F32, D, T);
    if (!out || s.ensure(T, D, I, E, (int32_t)K)) return nullptr;
    mi_moe_layer L{};
    L.n_embd = D;
    L.n_expert = E;
    L.n_expert_used = (int32_t)K;
    L.n_ff = I;
    L.gate = as_mi(gate_table);
    L.up = as_mi(up_table);
    L.down = as_mi(down_table);
    L.fused_gate_up = 0;
    L.act = mi_act_of(act);
    L.gating = 0;
    if (s.fail(mi_moe_expert_ffn(s.ctx(), &L, (const float *)x->data, T, (const float *)res->data,
                                 (const int32_t *)gate_up_ids->data, (const int32_t *)down_ids->data,
                                 (const float *)w->data, (float *)out->data, s.stream())))
        return nullptr;
    return out;
}

Tensor *build_expert_ffn_table(Session &s, Tensor *x, Tensor *gate_table, Tensor *up_table, Tensor *down_table,
                               Tensor *gate_up_ids, Tensor *down_ids, Tensor *w, UnaryOp act) {
    return build_expert_ffn_table_res(s, x, x, gate_table, up_table, down_table, gate_up_ids, down_ids, w, act);
}

// ------------------------------------------------------------------ v1 per-slot form
Tensor *build_expert_ffn_res(Session &s, Tensor *x, Tensor *res, const std::vector<Tensor *> &gate,
                             const std::vector<Tensor *> &up, const std::vector<Tensor *> &down, Tensor *w,
                             UnaryOp act) {
    // moe_compute.cpp:43-58, in order
    const size_t n_used = gate.size();
    if (!s.ctx() || !x || !res || !w || n_used == 0) return nullptr;
    if (up.size() != n_used || down.size() != n_used) return nullptr;
    if (w->type != MI_TYPE_F32) return nullptr;
    if (w->ne[0] != (int64_t)n_used) return nullptr;
    if (w->ne[1] != x->ne[1] || w->ne[2] != 1 || w->ne[3] != 1) return nullptr;
    if (res->ne[0] != x->ne[0] || res->ne[1] != x->ne[1]) return nullptr;
    for (size_t k = 0; k < n_used; k++) {
        if (!gate[k] || !up[k] || !down[k]) return nullptr;
        if (gate[k]->ne[0] != x->ne[0] || up[k]->ne[0] != x->ne[0]) return nullptr;
        if (down[k]->ne[0] != gate[k]->ne[1] || down[k]->ne[0] != up[k]->ne[1]) return nullptr;
        if (down[k]->ne[1] != x->ne[0]) return nullptr;
    }
    // this build: one type and shape per role, contiguous 2D tensors; slot k
    // of every token is expert tensor k, so the tables are the tensors packed
    // in slot order and the ids are 0 .. n_used - 1 for every token
    const std::vector<Tensor *> *roles[3] = {&gate, &up, &down};
    for (const auto *r : roles)
        for (const Tensor *t : *r)
            if (t->type != (*r)[0]->type || t->ne[1] != (*r)[0]->ne[1] || t->ne[2] != 1 || t->ne[3] != 1 ||
                !contiguous(t))
                return nullptr;
    const int64_t T = x->ne[1];
    const int64_t K = (int64_t)n_used;
    Tensor *tables[3];
    for (int r = 0; r < 3; ++r) {
        const Tensor *t0 = (*roles[r])[0];
        tables[r] = s.new_tensor(t0->type, t0->ne[0], t0->ne[1], K);
        if (!tables[r]) return nullptr;
        for (int64_t k = 0; k < K; ++k)
            if (s.fail(mi_memcpy_d2d((char *)tables[r]->data + (size_t)k * tables[r]->nb[2],
                                     (*roles[r])[k]->data, tables[r]->nb[2])))
                return nullptr;
    }
    Tensor *ids = s.new_tensor(MI_TYPE_I32, K, T);
    if (!ids) return nullptr;
    std::vector<int32_t> h((size_t)(K * T));
    for (int64_t t = 0; t < T; ++t)
        for (int64_t k = 0; k < K; ++k) h[(size_t)(t * K + k)] = (int32_t)k;
    if (s.set(ids, h.data(), h.size() * sizeof(int32_t))) return nullptr;
    return build_expert_ffn_table_res(s, x, res, tables[0], tables[1], tables[2], ids, ids, w, act);
}

Tensor *build_expert_ffn(Session &s, Tensor *x, const std::vector<Tensor *> &gate,
                         const std::vector<Tensor *> &up, const std::vector<Tensor *> &down, Tensor *w,
                         UnaryOp act) {
    return build_expert_ffn_res(s, x, x, gate, up, down, w, act);
}

}  // namespace moe
}  // namespace vqa

// ------------------------------------------------------------------ GraphB
namespace vqa {
namespace moe {

GraphB::GraphB(int device, const mi_moe_layer &layer, int64_t max_tokens, bool tiled)
    : layer_(layer), cap_T_(max_tokens) {
    const int64_t D = layer.n_embd, K = layer.n_expert_used;
    if (max_tokens <= 0 || D <= 0 || K <= 0) {
        fail(MI_MOE_ERR_SHAPE);
        return;
    }
    if (fail(mi_moe_ctx_create(&ctx_, device))) return;
    if (fail(mi_moe_ctx_reserve(ctx_, max_tokens, layer.n_embd, layer.n_ff, layer.n_expert, layer.n_expert_used)))
        return;
    if (fail(mi_stream_create(&stream_))) return;
    const size_t rows = sizeof(float) * (size_t)(max_tokens * D), route = 4 * (size_t)(max_tokens * K);
    if (fail(mi_dev_malloc((void **)&d_in_, rows)) || fail(mi_dev_malloc((void **)&d_xmid_, rows)) ||
        fail(mi_dev_malloc((void **)&d_out_, rows)) || fail(mi_dev_malloc((void **)&d_w_, route)) ||
        fail(mi_dev_malloc((void **)&d_ids_, route)))
        return;
    if (tiled) attach_tiled();
}

// Tiled copies of the tables the library takes them for (Q4_K gate / up, a
// fused [h | g] table with n_ff a multiple of 32, Q4_K or Q6_K down; whole
// 32-row groups): made on this object's stream, so every later call sees
// them complete.  A table that does not qualify, or whose copy fails, stays
// untiled (the status is not touched: the layer runs either way).
void GraphB::attach_tiled() {
    auto tile = [&](const mi_tensor &t, mi_tensor &slot) {
        const int64_t n = mi_moe_tiled_bytes(&t);
        void *buf = nullptr;
        if (n <= 0 || mi_dev_malloc(&buf, (size_t)n) != MI_MOE_OK) return false;
        if (mi_moe_tile(ctx_, &t, buf, &slot, stream_) != MI_MOE_OK) {
            (void)mi_dev_free(buf);
            slot = mi_tensor{};
            return false;
        }
        tiled_.push_back(buf);
        return true;
    };
    const bool gated = layer_.act != MI_ACT_RELU_SQR, sep = gated && !layer_.fused_gate_up;
    const bool gate_ok = layer_.gate.type == MI_TYPE_Q4_K && (!sep || layer_.up.type == MI_TYPE_Q4_K) &&
                         !(gated && layer_.fused_gate_up && layer_.n_ff % 32);
    if (gate_ok && tile(layer_.gate, layer_.gate_tiled) && sep && !tile(layer_.up, layer_.up_tiled))
        layer_.gate_tiled = mi_tensor{};   // both or neither (its buffer is freed with the others)
    (void)tile(layer_.down, layer_.down_tiled);
}

GraphB::~GraphB() {
    if (stream_) (void)mi_stream_synchronize(stream_);
    for (void *p : {(void *)d_in_, (void *)d_xmid_, (void *)d_out_, (void *)d_w_, (void *)d_ids_})
        if (p) (void)mi_dev_free(p);
    for (void *p : tiled_) (void)mi_dev_free(p);
    if (stream_) (void)mi_stream_destroy(stream_);
    mi_moe_ctx_destroy(ctx_);
}

int GraphB::fail(int rc) {
    if (rc && !status_) status_ = rc;
    return rc;
}

int GraphB::feed(const float *moe_in, const float *xmid_in, int64_t T, const int32_t *ids, const float *w) {
    if (status_) return status_;
    if (!moe_in || !xmid_in || (!ids) != (!w)) return MI_MOE_ERR_NULL;
    if (T <= 0 || T > cap_T_) return MI_MOE_ERR_CAPACITY;
    const size_t rows = sizeof(float) * (size_t)(T * layer_.n_embd), route = 4 * (size_t)(T * layer_.n_expert_used);
    int rc = mi_memcpy_h2d_async(d_in_, moe_in, rows, stream_);
    if (!rc) rc = mi_memcpy_h2d_async(d_xmid_, xmid_in, rows, stream_);
    if (!rc && ids) rc = mi_memcpy_h2d_async(d_ids_, ids, route, stream_);
    if (!rc && w) rc = mi_memcpy_h2d_async(d_w_, w, route, stream_);
    if (rc) return fail(rc);
    T_ = T;
    routed_ = ids != nullptr;
    return MI_MOE_OK;
}

int GraphB::compute(float *hid_out) {
    if (status_) return status_;
    if (!hid_out) return MI_MOE_ERR_NULL;
    if (T_ <= 0) return MI_MOE_ERR_ARG;   // nothing fed
    int rc = routed_ ? mi_moe_expert_ffn(ctx_, &layer_, d_in_, T_, d_xmid_, d_ids_, d_ids_, d_w_, d_out_, stream_)
                     : mi_moe_forward(ctx_, &layer_, d_in_, T_, d_xmid_, d_out_, nullptr, stream_);
    if (!rc) rc = mi_memcpy_d2h_async(hid_out, d_out_, sizeof(float) * (size_t)(T_ * layer_.n_embd), stream_);
    if (!rc) rc = mi_stream_synchronize(stream_);
    return rc ? fail(rc) : MI_MOE_OK;
}

}  // namespace moe
}  // namespace vqa

#ifdef VQA_MOE_SELFTEST
// The reference's self-test (moe_compute.cpp:154-230) on this build: D = 2,
// I = 3, K = 2, T = 1, F32, SiLU; out = x + 0.5 f0 + 1.0 f1 = [3.6423913,
// 4.1931758] (hand-computed there); a w with the wrong row count gives
// nullptr.  Added: the same answer through the slot-table form, the residual
// split (res != x), and the table form's argument checks.
//
// `vqa_moe_selftest --table DIR` instead runs build_expert_ffn_table_res on
// tables read from DIR (meta.txt: T D I E K gate_type down_type act same_ids
// gemm_threshold; x.bin res.bin gate.bin up.bin down.bin ids_gu.bin
// [ids_dn.bin] w.bin, raw little-endian) and writes out.bin: a caller's
// check of the table form on any table type and id pattern.
#include <cmath>
#include <cstdio>
#include <string>

static bool load_into(vqa::moe::Session &s, vqa::moe::Tensor *t, const std::string &path, size_t bytes) {
    if (!t) return false;
    std::FILE *f = std::fopen(path.c_str(), "rb");
    if (!f) return false;
    std::vector<char> buf(bytes);
    const size_t got = std::fread(buf.data(), 1, bytes, f);
    std::fclose(f);
    return got == bytes && s.set(t, buf.data(), bytes) == 0;
}

static int table_mode(const std::string &dir) {
    long T, D, I, E, K, gt, dt, act, same, thr;
    std::FILE *m = std::fopen((dir + "/meta.txt").c_str(), "r");
    if (!m) return 2;
    const int n = std::fscanf(m, "%ld %ld %ld %ld %ld %ld %ld %ld %ld %ld", &T, &D, &I, &E, &K, &gt, &dt, &act, &same, &thr);
    std::fclose(m);
    if (n != 10) return 2;
    vqa::moe::Session s(0);
    if (s.status()) return 3;
    using vqa::moe::Tensor;
    Tensor *x = s.new_tensor(MI_TYPE_F32, D, T), *res = s.new_tensor(MI_TYPE_F32, D, T);
    Tensor *g = s.new_tensor((int)gt, D, I, E), *u = s.new_tensor((int)gt, D, I, E), *d = s.new_tensor((int)dt, I, D, E);
    Tensor *ig = s.new_tensor(MI_TYPE_I32, K, T);
    Tensor *id = same ? ig : s.new_tensor(MI_TYPE_I32, K, T);
    Tensor *w = s.new_tensor(MI_TYPE_F32, K, T);
    bool ok = x && res && g && u && d && ig && id && w;
    ok = ok && load_into(s, x, dir + "/x.bin", x->nb[3]) && load_into(s, res, dir + "/res.bin", res->nb[3]);
    ok = ok && load_into(s, g, dir + "/gate.bin", g->nb[3]) && load_into(s, u, dir + "/up.bin", u->nb[3]);
    ok = ok && load_into(s, d, dir + "/down.bin", d->nb[3]) && load_into(s, ig, dir + "/ids_gu.bin", ig->nb[3]);
    ok = ok && (same || load_into(s, id, dir + "/ids_dn.bin", id->nb[3])) && load_into(s, w, dir + "/w.bin", w->nb[3]);
    if (!ok) return 4;
    if (mi_moe_ctx_set_gemm_threshold(s.ctx(), thr)) return 5;
    const vqa::moe::UnaryOp op = act == 0 ? vqa::moe::UnaryOp::SILU
                                 : act == 1 ? vqa::moe::UnaryOp::GELU : vqa::moe::UnaryOp::GELU_ERF;
    Tensor *out = vqa::moe::build_expert_ffn_table_res(s, x, res, g, u, d, ig, id, w, op);
    if (!out || s.compute()) {
        std::fprintf(stderr, "table build failed: status %d\n", s.status());
        return 6;
    }
    std::vector<char> o(out->nb[3]);
    if (s.get(out, o.data(), o.size())) return 7;
    std::FILE *f = std::fopen((dir + "/out.bin").c_str(), "wb");
    if (!f) return 8;
    const size_t wr = std::fwrite(o.data(), 1, o.size(), f);
    std::fclose(f);
    std::fprintf(stderr, "table mode: T=%ld D=%ld I=%ld E=%ld K=%ld types %ld/%ld, %s ids: wrote out.bin\n", T, D, I,
                 E, K, gt, dt, same ? "one" : "two");
    return wr == o.size() ? 0 : 9;
}

static int g_fail = 0;
#define CHECK(cond, msg)                                               \
    do {                                                               \
        if (!(cond)) {                                                 \
            std::fprintf(stderr, "FAIL %s (line %d)\n", msg, __LINE__); \
            g_fail++;                                                  \
        }                                                              \
    } while (0)

using vqa::moe::Tensor;

int main(int argc, char **argv) {
    if (argc == 3 && std::string(argv[1]) == "--table") return table_mode(argv[2]);
    vqa::moe::Session s(0);
    CHECK(s.status() == 0, "session");
    if (s.status()) return 1;
    const float gate0[6] = {0, 1, 1, 0, 0, 0};   // [I = 3 rows, D = 2]
    const float up0[6] = {1, 0, 0, 1, 1, 1};
    const float down0[6] = {1, 0, 0, 0, 1, 0};   // [D = 2 rows, I = 3]
    const float gate1[6] = {1, 0, 0, 1, 0, 0};
    const float up1[6] = {0, 1, 1, 0, 0, 0};
    const float down1[6] = {0, 1, 0, 1, 0, 0};
    const float xv[2] = {1.0f, 2.0f};
    const float wv[2] = {0.5f, 1.0f};
    const float want[2] = {3.6423913f, 4.1931758f};
    auto mk = [&](const float *d, int ne0, int ne1) {
        Tensor *t = s.new_tensor(MI_TYPE_F32, ne0, ne1);
        if (t) s.set(t, d, sizeof(float) * ne0 * ne1);
        return t;
    };
    std::vector<Tensor *> gate = {mk(gate0, 2, 3), mk(gate1, 2, 3)};
    std::vector<Tensor *> up = {mk(up0, 2, 3), mk(up1, 2, 3)};
    std::vector<Tensor *> down = {mk(down0, 3, 2), mk(down1, 3, 2)};
    Tensor *x = mk(xv, 2, 1);
    Tensor *w = mk(wv, 2, 1);

    Tensor *out = vqa::moe::build_expert_ffn(s, x, gate, up, down, w);
    CHECK(out, "build");
    float o[2] = {0, 0};
    if (out) {
        CHECK(s.compute() == 0, "compute");
        s.get(out, o, sizeof(o));
        CHECK(std::fabs(o[0] - want[0]) < 1e-5f && std::fabs(o[1] - want[1]) < 1e-5f, "values");
        std::fprintf(stderr, "moe out = [%.7f, %.7f] expected [%.7f, %.7f]\n", o[0], o[1], want[0], want[1]);
    }
    Tensor *wbad = s.new_tensor(MI_TYPE_F32, 3, 1);
    CHECK(vqa::moe::build_expert_ffn(s, x, gate, up, down, wbad) == nullptr, "bad w rows -> nullptr");

    // slot tables [D, I, 2] / [I, D, 2] and ids [2, 1]
    const float gt[12] = {0, 1, 1, 0, 0, 0, 1, 0, 0, 1, 0, 0};
    const float ut[12] = {1, 0, 0, 1, 1, 1, 0, 1, 1, 0, 0, 0};
    const float dt[12] = {1, 0, 0, 0, 1, 0, 0, 1, 0, 1, 0, 0};
    const int32_t idv[2] = {0, 1};
    Tensor *gT = s.new_tensor(MI_TYPE_F32, 2, 3, 2), *uT = s.new_tensor(MI_TYPE_F32, 2, 3, 2);
    Tensor *dT = s.new_tensor(MI_TYPE_F32, 3, 2, 2), *ids = s.new_tensor(MI_TYPE_I32, 2, 1);
    s.set(gT, gt, sizeof(gt));
    s.set(uT, ut, sizeof(ut));
    s.set(dT, dt, sizeof(dt));
    s.set(ids, idv, sizeof(idv));
    Tensor *out2 = vqa::moe::build_expert_ffn_table(s, x, gT, uT, dT, ids, ids, w);
    CHECK(out2, "table build");
    if (out2) {
        float o2[2] = {0, 0};
        CHECK(s.compute() == 0, "table compute");
        s.get(out2, o2, sizeof(o2));
        CHECK(std::fabs(o2[0] - want[0]) < 1e-5f && std::fabs(o2[1] - want[1]) < 1e-5f, "table values");
        std::fprintf(stderr, "table out = [%.7f, %.7f]\n", o2[0], o2[1]);
    }
    // residual split: res = [10, 20] -> out = res + (want - x)
    const float rv[2] = {10.0f, 20.0f};
    Tensor *res = mk(rv, 2, 1);
    Tensor *out3 = vqa::moe::build_expert_ffn_table_res(s, x, res, gT, uT, dT, ids, ids, w, vqa::moe::UnaryOp::SILU);
    CHECK(out3, "table_res build");
    if (out3) {
        float o3[2] = {0, 0};
        CHECK(s.compute() == 0, "table_res compute");
        s.get(out3, o3, sizeof(o3));
        CHECK(std::fabs(o3[0] - (10.0f + want[0] - 1.0f)) < 1e-5f &&
                  std::fabs(o3[1] - (20.0f + want[1] - 2.0f)) < 1e-5f,
              "table_res values");
    }
    // argument checks of the table form
    Tensor *ids_f = s.new_tensor(MI_TYPE_F32, 2, 1);
    CHECK(vqa::moe::build_expert_ffn_table(s, x, gT, uT, dT, ids_f, ids, w) == nullptr, "F32 ids -> nullptr");
    CHECK(vqa::moe::build_expert_ffn_table(s, x, gT, dT, dT, ids, ids, w) == nullptr,
          "gate/up shape mismatch -> nullptr");
    CHECK(vqa::moe::build_expert_ffn_table(s, x, gT, uT, gT, ids, ids, w) == nullptr, "down rows -> nullptr");
    CHECK(vqa::moe::build_expert_ffn_table(s, x, gT, uT, dT, ids, ids, wbad) == nullptr, "w rows -> nullptr");
    CHECK(s.compute() == 0, "session status");
    if (s.status()) std::fprintf(stderr, "session status %d (%s)\n", s.status(), mi_last_hip_error());

    // GraphB, the driver's graph B: (1) with the driver's routing, on the
    // known answer's F32 tables (experts 0, 1 = the slot tables above)
    {
        mi_moe_layer L{};
        L.n_embd = 2;
        L.n_ff = 3;
        L.n_expert = 2;
        L.n_expert_used = 2;
        auto desc = [](const Tensor *t) {
            mi_tensor m{};
            m.data = t->data;
            m.type = t->type;
            for (int i = 0; i < 4; ++i) {
                m.ne[i] = t->ne[i];
                m.nb[i] = t->nb[i];
            }
            return m;
        };
        L.gate = desc(gT);
        L.up = desc(uT);
        L.down = desc(dT);
        L.act = MI_ACT_SILU;
        vqa::moe::GraphB gb(0, L, 4);
        CHECK(gb.status() == 0, "graphb create");
        float hid[2] = {0, 0};
        CHECK(gb.feed(xv, xv, 1, idv, wv) == 0, "graphb feed");
        CHECK(gb.compute(hid) == 0, "graphb compute");
        CHECK(std::fabs(hid[0] - want[0]) < 1e-5f && std::fabs(hid[1] - want[1]) < 1e-5f, "graphb values");
        std::fprintf(stderr, "graphb out = [%.7f, %.7f]\n", hid[0], hid[1]);
        CHECK(gb.feed(xv, xv, 5, idv, wv) == MI_MOE_ERR_CAPACITY, "graphb rows beyond max_tokens");
        CHECK(gb.feed(xv, xv, 1, idv, nullptr) == MI_MOE_ERR_NULL, "graphb ids without weights");
    }
    // (2) routing itself: a Q4_K layer built on the device (D 512, I 256, E 8,
    // K 2), three rows, the same bits as mi_moe_forward
    {
        const int D = 512, I = 256, E = 8, K = 2, T = 3;
        mi_moe_layer L{};
        L.n_embd = D;
        L.n_ff = I;
        L.n_expert = E;
        L.n_expert_used = K;
        L.act = MI_ACT_GELU_ERF_GP1;
        L.fused_gate_up = 1;
        mi_moe_ctx *c = s.ctx();
        float *tmp = nullptr, *rw = nullptr, *xd = nullptr, *od = nullptr;
        void *gq = nullptr, *dq = nullptr;
        const size_t rg = mi_row_size(MI_TYPE_Q4_K, D), rd = mi_row_size(MI_TYPE_Q4_K, I);
        bool ok = mi_dev_malloc((void **)&tmp, sizeof(float) * E * 2 * I * D) == 0 &&
                  mi_dev_malloc((void **)&rw, sizeof(float) * E * D) == 0 &&
                  mi_dev_malloc((void **)&xd, sizeof(float) * T * D) == 0 &&
                  mi_dev_malloc((void **)&od, sizeof(float) * T * D) == 0 &&
                  mi_dev_malloc(&gq, rg * E * 2 * I) == 0 && mi_dev_malloc(&dq, rd * E * D) == 0;
        ok = ok && mi_moe_ctx_reserve(c, T, D, I, E, K) == 0;
        ok = ok && mi_fill_normal(c, rw, (int64_t)E * D, 7, 1, 0.f, 0.05f, s.stream()) == 0;
        ok = ok && mi_fill_normal(c, tmp, (int64_t)E * 2 * I * D, 7, 2, 0.f, 0.02f, s.stream()) == 0;
        ok = ok && mi_quantize(c, MI_TYPE_Q4_K, tmp, gq, (int64_t)E * 2 * I, D, s.stream()) == 0;
        ok = ok && mi_fill_normal(c, tmp, (int64_t)E * D * I, 7, 3, 0.f, 0.02f, s.stream()) == 0;
        ok = ok && mi_quantize(c, MI_TYPE_Q4_K, tmp, dq, (int64_t)E * D, I, s.stream()) == 0;
        ok = ok && mi_fill_normal(c, xd, (int64_t)T * D, 7, 4, 0.f, 1.f, s.stream()) == 0;
        L.router_w = rw;
        L.gate = mi_tensor{gq, MI_TYPE_Q4_K, {D, 2 * I, E, 1}, {144, rg, rg * 2 * I, rg * 2 * I * E}};
        L.down = mi_tensor{dq, MI_TYPE_Q4_K, {I, D, E, 1}, {144, rd, rd * D, rd * D * E}};
        ok = ok && mi_moe_forward(c, &L, xd, T, xd, od, nullptr, s.stream()) == 0 && s.compute() == 0;
        std::vector<float> x(T * D), want_o(T * D), got(T * D);
        ok = ok && mi_memcpy_d2h(x.data(), xd, sizeof(float) * T * D) == 0 &&
             mi_memcpy_d2h(want_o.data(), od, sizeof(float) * T * D) == 0;
        CHECK(ok, "graphb q4_k layer setup");
        vqa::moe::GraphB gb(0, L, 8);
        CHECK(gb.feed(x.data(), x.data(), T) == 0 && gb.compute(got.data()) == 0, "graphb routed by the layer");
        CHECK(std::memcmp(got.data(), want_o.data(), sizeof(float) * T * D) == 0, "graphb == mi_moe_forward");
        std::fprintf(stderr, "graphb q4_k layer: %s mi_moe_forward\n",
                     std::memcmp(got.data(), want_o.data(), sizeof(float) * T * D) ? "differs from" : "bit-identical to");
        // with tiled copies of the tables: 40 rows (past the batched decode
        // kernel's 16, so the grouped GEMMs run and read the copies)
        const int T2 = 40;
        float *xd2 = nullptr, *od2 = nullptr;
        bool ok2 = mi_dev_malloc((void **)&xd2, sizeof(float) * T2 * D) == 0 &&
                   mi_dev_malloc((void **)&od2, sizeof(float) * T2 * D) == 0 &&
                   mi_moe_ctx_reserve(c, T2, D, I, E, K) == 0 &&
                   mi_fill_normal(c, xd2, (int64_t)T2 * D, 7, 5, 0.f, 1.f, s.stream()) == 0 &&
                   mi_moe_forward(c, &L, xd2, T2, xd2, od2, nullptr, s.stream()) == 0 && s.compute() == 0;
        std::vector<float> x2(T2 * D), want2(T2 * D), got2(T2 * D);
        ok2 = ok2 && mi_memcpy_d2h(x2.data(), xd2, sizeof(float) * T2 * D) == 0 &&
              mi_memcpy_d2h(want2.data(), od2, sizeof(float) * T2 * D) == 0;
        CHECK(ok2, "graphb tiled setup");
        vqa::moe::GraphB gbt(0, L, T2, true);
        CHECK(gbt.status() == 0 && gbt.feed(x2.data(), x2.data(), T2) == 0 && gbt.compute(got2.data()) == 0,
              "graphb tiled");
        CHECK(std::memcmp(got2.data(), want2.data(), sizeof(float) * T2 * D) == 0, "graphb tiled == mi_moe_forward");
        std::fprintf(stderr, "graphb q4_k layer with tiled copies, %d rows: %s mi_moe_forward\n", T2,
                     std::memcmp(got2.data(), want2.data(), sizeof(float) * T2 * D) ? "differs from" : "bit-identical to");
        for (void *p : {(void *)xd2, (void *)od2})
            if (p) mi_dev_free(p);
        for (void *p : {(void *)tmp, (void *)rw, (void *)xd, (void *)od, gq, dq})
            if (p) mi_dev_free(p);
    }
    std::fprintf(stderr, "%s (%d failures)\n", g_fail ? "FAIL" : "PASS", g_fail);
    return g_fail ? 1 : 0;
}
#endif
