// vqa_moe.hpp - C++ host mirror of the reference's routed-expert FFN segment,
// namespace vqa::moe (src/core/engine/moe_compute.hpp:25-86), running on the
// libmimoe C ABI (include/mi_moe.h) instead of ggml.
//
// Same names, argument meaning and error behaviour as the reference:
//   build_expert_ffn / _res            per-slot expert tensors (v1 form)
//   build_expert_ffn_table / _res      3D slot tables + I32 ids (v3 form)
// each returns the output tensor, or nullptr on bad arguments (the checks of
// moe_compute.cpp:43-58 and :102-122, in the same order).  ggml builds a graph
// and computes it later; here a Session stands in for the (ggml_context,
// ggml_cgraph) pair: it owns the tensors it creates and a stream, every build_*
// call enqueues its work on that stream at once, and compute() waits for it
// (the reference's ggml_backend_graph_compute).  Tensors are ggml-layout
// descriptors of device memory (ne fastest-first, nb in bytes).
//
// Restrictions against the reference (nullptr where they do not hold): x, res
// and w are F32 and contiguous; the v1 form's per-slot tensors share one type
// and shape (they are packed into a session-owned slot table); the v3 form's
// gate, up and down tables have the same slot count.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "mi_moe.h"
#include "mi_moe_util.h"

namespace vqa {
namespace moe {

// the ggml_unary_op values the reference's callers pass as `act`
enum class UnaryOp {
    SILU,       // GGML_UNARY_OP_SILU: swiglu_split(gate, up)
    GELU,       // GGML_UNARY_OP_GELU (tanh form): gelu(gate) * up
    GELU_ERF,   // GGML_UNARY_OP_GELU_ERF: gelu_erf(gate) * up
};

// ggml_tensor stand-in: device data, ggml type id (MI_TYPE_*), ne / nb
struct Tensor {
    void *data = nullptr;
    int type = MI_TYPE_F32;
    int64_t ne[4] = {1, 1, 1, 1};
    size_t nb[4] = {0, 0, 0, 0};
};

class Session {
public:
    explicit Session(int device = 0);
    ~Session();
    Session(const Session &) = delete;
    Session &operator=(const Session &) = delete;

    // 0, or the first negative mi_moe_status a call of this session returned
    int status() const { return status_; }
    // a new contiguous device tensor owned by the session (nullptr on failure)
    Tensor *new_tensor(int type, int64_t ne0, int64_t ne1 = 1, int64_t ne2 = 1);
    // host <-> device copies of a whole contiguous tensor (get waits for the stream)
    int set(Tensor *t, const void *host, size_t bytes);
    int get(const Tensor *t, void *host, size_t bytes);
    // wait for everything built so far (ggml_backend_graph_compute)
    int compute();

    mi_moe_ctx *ctx() const { return ctx_; }
    mi_stream_t stream() const { return stream_; }
    // record a failure; returns rc
    int fail(int rc);
    // grow the context's workspace to hold a call of these dims
    int ensure(int64_t T, int32_t D, int32_t I, int32_t E, int32_t K);

private:
    mi_moe_ctx *ctx_ = nullptr;
    mi_stream_t stream_ = nullptr;
    int status_ = 0;
    int64_t cap_T_ = 0;
    int32_t cap_D_ = 0, cap_I_ = 0, cap_E_ = 0, cap_K_ = 0;
    std::vector<Tensor *> owned_;
};

// out = res + sum_k w[k] * down_k(act(gate_k x, up_k x)); nullptr on bad args
Tensor *build_expert_ffn_res(Session &s, Tensor *x, Tensor *res, const std::vector<Tensor *> &gate,
                             const std::vector<Tensor *> &up, const std::vector<Tensor *> &down, Tensor *w,
                             UnaryOp act);
// the res = x case
Tensor *build_expert_ffn(Session &s, Tensor *x, const std::vector<Tensor *> &gate,
                         const std::vector<Tensor *> &up, const std::vector<Tensor *> &down, Tensor *w,
                         UnaryOp act = UnaryOp::SILU);
// slot-table form: tables [ne0, ne1, n_slots], ids I32 [n_used, T]
Tensor *build_expert_ffn_table_res(Session &s, Tensor *x, Tensor *res, Tensor *gate_table, Tensor *up_table,
                                   Tensor *down_table, Tensor *gate_up_ids, Tensor *down_ids, Tensor *w,
                                   UnaryOp act);
Tensor *build_expert_ffn_table(Session &s, Tensor *x, Tensor *gate_table, Tensor *up_table, Tensor *down_table,
                               Tensor *gate_up_ids, Tensor *down_ids, Tensor *w,
                               UnaryOp act = UnaryOp::SILU);

// The expert-cache decode driver's graph B on the GPU: the body a
// Hooks::build_b / feed_b pair runs (src/core/engine/moe_decode_driver.hpp:
// 125-144, called at :493-519; the driver's default build at :503-514).  Per
// layer and step the driver hands over the normed rows (moe_in), the residual
// rows (xmid_in), and either its routing (the K selected experts and weights
// of each row) or nothing (a model whose graph B routes moe_in itself,
// moondream.cpp:509-516); graph B returns hid = xmid + sum_k w_k down_k(act(
// gate_k moe_in, up_k moe_in)).  The layer's tables stay resident in HBM
// whole, so the driver's cache slots are plain expert ids here.
//   feed()     feed_b: uploads the rows (host memory) on this object's stream
//   compute()  the graph compute and readback of hid; waits on this object's
//              stream only (other streams of the GPU keep running)
// Not thread-safe (one GraphB per layer and driver thread, as the driver's
// per-layer graph state).
class GraphB {
public:
    // layer: device tables of one MoE layer (mi_gguf_load_moe_layer, or built
    // by the caller); max_tokens: rows per step; tiled: also make and attach
    // tiled copies of the tables that allow them (mi_moe_tile; owned by this
    // object, the output stays bit-identical)
    GraphB(int device, const mi_moe_layer &layer, int64_t max_tokens, bool tiled = false);
    ~GraphB();
    GraphB(const GraphB &) = delete;
    GraphB &operator=(const GraphB &) = delete;
    // 0, or the first negative mi_moe_status of a call
    int status() const { return status_; }
    // moe_in, xmid_in: host F32 [T][D]; ids (I32 [T][K], expert ids) and w
    // (F32 [T][K]) both given, or both nullptr (the layer's router)
    int feed(const float *moe_in, const float *xmid_in, int64_t T, const int32_t *ids = nullptr,
             const float *w = nullptr);
    // hid_out: host F32 [T][D] of the last feed()
    int compute(float *hid_out);
    mi_stream_t stream() const { return stream_; }

private:
    int fail(int rc);
    void attach_tiled();
    mi_moe_layer layer_{};
    std::vector<void *> tiled_;   // the tiled copies' device buffers
    mi_moe_ctx *ctx_ = nullptr;
    mi_stream_t stream_ = nullptr;
    int64_t cap_T_ = 0, T_ = 0;
    bool routed_ = false;
    float *d_in_ = nullptr, *d_xmid_ = nullptr, *d_out_ = nullptr, *d_w_ = nullptr;
    int32_t *d_ids_ = nullptr;
    int status_ = 0;
};

}  // namespace moe
}  // namespace vqa
