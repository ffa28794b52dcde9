// gguf.cpp - GGUF (versions 2 and 3) reader for the MoE block's tensors, the
// on-disk side of the path: the reference's converters write the experts as
// one 3D tensor per projection (convert/convert_hf_to_gguf.py:173-183 writes
// moondream3's fused [h | g] ffn_up_exps and ffn_down_exps;
// convert/convert_qwen3omni.py:188-219 writes qwen3omni's ffn_router,
// ffn_gate_exps, ffn_up_exps, ffn_down_exps), and moondream3 binds
// blk.N.ffn_gate_inp.{weight,bias} as the router (moondream.cpp:241-251),
// its F16 router promoted to F32 at load (moondream.cpp:149-172).
//
// The file is mapped read-only; every read is bounds-checked, so a truncated
// or malformed file gives MI_MOE_ERR_FORMAT instead of a read past the map.
// Layout read: magic "GGUF", u32 version, u64 tensor count, u64 metadata
// count; metadata (string key, u32 type, value; arrays as u32 element type,
// u64 count, elements); tensor infos (string name, u32 n_dims, u64 ne[n_dims],
// u32 ggml type, u64 offset); data from the first multiple of
// general.alignment (default 32) after the infos.
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/mi_moe.h"
#include "common.hpp"
#include "launch.hpp"

namespace {

struct TensorInfo {
    int32_t type = 0;
    int n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint64_t off = 0;
};

struct Cursor {
    const uint8_t *p, *end;
    bool ok = true;
    template <typename T>
    T get() {
        T v{};
        if (!ok || (size_t)(end - p) < sizeof(T)) {
            ok = false;
            return v;
        }
        std::memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!ok || (uint64_t)(end - p) < n) {
            ok = false;
            return {};
        }
        std::string s((const char *)p, (size_t)n);
        p += n;
        return s;
    }
    void skip(uint64_t n) {
        if (!ok || (uint64_t)(end - p) < n) {
            ok = false;
            return;
        }
        p += n;
    }
};

enum : uint32_t {
    GV_U8 = 0, GV_I8 = 1, GV_U16 = 2, GV_I16 = 3, GV_U32 = 4, GV_I32 = 5, GV_F32 = 6, GV_BOOL = 7,
    GV_STR = 8, GV_ARR = 9, GV_U64 = 10, GV_I64 = 11, GV_F64 = 12,
};

int scalar_bytes(uint32_t t) {
    switch (t) {
    case GV_U8: case GV_I8: case GV_BOOL: return 1;
    case GV_U16: case GV_I16: return 2;
    case GV_U32: case GV_I32: case GV_F32: return 4;
    case GV_U64: case GV_I64: case GV_F64: return 8;
    default: return 0;
    }
}

// bytes of a ggml tensor of these dims (F32, F16, I32, Q4_0, Q5_0, Q8_0, Q4_K, Q6_K), 0 if not
// one of them; UINT64_MAX if the product overflows (dims come from the file)
uint64_t tensor_bytes(int32_t type, const int64_t ne[4]) {
    for (int d = 0; d < 4; ++d)
        if (ne[d] < 1) return UINT64_MAX;
    if ((uint64_t)ne[0] > ((uint64_t)1 << 40)) return UINT64_MAX;
    const size_t row = type == MI_TYPE_I32 ? 4 * (size_t)ne[0] : mi_row_size(type, ne[0]);
    if (!row) return 0;
    uint64_t n = row;
    for (int d = 1; d < 4; ++d) {
        if ((uint64_t)ne[d] > UINT64_MAX / n) return UINT64_MAX;
        n *= (uint64_t)ne[d];
    }
    return n;
}

}  // namespace

struct mi_gguf {
    int fd = -1;
    uint8_t *map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint64_t data_off = 0;
    std::unordered_map<std::string, TensorInfo> tensors;
    std::unordered_map<std::string, uint64_t> ints;
    std::unordered_map<std::string, std::string> strs;
};

namespace {

int parse(mi_gguf *g) {
    Cursor c{g->map, g->map + g->size};
    const uint32_t magic = c.get<uint32_t>();
    if (!c.ok || std::memcmp(&magic, "GGUF", 4) != 0) return MI_MOE_ERR_FORMAT;
    g->version = c.get<uint32_t>();
    if (g->version != 2 && g->version != 3) return MI_MOE_ERR_FORMAT;
    const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    if (!c.ok || n_tensors > (1u << 24) || n_kv > (1u << 24)) return MI_MOE_ERR_FORMAT;
    uint64_t alignment = 32;
    for (uint64_t i = 0; i < n_kv && c.ok; ++i) {
        const std::string key = c.str();
        const uint32_t t = c.get<uint32_t>();
        if (t == GV_STR) {
            g->strs[key] = c.str();
        } else if (t == GV_ARR) {
            const uint32_t et = c.get<uint32_t>();
            const uint64_t n = c.get<uint64_t>();
            if (et == GV_STR) {
                for (uint64_t j = 0; j < n && c.ok; ++j) c.str();
            } else {
                const int b = scalar_bytes(et);
                if (!b || n > g->size) return MI_MOE_ERR_FORMAT;
                c.skip(n * (uint64_t)b);
            }
        } else {
            const int b = scalar_bytes(t);
            if (!b) return MI_MOE_ERR_FORMAT;
            uint64_t v = 0;
            switch (t) {
            case GV_U8: case GV_BOOL: v = c.get<uint8_t>(); break;
            case GV_I8: v = (uint64_t)(int64_t)c.get<int8_t>(); break;
            case GV_U16: v = c.get<uint16_t>(); break;
            case GV_I16: v = (uint64_t)(int64_t)c.get<int16_t>(); break;
            case GV_U32: v = c.get<uint32_t>(); break;
            case GV_I32: v = (uint64_t)(int64_t)c.get<int32_t>(); break;
            case GV_U64: v = c.get<uint64_t>(); break;
            case GV_I64: v = (uint64_t)c.get<int64_t>(); break;
            default: c.skip((uint64_t)b); continue;   // floats: not needed here
            }
            g->ints[key] = v;
        }
    }
    if (!c.ok) return MI_MOE_ERR_FORMAT;
    const auto al = g->ints.find("general.alignment");
    if (al != g->ints.end()) alignment = al->second;
    if (alignment == 0 || (alignment & (alignment - 1))) return MI_MOE_ERR_FORMAT;
    for (uint64_t i = 0; i < n_tensors && c.ok; ++i) {
        const std::string name = c.str();
        TensorInfo ti;
        ti.n_dims = (int)c.get<uint32_t>();
        if (ti.n_dims < 1 || ti.n_dims > 4) return MI_MOE_ERR_FORMAT;
        for (int d = 0; d < ti.n_dims; ++d) ti.ne[d] = (int64_t)c.get<uint64_t>();
        ti.type = (int32_t)c.get<uint32_t>();
        ti.off = c.get<uint64_t>();
        g->tensors[name] = ti;
    }
    if (!c.ok) return MI_MOE_ERR_FORMAT;
    const uint64_t info_end = (uint64_t)(c.p - g->map);
    g->data_off = (info_end + alignment - 1) / alignment * alignment;
    // every tensor of a known type must lie inside the file
    for (const auto &kv : g->tensors) {
        const uint64_t nb = tensor_bytes(kv.second.type, kv.second.ne);
        if (nb == UINT64_MAX) return MI_MOE_ERR_FORMAT;
        if (nb && (g->data_off > g->size || kv.second.off > g->size - g->data_off ||
                   nb > g->size - g->data_off - kv.second.off))
            return MI_MOE_ERR_FORMAT;
    }
    return MI_MOE_OK;
}

const TensorInfo *find(const mi_gguf *g, const std::string &name) {
    const auto it = g->tensors.find(name);
    return it == g->tensors.end() ? nullptr : &it->second;
}

std::string blk_name(int32_t blk, const char *leaf) {
    char b[128];
    std::snprintf(b, sizeof(b), "blk.%d.%s", (int)blk, leaf);
    return b;
}

float h2f_host(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
    uint32_t u;
    if (e == 0) {
        if (m == 0) {
            u = s;
        } else {   // subnormal: m * 2^-24
            float f = (float)m * 5.9604644775390625e-08f;
            std::memcpy(&u, &f, 4);
            u |= s;
        }
    } else if (e == 31) {
        u = s | 0x7f800000u | (m << 13);
    } else {
        u = s | ((e + 112) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

}  // namespace

extern "C" {

int mi_gguf_open(mi_gguf **out, const char *path) {
    if (!out || !path) return MI_MOE_ERR_NULL;
    *out = nullptr;
    mi_gguf *g = new mi_gguf;
    g->fd = ::open(path, O_RDONLY);
    struct stat st {};
    if (g->fd < 0 || fstat(g->fd, &st) != 0 || st.st_size < 24) {
        mi_gguf_close(g);
        return MI_MOE_ERR_FORMAT;
    }
    g->size = (size_t)st.st_size;
    void *m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) {
        mi_gguf_close(g);
        return MI_MOE_ERR_FORMAT;
    }
    g->map = (uint8_t *)m;
    const int rc = parse(g);
    if (rc) {
        mi_gguf_close(g);
        return rc;
    }
    *out = g;
    return MI_MOE_OK;
}

void mi_gguf_close(mi_gguf *g) {
    if (!g) return;
    if (g->map) munmap(g->map, g->size);
    if (g->fd >= 0) ::close(g->fd);
    delete g;
}

int mi_gguf_get_int(const mi_gguf *g, const char *key, int64_t *value) {
    if (!g || !key || !value) return MI_MOE_ERR_NULL;
    const auto it = g->ints.find(key);
    if (it == g->ints.end()) return MI_MOE_ERR_ARG;
    *value = (int64_t)it->second;
    return MI_MOE_OK;
}

int mi_gguf_tensor_info(const mi_gguf *g, const char *name, int32_t *type, int64_t ne[4], uint64_t *nbytes) {
    if (!g || !name) return MI_MOE_ERR_NULL;
    const TensorInfo *t = find(g, name);
    if (!t) return MI_MOE_ERR_ARG;
    if (type) *type = t->type;
    if (ne)
        for (int d = 0; d < 4; ++d) ne[d] = t->ne[d];
    if (nbytes) *nbytes = tensor_bytes(t->type, t->ne);
    return MI_MOE_OK;
}

int mi_gguf_load_moe_layer(const mi_gguf *g, int32_t blk, int32_t act, mi_moe_layer *layer, void **device_buffer) {
    if (!g || !layer || !device_buffer) return MI_MOE_ERR_NULL;
    *device_buffer = nullptr;
    if (act < MI_ACT_SILU || act > MI_ACT_GELU_ERF) return MI_MOE_ERR_ARG;
    const TensorInfo *rw = find(g, blk_name(blk, "ffn_gate_inp.weight"));
    const TensorInfo *rb = rw ? find(g, blk_name(blk, "ffn_gate_inp.bias")) : nullptr;
    if (!rw) rw = find(g, blk_name(blk, "ffn_router.weight"));
    const TensorInfo *gate = find(g, blk_name(blk, "ffn_gate_exps.weight"));
    const TensorInfo *up = find(g, blk_name(blk, "ffn_up_exps.weight"));
    const TensorInfo *down = find(g, blk_name(blk, "ffn_down_exps.weight"));
    if (!rw || !up || !down) return MI_MOE_ERR_ARG;
    const bool fused = gate == nullptr;
    // shapes: router [D, E]; up (fused [D, 2I, E] or [D, I, E]); down [I, D, E]
    const int64_t D = rw->ne[0], E = rw->ne[1], I = down->ne[0];
    if ((rw->type != MI_TYPE_F32 && rw->type != MI_TYPE_F16) || rw->ne[2] != 1) return MI_MOE_ERR_TYPE;
    if (rb && ((rb->type != MI_TYPE_F32 && rb->type != MI_TYPE_F16) || rb->ne[0] != E || rb->ne[1] != 1))
        return MI_MOE_ERR_SHAPE;
    if (up->ne[0] != D || up->ne[2] != E || up->ne[1] != (fused ? 2 * I : I)) return MI_MOE_ERR_SHAPE;
    if (!fused && (gate->ne[0] != D || gate->ne[1] != I || gate->ne[2] != E || gate->type != up->type))
        return MI_MOE_ERR_SHAPE;
    if (down->ne[1] != D || down->ne[2] != E) return MI_MOE_ERR_SHAPE;
    // expert tables as the converters write them: k-quants, the 32-value block
    // formats (Q8_0 by default, Q5_0, Q4_0), F16 or F32 (one family per layer:
    // the forward's validation refuses a mix)
    auto table_type = [](int32_t t) {
        return t == MI_TYPE_Q4_K || t == MI_TYPE_Q6_K || t == MI_TYPE_Q4_0 || t == MI_TYPE_Q5_0 ||
               t == MI_TYPE_Q8_0 || t == MI_TYPE_F16 || t == MI_TYPE_F32;
    };
    for (const TensorInfo *t : {up, down, fused ? up : gate})
        if (!table_type(t->type)) return MI_MOE_ERR_TYPE;
    int64_t K = 0;
    const auto arch = g->strs.find("general.architecture");
    if (arch == g->strs.end() || mi_gguf_get_int(g, (arch->second + ".expert_used_count").c_str(), &K) ||
        K <= 0 || K > E)
        return MI_MOE_ERR_FORMAT;
    if (D > INT32_MAX || E > INT32_MAX || I > INT32_MAX) return MI_MOE_ERR_SHAPE;

    // one device allocation: router F32, bias F32, gate, up, down (256-B aligned parts)
    auto al = [](uint64_t n) { return (n + 255) / 256 * 256; };
    const uint64_t b_rw = (uint64_t)D * E * 4, b_rb = rb ? (uint64_t)E * 4 : 0;
    const uint64_t b_gate = fused ? 0 : tensor_bytes(gate->type, gate->ne);
    const uint64_t b_up = tensor_bytes(up->type, up->ne), b_down = tensor_bytes(down->type, down->ne);
    if (!b_up || !b_down || (!fused && !b_gate)) return MI_MOE_ERR_SHAPE;   // k-quant rows not whole blocks
    const uint64_t total = al(b_rw) + al(b_rb) + al(b_gate) + al(b_up) + al(b_down);
    uint8_t *dev = nullptr;
    if (hipMalloc((void **)&dev, total) != hipSuccess) return MI_MOE_ERR_HIP;
    auto src = [&](const TensorInfo *t) { return g->map + g->data_off + t->off; };
    auto promote = [&](const TensorInfo *t, uint64_t n, uint8_t *dst) {
        if (t->type == MI_TYPE_F32) return hipMemcpy(dst, src(t), n * 4, hipMemcpyHostToDevice);
        std::vector<float> f(n);
        const uint8_t *s = src(t);
        for (uint64_t i = 0; i < n; ++i) {
            uint16_t h;
            std::memcpy(&h, s + 2 * i, 2);
            f[i] = h2f_host(h);
        }
        return hipMemcpy(dst, f.data(), n * 4, hipMemcpyHostToDevice);
    };
    uint8_t *p = dev;
    uint8_t *d_rw = p; p += al(b_rw);
    uint8_t *d_rb = rb ? p : nullptr; p += al(b_rb);
    uint8_t *d_gate = fused ? nullptr : p; p += al(b_gate);
    uint8_t *d_up = p; p += al(b_up);
    uint8_t *d_down = p;
    hipError_t e = promote(rw, (uint64_t)D * E, d_rw);
    if (e == hipSuccess && rb) e = promote(rb, (uint64_t)E, d_rb);
    if (e == hipSuccess && !fused) e = hipMemcpy(d_gate, src(gate), b_gate, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(d_up, src(up), b_up, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(d_down, src(down), b_down, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(dev);
        return MI_MOE_ERR_HIP;
    }
    auto desc = [](const TensorInfo *t, uint8_t *data) {
        mi_tensor m{};
        m.data = data;
        m.type = t->type;
        const size_t row = mi_row_size(t->type, t->ne[0]);
        for (int d = 0; d < 4; ++d) m.ne[d] = t->ne[d];
        switch (t->type) {
        case MI_TYPE_F32: m.nb[0] = 4; break;
        case MI_TYPE_F16: m.nb[0] = 2; break;
        case MI_TYPE_Q4_K: case MI_TYPE_Q6_K: m.nb[0] = row / (size_t)(t->ne[0] / 256); break;
        default: m.nb[0] = row / (size_t)(t->ne[0] / 32); break;   // 32-value blocks
        }
        m.nb[1] = row;
        m.nb[2] = row * (size_t)t->ne[1];
        m.nb[3] = m.nb[2] * (size_t)t->ne[2];
        return m;
    };
    mi_moe_layer L{};
    L.n_embd = (int32_t)D;
    L.n_expert = (int32_t)E;
    L.n_expert_used = (int32_t)K;
    L.n_ff = (int32_t)I;
    L.router_w = (const float *)d_rw;
    L.router_b = (const float *)d_rb;
    L.gate = desc(fused ? up : gate, fused ? d_up : d_gate);
    if (!fused) L.up = desc(up, d_up);
    L.down = desc(down, d_down);
    L.fused_gate_up = fused ? 1 : 0;
    L.act = act;
    L.gating = MI_GATING_SOFTMAX_TOPK;
    *layer = L;
    *device_buffer = dev;
    return MI_MOE_OK;
}

}  // extern "C"
