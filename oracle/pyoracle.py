"""ctypes wrapper around oracle/_build/liboracle.so.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker (or the timed CPU
baseline), never as the thing measured or shipped.  The product library under
skyvision.cpp_amd/ never loads this.
"""
from __future__ import annotations

import ctypes as C
import os
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"

TYPE_F32, TYPE_F16, TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_K, TYPE_I32 = 0, 1, 12, 14, 15, 26
TYPE_Q4_0, TYPE_Q5_0, TYPE_Q8_0 = 2, 6, 8
ACT_SILU, ACT_GELU_ERF_GP1, ACT_GELU_TANH, ACT_GELU_ERF = 0, 1, 2, 3
QK_K = 256
QK32 = 32
BLOCK_BYTES = {TYPE_Q4_K: 144, TYPE_Q6_K: 210, TYPE_Q8_K: 292, TYPE_Q4_0: 18, TYPE_Q5_0: 22, TYPE_Q8_0: 34}
B32_TYPES = (TYPE_Q4_0, TYPE_Q5_0, TYPE_Q8_0)


def block_values(type_: int) -> int:
    """values per block of a quantized type (1 for F32 / F16)"""
    return QK32 if type_ in B32_TYPES else QK_K if type_ in (TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_K) else 1

_lib = None


def build() -> None:
    """Compile the oracle (make -C oracle)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = C.CDLL(str(LIB_PATH))
        _declare(_lib)
    return _lib


P = C.c_void_p
i64 = C.c_int64


def _declare(L: C.CDLL) -> None:
    L.orc_fp16_to_fp32.argtypes = [C.c_uint16]
    L.orc_fp16_to_fp32.restype = C.c_float
    L.orc_fp32_to_fp16.argtypes = [C.c_float]
    L.orc_fp32_to_fp16.restype = C.c_uint16
    L.orc_nearest_int.argtypes = [C.c_float]
    L.orc_nearest_int.restype = C.c_int
    L.orc_quantize_row_q4_K.argtypes = [P, P, i64]
    L.orc_quantize_row_q4_K_port.argtypes = [P, P, i64, C.c_int]
    L.orc_quantize_row_q6_K.argtypes = [P, P, i64, C.c_int]
    L.orc_quantize_row_q8_K.argtypes = [P, P, i64]
    L.orc_quantize_rows.argtypes = [C.c_int, P, P, i64, i64, C.c_int]
    for n in ("q4_K", "q6_K", "q8_K", "q4_0", "q5_0", "q8_0"):
        getattr(L, f"orc_dequantize_row_{n}").argtypes = [P, P, i64]
    for n in ("q4_0", "q5_0", "q8_0"):
        getattr(L, f"orc_quantize_row_{n}").argtypes = [P, P, i64]
        getattr(L, f"orc_vec_dot_{n}_q8_0").argtypes = [C.c_int, P, P]
        getattr(L, f"orc_vec_dot_{n}_q8_0").restype = C.c_float
    L.orc_vec_dot_f16.argtypes = [C.c_int, P, P]
    L.orc_vec_dot_f16.restype = C.c_float
    L.orc_vec_dot_kq_simd.argtypes = [C.c_int, C.c_int, P, P]
    L.orc_vec_dot_kq_simd.restype = C.c_float
    L.orc_set_simd.argtypes = [C.c_int]
    L.orc_set_simd.restype = C.c_int
    L.orc_row_size.argtypes = [C.c_int, i64]
    L.orc_row_size.restype = C.c_size_t
    L.orc_vec_dot_q4_K_q8_K.argtypes = [C.c_int, P, P]
    L.orc_vec_dot_q4_K_q8_K.restype = C.c_float
    L.orc_vec_dot_q6_K_q8_K.argtypes = [C.c_int, P, P]
    L.orc_vec_dot_q6_K_q8_K.restype = C.c_float
    L.orc_rng_u64.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64]
    L.orc_rng_u64.restype = C.c_uint64
    L.orc_fill_normal.argtypes = [P, i64, C.c_uint64, C.c_uint64, C.c_float, C.c_float, C.c_int]
    L.orc_poly_log.argtypes = [C.c_double]
    L.orc_poly_log.restype = C.c_double
    L.orc_poly_sincos_2pi.argtypes = [C.c_double, P, P]
    L.orc_router_logits.argtypes = [P, P, P, i64, C.c_int, C.c_int, P, C.c_int]
    L.orc_top_k.argtypes = [P, i64, C.c_int, C.c_int, P]
    L.orc_softmax_selected.argtypes = [P, P, i64, C.c_int, C.c_int, P]
    L.orc_route_gated.argtypes = [P, i64, C.c_int, C.c_int, C.c_int, P, P, C.c_float, C.c_float, P, P]
    L.orc_dispatch.argtypes = [P, i64, C.c_int, C.c_int, P, P, P]
    L.orc_mul_mat_id.argtypes = [C.c_int, P, i64, i64, C.c_int, P, C.c_int, P, C.c_int, i64, P,
                                 C.c_int, C.c_int]
    L.orc_mul_mat_id.restype = C.c_int
    L.orc_act_pair.argtypes = [C.c_int, C.c_float, C.c_float]
    L.orc_act_pair.restype = C.c_float
    L.orc_moe_forward.argtypes = [P, P, i64, P, P, P, P, P, P, C.c_int, C.c_int]
    L.orc_moe_forward.restype = C.c_int
    L.orc_max_threads.restype = C.c_int


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ----------------------------------------------------------------- formats
def fp16_to_fp32(h: int) -> float:
    return lib().orc_fp16_to_fp32(h)


def fp32_to_fp16(f: float) -> int:
    return lib().orc_fp32_to_fp16(f)


def nearest_int(f: float) -> int:
    return lib().orc_nearest_int(f)


def row_size(type_: int, k: int) -> int:
    return lib().orc_row_size(type_, k)


PORT_FP32_D, PORT_ZERO_L, PORT_FIXED_SPAN = 1, 2, 4


def quantize(type_: int, x: np.ndarray, nthreads: int = 0, requant_fp32_d: bool = False,
             port: int = 0) -> np.ndarray:
    """x float32 [..., k] (k % 256 == 0) -> uint8 [..., row_size].  port: the
    reference Python ports' conventions (PORT_* bits), golden comparison only"""
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    assert k % block_values(type_) == 0
    rows = x.reshape(-1, k)
    rs = row_size(type_, k)
    out = np.zeros((rows.shape[0], rs), dtype=np.uint8)
    if requant_fp32_d:
        port |= PORT_FP32_D
    if port and type_ == TYPE_Q6_K:
        for r in range(rows.shape[0]):
            lib().orc_quantize_row_q6_K(_p(rows[r]), _p(out[r]), k, port)
    elif port and type_ == TYPE_Q4_K:
        for r in range(rows.shape[0]):
            lib().orc_quantize_row_q4_K_port(_p(rows[r]), _p(out[r]), k, port)
    else:
        lib().orc_quantize_rows(type_, _p(rows), _p(out), rows.shape[0], k, nthreads)
    return out.reshape(*x.shape[:-1], rs)


def dequantize(type_: int, q: np.ndarray, k: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    rs = row_size(type_, k)
    rows = q.reshape(-1, rs)
    out = np.zeros((rows.shape[0], k), dtype=np.float32)
    if type_ == TYPE_F16:
        return rows.view(np.float16).astype(np.float32).reshape(*q.shape[:-1], k)
    fn = {TYPE_Q4_K: lib().orc_dequantize_row_q4_K, TYPE_Q6_K: lib().orc_dequantize_row_q6_K,
          TYPE_Q8_K: lib().orc_dequantize_row_q8_K, TYPE_Q4_0: lib().orc_dequantize_row_q4_0,
          TYPE_Q5_0: lib().orc_dequantize_row_q5_0, TYPE_Q8_0: lib().orc_dequantize_row_q8_0}[type_]
    for r in range(rows.shape[0]):
        fn(_p(rows[r]), _p(out[r]), k)
    return out.reshape(*q.shape[:-1], k)


def vec_dot(type_: int, wrow: np.ndarray, q8row: np.ndarray, k: int) -> float:
    """ggml's dot of one weight row with one activation row in the type's
    vec_dot_type (Q8_K bytes for k-quants, Q8_0 bytes for 32-value formats,
    fp16 values for F16)"""
    fn = {TYPE_Q4_K: lib().orc_vec_dot_q4_K_q8_K, TYPE_Q6_K: lib().orc_vec_dot_q6_K_q8_K,
          TYPE_Q4_0: lib().orc_vec_dot_q4_0_q8_0, TYPE_Q5_0: lib().orc_vec_dot_q5_0_q8_0,
          TYPE_Q8_0: lib().orc_vec_dot_q8_0_q8_0, TYPE_F16: lib().orc_vec_dot_f16}[type_]
    return fn(k, _p(np.ascontiguousarray(wrow)), _p(np.ascontiguousarray(q8row)))


def vec_dot_simd(type_: int, wrow: np.ndarray, q8row: np.ndarray, k: int) -> float:
    """the AVX-512 VNNI form of the Q4_K / Q6_K x Q8_K dot (the scalar form
    where the host lacks AVX-512 VNNI)"""
    return lib().orc_vec_dot_kq_simd(type_, k, _p(np.ascontiguousarray(wrow)), _p(np.ascontiguousarray(q8row)))


def set_simd(on: bool) -> bool:
    """mul_mat_id's k-quant dots on the AVX-512 VNNI forms (bit for bit the
    scalar ones); returns whether they are in use on this host"""
    return bool(lib().orc_set_simd(int(on)))


def host_has_avx512_vnni() -> bool:
    on = set_simd(True)
    set_simd(False)
    return on


# ----------------------------------------------------------------- data
def fill_normal(n: int, seed: int, stream: int, mean: float = 0.0, std: float = 1.0,
                nthreads: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_normal(_p(out), n, seed, stream, mean, std, nthreads)
    return out


def rng_u64(seed: int, stream: int, i: int) -> int:
    return lib().orc_rng_u64(seed, stream, i)


def poly_log(x: float) -> float:
    return lib().orc_poly_log(x)


def poly_sincos_2pi(u: float):
    s, c = C.c_double(), C.c_double()
    lib().orc_poly_sincos_2pi(u, C.byref(s), C.byref(c))
    return s.value, c.value


# ----------------------------------------------------------------- routing
def router_logits(W: np.ndarray, b, x: np.ndarray, nthreads: int = 0) -> np.ndarray:
    W = np.ascontiguousarray(W, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    E, D = W.shape
    T = x.shape[0]
    out = np.zeros((T, E), dtype=np.float32)
    bb = None if b is None else np.ascontiguousarray(b, dtype=np.float32)
    lib().orc_router_logits(_p(W), _p(bb), _p(x), T, D, E, _p(out), nthreads)
    return out


def top_k(logits: np.ndarray, K: int) -> np.ndarray:
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = logits.shape
    sel = np.zeros((T, K), dtype=np.int32)
    lib().orc_top_k(_p(logits), T, E, K, _p(sel))
    return sel


def softmax_selected(logits: np.ndarray, sel: np.ndarray) -> np.ndarray:
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    sel = np.ascontiguousarray(sel, dtype=np.int32)
    T, E = logits.shape
    K = sel.shape[1]
    w = np.zeros((T, K), dtype=np.float32)
    lib().orc_softmax_selected(_p(logits), _p(sel), T, E, K, _p(w))
    return w


def route_gated(logits: np.ndarray, K: int, kind: int, sel_bias=None, expert_scale=None, scaling: float = 1.0,
                eps: float = 0.0):
    """Router gating variants (moe_oracle.c orc_route_gated): (sel, w)."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = logits.shape
    sel = np.zeros((T, K), dtype=np.int32)
    w = np.zeros((T, K), dtype=np.float32)
    sb = None if sel_bias is None else np.ascontiguousarray(sel_bias, dtype=np.float32)
    es = None if expert_scale is None else np.ascontiguousarray(expert_scale, dtype=np.float32)
    lib().orc_route_gated(_p(logits), T, E, K, kind, _p(sb), _p(es), scaling, eps, _p(sel), _p(w))
    return sel, w


def dispatch(sel: np.ndarray, E: int):
    sel = np.ascontiguousarray(sel, dtype=np.int32)
    T, K = sel.shape
    counts = np.zeros(E, dtype=np.int32)
    offsets = np.zeros(E + 1, dtype=np.int32)
    perm = np.zeros(T * K, dtype=np.int32)
    lib().orc_dispatch(_p(sel), T, K, E, _p(counts), _p(offsets), _p(perm))
    return counts, offsets, perm


def mul_mat_id(type_: int, as_: np.ndarray, Kin: int, N: int, E: int, b: np.ndarray,
               ids: np.ndarray, exact: bool = False, nthreads: int = 0) -> np.ndarray:
    """as_: bytes/floats of E x N rows; b: float32 [T, ne11, Kin]; ids int32 [T, n_used]"""
    b = np.ascontiguousarray(b, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    T, n_used = ids.shape
    ne11 = b.shape[1]
    dst = np.zeros((T, n_used, N), dtype=np.float32)
    rc = lib().orc_mul_mat_id(type_, _p(np.ascontiguousarray(as_)), Kin, N, E, _p(b), ne11,
                              _p(ids), n_used, T, _p(dst), int(exact), nthreads)
    if rc != 0:
        raise ValueError("orc_mul_mat_id: bad arguments")
    return dst


def act_pair(act: int, a: float, b: float) -> float:
    return lib().orc_act_pair(act, a, b)


# ----------------------------------------------------------------- layer
class _Layer(C.Structure):
    _fields_ = [("D", C.c_int32), ("E", C.c_int32), ("K", C.c_int32), ("I", C.c_int32),
                ("router_w", P), ("router_b", P),
                ("gate_type", C.c_int32), ("gate", P), ("up", P), ("fused_gate_up", C.c_int32),
                ("down_type", C.c_int32), ("down", P), ("act", C.c_int32),
                ("gating", C.c_int32), ("sel_bias", P), ("expert_scale", P),
                ("routed_scaling", C.c_float), ("gate_eps", C.c_float),
                ("sh_I", C.c_int32), ("sh_act", C.c_int32), ("sh_type", C.c_int32), ("sh_gate", P),
                ("sh_up", P), ("sh_down_type", C.c_int32), ("sh_down", P), ("sh_gate_inp", P)]


class _Debug(C.Structure):
    _fields_ = [("logits", P), ("sel", P), ("w", P), ("counts", P), ("offsets", P),
                ("perm", P), ("act", P), ("ff", P), ("sh", P)]


ACT_RELU_SQR = 4
GATING_SOFTMAX_TOPK, GATING_SIGMOID_BIAS, GATING_SOFTMAX_ALL = 0, 1, 2


def moe_forward(layer: dict, x: np.ndarray, res=None, exact: bool = False,
                sel_in=None, w_in=None, nthreads: int = 0, debug: bool = True, down_sel_in=None):
    """layer: dict(D, E, K, I, router_w, router_b, gate_type, gate, up, fused,
    down_type, down, act) and optionally the gating (gating, sel_bias,
    expert_scale, routed_scaling, gate_eps) and a shared expert (sh_I, sh_act,
    sh_type, sh_gate, sh_up, sh_down_type, sh_down, sh_gate_inp).
    sel_in / w_in: caller routing (down_sel_in: separate down ids).
    Returns (out, dbg dict)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, D = x.shape
    E, K, I = layer["E"], layer["K"], layer["I"]
    keep = []

    def arr(a, dt=None):
        if a is None:
            return None
        a = np.ascontiguousarray(a if dt is None else a.astype(dt, copy=False))
        keep.append(a)
        return a

    L = _Layer()
    L.D, L.E, L.K, L.I = D, E, K, I
    L.router_w = _p(arr(layer.get("router_w"), np.float32))
    L.router_b = _p(arr(layer.get("router_b"), np.float32))
    L.gate_type = layer["gate_type"]
    L.gate = _p(arr(layer["gate"]))
    L.up = _p(arr(layer.get("up")))
    L.fused_gate_up = int(layer.get("fused", False))
    L.down_type = layer["down_type"]
    L.down = _p(arr(layer["down"]))
    L.act = layer["act"]
    L.gating = int(layer.get("gating", 0))
    L.sel_bias = _p(arr(layer.get("sel_bias"), np.float32))
    L.expert_scale = _p(arr(layer.get("expert_scale"), np.float32))
    L.routed_scaling = float(layer.get("routed_scaling", 0.0))
    L.gate_eps = float(layer.get("gate_eps", 0.0))
    L.sh_I = int(layer.get("sh_I", 0))
    if L.sh_I:
        L.sh_act = layer["sh_act"]
        L.sh_type = layer["sh_type"]
        L.sh_gate = _p(arr(layer["sh_gate"]))
        L.sh_up = _p(arr(layer.get("sh_up")))
        L.sh_down_type = layer["sh_down_type"]
        L.sh_down = _p(arr(layer["sh_down"]))
        L.sh_gate_inp = _p(arr(layer.get("sh_gate_inp"), np.float32))
    out = np.zeros((T, D), dtype=np.float32)
    dbg = None
    d = {}
    if debug:
        d = dict(logits=np.zeros((T, E), np.float32), sel=np.zeros((T, K), np.int32),
                 w=np.zeros((T, K), np.float32), counts=np.zeros(E, np.int32),
                 offsets=np.zeros(E + 1, np.int32), perm=np.zeros(T * K, np.int32),
                 act=np.zeros((T, K, I), np.float32), ff=np.zeros((T, K, D), np.float32),
                 sh=np.zeros((T, D), np.float32))
        dbg = _Debug(*[_p(d[f]) for f, _ in _Debug._fields_])
    rres = arr(res, np.float32)
    s_in = arr(sel_in, np.int32)
    w_in_ = arr(w_in, np.float32)
    ds_in = arr(down_sel_in, np.int32)
    rc = lib().orc_moe_forward(C.byref(L), _p(x), T, _p(rres), _p(out),
                               C.byref(dbg) if dbg is not None else None,
                               _p(s_in), _p(ds_in), _p(w_in_), int(exact), nthreads)
    if rc != 0:
        raise ValueError("orc_moe_forward: bad arguments")
    return out, d


def max_threads() -> int:
    return lib().orc_max_threads()


def physical_cores() -> int:
    """Physical core count (one thread per core), counted like the reference's
    backend.cpp:53-82: distinct (physical id, core id) pairs in /proc/cpuinfo,
    limited to this process's CPU affinity."""
    try:
        allowed = os.sched_getaffinity(0)
    except AttributeError:
        allowed = set(range(os.cpu_count() or 1))
    cores = set()
    try:
        cur = {}
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    if "processor" in cur and int(cur["processor"]) in allowed:
                        cores.add((cur.get("physical id", "0"), cur.get("core id", cur["processor"])))
                    cur = {}
                    continue
                k, _, v = line.partition(":")
                cur[k.strip()] = v.strip()
        if "processor" in cur and int(cur["processor"]) in allowed:
            cores.add((cur.get("physical id", "0"), cur.get("core id", cur["processor"])))
    except OSError:
        pass
    return max(1, len(cores) if cores else len(allowed))
