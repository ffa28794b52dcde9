"""ctypes binding of libmimoe.so (include/mi_moe.h, include/mi_moe_util.h).

Plumbing for Python callers (tests, bench.py): device buffers, copies, streams
and the MoE entry points.  There is no compute here and no fallback: if the
HIP library is missing or fails to load, every call raises.
"""
from __future__ import annotations

import ctypes as C
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "libmimoe.so"

DECODE_CHAIN, DECODE_FUSED_COOPERATIVE, DECODE_FUSED = 0, 1, 2
DECODE_FUSED_EXCLUSIVE = DECODE_FUSED   # former name

TYPE_F32, TYPE_F16, TYPE_Q4_K, TYPE_Q6_K, TYPE_I32 = 0, 1, 12, 14, 26
TYPE_Q4_0, TYPE_Q5_0, TYPE_Q8_0 = 2, 6, 8
ACT_SILU, ACT_GELU_ERF_GP1, ACT_GELU_TANH, ACT_GELU_ERF, ACT_RELU_SQR = 0, 1, 2, 3, 4
NORM_NONE, NORM_RMS, NORM_LAYER = 0, 1, 2
GATING_SOFTMAX_TOPK, GATING_SIGMOID_BIAS, GATING_SOFTMAX_ALL = 0, 1, 2
ABI_VERSION = 3
# mi_moe_status
OK, ERR_NULL, ERR_SHAPE, ERR_TYPE, ERR_CAPACITY, ERR_HIP = 0, -1, -2, -3, -4, -5
ERR_UNSUPPORTED, ERR_DEVICE, ERR_ARG, ERR_FORMAT = -6, -7, -8, -9
QK_K = 256
BLOCK_BYTES = {TYPE_Q4_K: 144, TYPE_Q6_K: 210, TYPE_Q4_0: 18, TYPE_Q5_0: 22, TYPE_Q8_0: 34}
STATUS = {0: "ok", -1: "null", -2: "shape", -3: "type", -4: "capacity", -5: "hip",
          -6: "unsupported", -7: "device", -8: "arg"}

_lib = None


class MimoeError(RuntimeError):
    def __init__(self, fn: str, rc: int):
        self.rc = rc
        extra = ""
        if rc == -5 and _lib is not None:
            extra = ": " + _lib.mi_last_hip_error().decode(errors="replace")
        super().__init__(f"{fn} failed with {rc} ({STATUS.get(rc, '?')}){extra}")


P = C.c_void_p
i64 = C.c_int64
i32 = C.c_int32


class Tensor(C.Structure):
    _fields_ = [("data", P), ("type", i32), ("ne", i64 * 4), ("nb", C.c_size_t * 4)]


class Layer(C.Structure):
    _fields_ = [("n_embd", i32), ("n_expert", i32), ("n_expert_used", i32), ("n_ff", i32),
                ("router_w", P), ("router_b", P), ("gate", Tensor), ("up", Tensor),
                ("down", Tensor), ("fused_gate_up", i32), ("act", i32), ("gating", i32),
                ("sel_bias", P), ("expert_scale", P), ("routed_scaling", C.c_float), ("gate_eps", C.c_float),
                ("sh_n_ff", i32), ("sh_act", i32), ("sh_gate", Tensor), ("sh_up", Tensor), ("sh_down", Tensor),
                ("sh_gate_inp", P), ("gate_tiled", Tensor), ("up_tiled", Tensor), ("down_tiled", Tensor)]


class Norm(C.Structure):
    _fields_ = [("kind", C.c_int32), ("eps", C.c_float), ("weight", C.c_void_p), ("bias", C.c_void_p)]


def make_norm(kind: int, eps: float, weight=None, bias=None) -> Norm:
    """weight / bias: DeviceBuffer (kept alive by the returned Norm) or a
    device address."""
    n = Norm()
    n.kind, n.eps = kind, eps
    n.weight = weight.addr if isinstance(weight, DeviceBuffer) else weight
    n.bias = bias.addr if isinstance(bias, DeviceBuffer) else bias
    n._buffers = (weight, bias)
    return n


class Routing(C.Structure):
    _fields_ = [("logits", P), ("sel", P), ("weights", P), ("counts", P), ("offsets", P),
                ("perm", P)]


SYMBOLS = {
    # mi_moe.h
    "mi_moe_ctx_create": ([C.POINTER(P), C.c_int], C.c_int),
    "mi_moe_ctx_destroy": ([P], None),
    "mi_moe_ctx_reserve": ([P, i64, i32, i32, i32, i32], C.c_int),
    "mi_moe_ctx_take_errors": ([P, C.POINTER(i64), C.POINTER(i64), C.POINTER(i64)], C.c_int),
    "mi_moe_forward": ([P, C.POINTER(Layer), P, i64, P, P, C.POINTER(Routing), P], C.c_int),
    "mi_moe_forward_noalloc": ([C.POINTER(Layer), P, i64, P, P, C.POINTER(Routing), P], C.c_int),
    "mi_moe_forward_router_input": ([P, C.POINTER(Layer), P, P, i64, P, P, C.POINTER(Routing), P], C.c_int),
    "mi_moe_expert_ffn": ([P, C.POINTER(Layer), P, i64, P, P, P, P, P, P], C.c_int),
    "mi_top_k": ([P, C.POINTER(Tensor), i32, C.POINTER(Tensor), P], C.c_int),
    "mi_mul_mat_id": ([P, C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Tensor),
                       C.POINTER(Tensor), P], C.c_int),
    "mi_quantize": ([P, i32, P, P, i64, i64, P], C.c_int),
    "mi_moe_tiled_bytes": ([C.POINTER(Tensor)], i64),
    "mi_moe_tile": ([P, C.POINTER(Tensor), P, C.POINTER(Tensor), P], C.c_int),
    "mi_fill_normal": ([P, P, i64, C.c_uint64, C.c_uint64, C.c_float, C.c_float, P], C.c_int),
    "mi_rmsnorm": ([P, P, i64, C.c_int32, C.c_float, P, P], C.c_int),
    "mi_norm": ([P, C.POINTER(Norm), P, i64, C.c_int32, P, P], C.c_int),
    "mi_moe_forward_norm": ([P, C.POINTER(Layer), C.POINTER(Norm), P, i64, P, P, C.POINTER(Routing), P],
                            C.c_int),
    "mi_moe_ctx_set_profiling": ([P, C.c_int], C.c_int),
    "mi_moe_ctx_stage_clock": ([P, C.c_char_p, C.POINTER(C.c_double), C.POINTER(C.c_int)], C.c_int),
    "mi_moe_ctx_stage_times": ([P, C.c_int, C.POINTER(C.c_char_p), C.POINTER(C.c_float),
                                C.POINTER(C.c_int)], C.c_int),
    "mi_moe_ctx_set_gemm_threshold": ([P, i64], C.c_int),
    "mi_moe_ctx_set_gemm_tiles": ([P, C.c_int], C.c_int),
    "mi_moe_ctx_set_fused_decode": ([P, C.c_int], C.c_int),
    "mi_moe_ctx_set_decode_rescue": ([P, C.c_int], C.c_int),
    "mi_row_size": ([i32, i64], C.c_size_t),
    "mi_moe_status_string": ([C.c_int], C.c_char_p),
    "mi_moe_abi_version": ([], C.c_int),
    # mi_moe_util.h
    "mi_device_count": ([C.POINTER(C.c_int)], C.c_int),
    "mi_set_device": ([C.c_int], C.c_int),
    "mi_device_info": ([C.c_int, C.c_char_p, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int),
                        C.c_char_p, C.c_int], C.c_int),
    "mi_dev_malloc": ([C.POINTER(P), C.c_size_t], C.c_int),
    "mi_dev_free": ([P], C.c_int),
    "mi_memcpy_h2d": ([P, P, C.c_size_t], C.c_int),
    "mi_memcpy_d2h": ([P, P, C.c_size_t], C.c_int),
    "mi_memcpy_d2d": ([P, P, C.c_size_t], C.c_int),
    "mi_memset_d": ([P, C.c_int, C.c_size_t], C.c_int),
    "mi_device_synchronize": ([], C.c_int),
    "mi_stream_create": ([C.POINTER(P)], C.c_int),
    "mi_stream_destroy": ([P], C.c_int),
    "mi_stream_synchronize": ([P], C.c_int),
    "mi_event_create": ([C.POINTER(P)], C.c_int),
    "mi_event_destroy": ([P], C.c_int),
    "mi_event_record": ([P, P], C.c_int),
    "mi_event_synchronize": ([P], C.c_int),
    "mi_event_elapsed_ms": ([C.POINTER(C.c_float), P, P], C.c_int),
    "mi_last_hip_error": ([], C.c_char_p),
    "mi_gguf_open": ([C.POINTER(P), C.c_char_p], C.c_int),
    "mi_gguf_close": ([P], None),
    "mi_gguf_get_int": ([P, C.c_char_p, C.POINTER(i64)], C.c_int),
    "mi_gguf_tensor_info": ([P, C.c_char_p, C.POINTER(C.c_int32), C.POINTER(i64), C.POINTER(C.c_uint64)], C.c_int),
    "mi_gguf_load_moe_layer": ([P, C.c_int32, C.c_int32, C.POINTER(Layer), C.POINTER(P)], C.c_int),
    "mi_stream_begin_capture": ([P], C.c_int),
    "mi_stream_end_capture": ([P, C.POINTER(P)], C.c_int),
    "mi_graph_launch": ([P, P], C.c_int),
    "mi_graph_destroy": ([P], C.c_int),
}


def load(path: str | None = None) -> C.CDLL:
    """Load the in-tree HIP library (raises if it is not built)."""
    global _lib
    if _lib is None:
        p = pathlib.Path(path) if path else LIB_PATH
        if not p.exists():
            raise FileNotFoundError(f"{p} not built: run __graft_entry__.build()")
        lib = C.CDLL(str(p))
        for name, (args, res) in SYMBOLS.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        if lib.mi_moe_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{p}: ABI {lib.mi_moe_abi_version()}, binding expects {ABI_VERSION}: rebuild")
        _lib = lib
    return _lib


def check(fn: str, rc: int) -> None:
    if rc != 0:
        raise MimoeError(fn, rc)


def call(name: str, *args) -> int:
    rc = getattr(load(), name)(*args)
    check(name, rc)
    return rc


def device_count() -> int:
    n = C.c_int(0)
    rc = load().mi_device_count(C.byref(n))
    return n.value if rc == 0 else 0


def device_info(dev: int = 0) -> dict:
    name = C.create_string_buffer(256)
    arch = C.create_string_buffer(256)
    cu, clk = C.c_int(), C.c_int()
    call("mi_device_info", dev, name, 256, C.byref(cu), C.byref(clk), arch, 256)
    return {"name": name.value.decode(), "arch": arch.value.decode(), "cu": cu.value,
            "clock_khz": clk.value}


def row_size(type_: int, n: int) -> int:
    return load().mi_row_size(type_, n)


# ------------------------------------------------------------------ buffers
class DeviceBuffer:
    """Owned device allocation."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = P()
        call("mi_dev_malloc", C.byref(self.ptr), max(1, self.nbytes))

    @property
    def addr(self) -> int:
        return self.ptr.value or 0

    def upload(self, a: np.ndarray, offset: int = 0) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        call("mi_memcpy_h2d", P(self.addr + offset), a.ctypes.data_as(P), a.nbytes)
        return self

    def download(self, dtype, shape, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        call("mi_memcpy_d2h", out.ctypes.data_as(P), P(self.addr + offset), out.nbytes)
        return out

    def zero(self) -> "DeviceBuffer":
        call("mi_memset_d", self.ptr, 0, self.nbytes)
        return self

    def free(self) -> None:
        if self.ptr and self.ptr.value:
            load().mi_dev_free(self.ptr)
            self.ptr = P()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def to_device(a: np.ndarray) -> DeviceBuffer:
    a = np.ascontiguousarray(a)
    return DeviceBuffer(a.nbytes).upload(a)


def synchronize() -> None:
    call("mi_device_synchronize")


def tensor(buf, type_: int, ne, nb=None, offset: int = 0) -> Tensor:
    """ggml-style descriptor; default strides are ggml's contiguous ones."""
    ne = list(ne) + [1] * (4 - len(ne))
    if nb is None:
        if type_ in (TYPE_Q4_K, TYPE_Q6_K, TYPE_Q4_0, TYPE_Q5_0, TYPE_Q8_0):
            nb0 = BLOCK_BYTES[type_]
            nb1 = row_size(type_, ne[0])
        else:
            nb0 = {TYPE_F32: 4, TYPE_F16: 2, TYPE_I32: 4}[type_]
            nb1 = nb0 * ne[0]
        nb = [nb0, nb1, nb1 * ne[1], nb1 * ne[1] * ne[2]]
    t = Tensor()
    t.data = P((buf.addr if isinstance(buf, DeviceBuffer) else int(buf)) + offset)
    t._buf = buf   # a DeviceBuffer stays alive as long as the descriptor
    t.type = type_
    for i in range(4):
        t.ne[i] = int(ne[i])
        t.nb[i] = int(nb[i])
    return t


class Context:
    def __init__(self, device: int = 0):
        self.h = P()
        call("mi_moe_ctx_create", C.byref(self.h), device)

    def reserve(self, max_tokens: int, D: int, I: int, E: int, K: int) -> None:
        call("mi_moe_ctx_reserve", self.h, max_tokens, D, I, E, K)

    def set_gemm_threshold(self, t: int) -> None:
        """GEMM from t tokens on; 0 = by shape (GEMM when 2 T K >= E)."""
        call("mi_moe_ctx_set_gemm_threshold", self.h, t)

    def set_gemm_tiles(self, kind: int) -> None:
        """Q4_K-gate GEMM row tiles: 0 by shape, 1 192-row, 2 32-row, 3 the
        skinny 16-row products (all-Q4_K layers), 4 8-row where they apply,
        5 64-row"""
        call("mi_moe_ctx_set_gemm_tiles", self.h, int(kind))

    def set_fused_decode(self, mode) -> None:
        """False / DECODE_CHAIN, True / DECODE_FUSED (DECODE_FUSED_COOPERATIVE is
        retired: the library refuses it)"""
        m = DECODE_FUSED if mode is True else DECODE_CHAIN if mode is False else int(mode)
        call("mi_moe_ctx_set_fused_decode", self.h, m)

    def set_decode_rescue(self, polls: int) -> None:
        """Polls before a fused-decode work-group computes a result it waits for."""
        call("mi_moe_ctx_set_decode_rescue", self.h, int(polls))

    def take_errors(self):
        """(bad ids, fused-decode wait failures) since the last take; syncs the
        device.  The fp16-saturated block count is take_all_errors()[2]."""
        return self.take_all_errors()[:2]

    def take_all_errors(self):
        """(bad ids, fused-decode wait failures, GEMM-path Q8_K blocks clamped
        at the fp16 range) since the last take; syncs the device."""
        b, f, r = i64(), i64(), i64()
        call("mi_moe_ctx_take_errors", self.h, C.byref(b), C.byref(f), C.byref(r))
        return b.value, f.value, r.value

    def set_profiling(self, on: bool) -> None:
        call("mi_moe_ctx_set_profiling", self.h, int(on))

    def stage_times(self):
        names = (C.c_char_p * 16)()
        ms = (C.c_float * 16)()
        n = C.c_int()
        call("mi_moe_ctx_stage_times", self.h, 16, names, ms, C.byref(n))
        return [(names[i].decode(), ms[i]) for i in range(n.value)]

    def stage_clock(self, stage: str):
        """(GHz, work-groups measured) of the shader clock under the last
        profiled forward's `stage` GEMM ("gate_up" / "down"), or None when that
        stage did not run on the 4-wave GEMM path."""
        ghz, n = C.c_double(), C.c_int()
        rc = load().mi_moe_ctx_stage_clock(self.h, stage.encode(), C.byref(ghz), C.byref(n))
        if rc == ERR_ARG:
            return None
        check("mi_moe_ctx_stage_clock", rc)
        return ghz.value, n.value

    def forward(self, layer: Layer, x, T: int, res, out, routing: Routing | None = None,
                stream=None) -> int:
        return load().mi_moe_forward(self.h, C.byref(layer), _addr(x), T, _addr(res), _addr(out),
                                     C.byref(routing) if routing is not None else None,
                                     _addr(stream))

    def forward_router_input(self, layer: Layer, x, x_router, T: int, res, out, routing: Routing | None = None,
                             stream=None) -> int:
        """mi_moe_forward_router_input: the router reads x_router, the experts x."""
        return load().mi_moe_forward_router_input(self.h, C.byref(layer), _addr(x), _addr(x_router), T, _addr(res),
                                                  _addr(out), C.byref(routing) if routing is not None else None,
                                                  _addr(stream))

    def expert_ffn(self, layer: Layer, x, T: int, res, ids_gu, ids_dn, w, out, stream=None) -> int:
        return load().mi_moe_expert_ffn(self.h, C.byref(layer), _addr(x), T, _addr(res),
                                        _addr(ids_gu), _addr(ids_dn), _addr(w), _addr(out),
                                        _addr(stream))

    def top_k(self, a: Tensor, k: int, dst: Tensor, stream=None) -> int:
        return load().mi_top_k(self.h, C.byref(a), k, C.byref(dst), _addr(stream))

    def mul_mat_id(self, as_: Tensor, b: Tensor, ids: Tensor, dst: Tensor, stream=None) -> int:
        return load().mi_mul_mat_id(self.h, C.byref(as_), C.byref(b), C.byref(ids),
                                    C.byref(dst), _addr(stream))

    def quantize(self, type_: int, src, dst, nrows: int, n_per_row: int, stream=None) -> int:
        return load().mi_quantize(self.h, type_, _addr(src), _addr(dst), nrows, n_per_row,
                                  _addr(stream))

    def tile(self, src: Tensor, dst, desc: Tensor | None = None, stream=None) -> int:
        """dst = src (a Q4_K or Q6_K table) in the grouped GEMMs' tiled order;
        desc (if given) receives the copy's descriptor."""
        return load().mi_moe_tile(self.h, C.byref(src), _addr(dst), C.byref(desc) if desc is not None else None,
                                  _addr(stream))

    def fill_normal(self, dst, n: int, seed: int, stream_id: int, mean: float, std: float,
                    stream=None) -> int:
        return load().mi_fill_normal(self.h, _addr(dst), n, seed, stream_id, mean, std,
                                     _addr(stream))

    def norm(self, norm: Norm, x, n_rows: int, n_cols: int, y, stream=None) -> int:
        return load().mi_norm(self.h, C.byref(norm), _addr(x), n_rows, n_cols, _addr(y), _addr(stream))

    def forward_norm(self, layer: Layer, norm: Norm | None, h, T: int, res, out, routing: Routing | None = None,
                     stream=None) -> int:
        return load().mi_moe_forward_norm(self.h, C.byref(layer), C.byref(norm) if norm is not None else None,
                                          _addr(h), T, _addr(res), _addr(out),
                                          C.byref(routing) if routing is not None else None, _addr(stream))

    def rmsnorm(self, x, n_rows: int, n_cols: int, eps: float, y, stream=None) -> int:
        return load().mi_rmsnorm(self.h, _addr(x), n_rows, n_cols, eps, _addr(y), _addr(stream))

    def close(self) -> None:
        if self.h and self.h.value:
            load().mi_moe_ctx_destroy(self.h)
            self.h = P()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


NOALLOC_MAX_TOKENS = 64


def forward_noalloc(layer: Layer, x, T: int, res, out, routing: Routing | None = None, stream=None) -> int:
    """mi_moe_forward_noalloc: the forward with the library's per-GPU static
    workspace (no context, no allocation)."""
    return load().mi_moe_forward_noalloc(C.byref(layer), _addr(x), T, _addr(res), _addr(out),
                                         C.byref(routing) if routing is not None else None, _addr(stream))


def _addr(x):
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return P(x.addr)
    if isinstance(x, P):
        return x
    return P(int(x))


class Gguf:
    """A GGUF file opened by the library (mi_gguf_*)."""

    def __init__(self, path: str):
        self.h = P()
        check("mi_gguf_open", load().mi_gguf_open(C.byref(self.h), str(path).encode()))

    def get_int(self, key: str):
        v = i64()
        rc = load().mi_gguf_get_int(self.h, key.encode(), C.byref(v))
        return None if rc else v.value

    def tensor_info(self, name: str):
        t, ne, nb = C.c_int32(), (i64 * 4)(), C.c_uint64()
        rc = load().mi_gguf_tensor_info(self.h, name.encode(), C.byref(t), ne, C.byref(nb))
        return None if rc else (t.value, list(ne), nb.value)

    def load_moe_layer(self, block: int, act: int):
        """(Layer, device buffer address); free the buffer with mi_dev_free."""
        L, buf = Layer(), P()
        check("mi_gguf_load_moe_layer", load().mi_gguf_load_moe_layer(self.h, block, act, C.byref(L), C.byref(buf)))
        return L, buf

    def close(self) -> None:
        if self.h:
            load().mi_gguf_close(self.h)
            self.h = P()


class Stream:
    def __init__(self):
        self.h = P()
        call("mi_stream_create", C.byref(self.h))

    @property
    def addr(self) -> int:
        return self.h.value or 0

    def synchronize(self) -> None:
        call("mi_stream_synchronize", self.h)

    def destroy(self) -> None:
        if self.h:
            call("mi_stream_destroy", self.h)
            self.h = P()


class Graph:
    """Library calls captured on a stream (mi_stream_begin_capture ..
    mi_stream_end_capture) and instantiated; launch() replays them."""

    def __init__(self, stream: Stream, record):
        call("mi_stream_begin_capture", stream.h)
        self.h = P()
        try:
            record(stream)
        finally:
            rc = load().mi_stream_end_capture(stream.h, C.byref(self.h))
        check("end capture", rc)

    def launch(self, stream: Stream) -> None:
        call("mi_graph_launch", self.h, stream.h)

    def destroy(self) -> None:
        if self.h:
            call("mi_graph_destroy", self.h)
            self.h = P()


class Event:
    def __init__(self):
        self.h = P()
        call("mi_event_create", C.byref(self.h))

    def record(self, stream=None) -> None:
        call("mi_event_record", self.h, _addr(stream))

    def synchronize(self) -> None:
        call("mi_event_synchronize", self.h)

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        call("mi_event_elapsed_ms", C.byref(ms), self.h, end.h)
        return ms.value


def tiled_bytes(src: Tensor) -> int:
    """bytes of src's tiled copy (negative: an mi_moe_status)"""
    return load().mi_moe_tiled_bytes(C.byref(src))


def make_layer(D: int, E: int, K: int, I: int, router_w, router_b, gate: Tensor, up: Tensor | None,
               down: Tensor, fused: bool, act: int) -> Layer:
    L = Layer()
    L.n_embd, L.n_expert, L.n_expert_used, L.n_ff = D, E, K, I
    L.router_w = _addr(router_w)
    L.router_b = _addr(router_b)
    L.gate = gate
    if up is not None:
        L.up = up
    L.down = down
    L.fused_gate_up = int(fused)
    L.act = act
    L.gating = GATING_SOFTMAX_TOPK
    L._refs = (router_w, router_b, gate, up, down)   # device memory the descriptor points to
    return L
