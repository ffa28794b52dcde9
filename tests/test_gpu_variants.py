"""Router and expert variants of the other MoE consumers, through the C ABI,
against the CPU oracle.

  nemotronomni   sigmoid gating with selection bias, renorm x 2.5
                 (nemotronomni_model.cpp:344-354), non-gated relu^2 experts
                 (:364-367) and a relu^2 shared expert added unscaled
                 (:371-376); k-quant tables on the GEMV and GEMM paths, and
                 F32 tables at the model's own inner dims (1856 routed, 3712
                 shared), which no 256-value k-quant row fits
  qwen3omni talker  softmax top-k gating, SwiGLU experts and a SwiGLU shared
                 expert times the sigmoid of a scalar gate row
                 (qwen3omni_talker.cpp:379-402)
  diffusiongemma softmax over all experts, top-k on the probabilities, renorm,
                 per-expert scale (diffusiongemma_model.cpp:917-937), GeGLU;
                 also with router logits spread so far that probabilities
                 underflow to equal zeros (ties broken by id, unlike the logits)

Bars: logits, ids, counts, offsets, permutation bit-exact; weights within
1e-6; output rel-L2 <= 1e-2 (logged with max-abs).
"""
import ctypes as C
import sys

import numpy as np
import pytest

import mimoe as M
import pyoracle as O
from _util import max_abs, rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-2


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class Variant:
    """A layer built on the CPU (oracle quantizers), uploaded, with the oracle
    dict and the ABI descriptor of the same bytes."""

    def __init__(self, D, E, K, I, act, gating, qtype=O.TYPE_Q4_K, dtype=O.TYPE_Q4_K, sh_I=0, sh_act=0,
                 sh_gate=False, router_std=0.05, w_std=0.02, seed=0):
        rng = np.random.default_rng(seed)
        f = lambda *s: (rng.standard_normal(s) * w_std).astype(np.float32)  # noqa: E731
        q = lambda t, a: a if t == O.TYPE_F32 else O.quantize(t, a.reshape(-1, a.shape[-1])).ravel()  # noqa: E731
        gated = act != M.ACT_RELU_SQR
        self.keep = []
        self.o = dict(D=D, E=E, K=K, I=I, router_w=(rng.standard_normal((E, D)) * router_std).astype(np.float32),
                      router_b=None, gate_type=qtype, down_type=dtype, fused=False, act=act, gating=gating)
        self.o["gate"] = q(qtype, f(E, I, D))
        self.o["up"] = q(qtype, f(E, I, D)) if gated else None
        self.o["down"] = q(dtype, f(E, D, I))
        if gating == M.GATING_SIGMOID_BIAS:
            self.o.update(sel_bias=(rng.standard_normal(E) * 0.05).astype(np.float32), routed_scaling=2.5,
                          gate_eps=1e-20)
        if gating == M.GATING_SOFTMAX_ALL:
            self.o["expert_scale"] = (0.5 + rng.random(E)).astype(np.float32)
        if sh_I:
            sg = sh_act != M.ACT_RELU_SQR
            self.o.update(sh_I=sh_I, sh_act=sh_act, sh_type=qtype, sh_down_type=dtype, sh_gate=q(qtype, f(sh_I, D)),
                          sh_up=q(qtype, f(sh_I, D)) if sg else None, sh_down=q(dtype, f(D, sh_I)),
                          sh_gate_inp=(rng.standard_normal(D) * 0.05).astype(np.float32) if sh_gate else None)
        L = M.Layer()
        L.n_embd, L.n_expert, L.n_expert_used, L.n_ff = D, E, K, I
        L.router_w = self._dev(self.o["router_w"])
        L.gate = M.tensor(self._buf(self.o["gate"]), qtype, [D, I, E])
        if gated:
            L.up = M.tensor(self._buf(self.o["up"]), qtype, [D, I, E])
        L.down = M.tensor(self._buf(self.o["down"]), dtype, [I, D, E])
        L.fused_gate_up, L.act, L.gating = 0, act, gating
        if "sel_bias" in self.o:
            L.sel_bias, L.routed_scaling, L.gate_eps = self._dev(self.o["sel_bias"]), 2.5, 1e-20
        if "expert_scale" in self.o:
            L.expert_scale = self._dev(self.o["expert_scale"])
        if sh_I:
            L.sh_n_ff, L.sh_act = sh_I, sh_act
            L.sh_gate = M.tensor(self._buf(self.o["sh_gate"]), qtype, [D, sh_I])
            if self.o["sh_up"] is not None:
                L.sh_up = M.tensor(self._buf(self.o["sh_up"]), qtype, [D, sh_I])
            L.sh_down = M.tensor(self._buf(self.o["sh_down"]), dtype, [sh_I, D])
            if self.o["sh_gate_inp"] is not None:
                L.sh_gate_inp = self._dev(self.o["sh_gate_inp"])
        self.L = L

    def _buf(self, a):
        b = M.to_device(np.ascontiguousarray(a))
        self.keep.append(b)
        return b

    def _dev(self, a):
        return self._buf(a).addr


def _routing_buffers(T, E, K):
    bufs = dict(logits=M.DeviceBuffer(4 * T * E), sel=M.DeviceBuffer(4 * T * K),
                weights=M.DeviceBuffer(4 * T * K), counts=M.DeviceBuffer(4 * E),
                offsets=M.DeviceBuffer(4 * (E + 1)), perm=M.DeviceBuffer(4 * T * K))
    r = M.Routing()
    for k, v in bufs.items():
        setattr(r, k, C.c_void_p(v.addr))
    return bufs, r


def _run(v: Variant, T, paths, name, seed=1, x_scale=1.0):
    D, E, K = v.o["D"], v.o["E"], v.o["K"]
    ctx = M.Context(0)
    ctx.reserve(max(T, 1), D, v.o["I"], E, K)
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((T, D)) * x_scale).astype(np.float32)
    res = rng.standard_normal((T, D)).astype(np.float32)
    ref, dbg = O.moe_forward(v.o, x, res)
    for pname, thr in paths:
        ctx.set_gemm_threshold(thr)
        out = M.DeviceBuffer(4 * T * D)
        bufs, r = _routing_buffers(T, E, K)
        M.check("forward", ctx.forward(v.L, M.to_device(x), T, M.to_device(res), out, r))
        got = out.download(np.float32, (T, D))
        gl = bufs["logits"].download(np.float32, (T, E))
        assert np.array_equal(gl.view(np.uint32), dbg["logits"].view(np.uint32)), f"{name}: logits"
        assert np.array_equal(bufs["sel"].download(np.int32, (T, K)), dbg["sel"]), f"{name} {pname}: ids"
        assert np.allclose(bufs["weights"].download(np.float32, (T, K)), dbg["w"], rtol=1e-6, atol=1e-7), \
            f"{name} {pname}: weights"
        assert np.array_equal(bufs["perm"].download(np.int32, (T * K,)), dbg["perm"]), f"{name}: permutation"
        e = rel_l2(got - res, ref - res)
        log(f"{name} {pname} T={T}: rel-L2 {e:.3e} max-abs {max_abs(got, ref):.3e}")
        assert e <= TOL, (name, pname, T)
    ctx.close()
    return dbg


PATHS = [("gemv", 1 << 30), ("gemm", 1)]


@pytest.mark.parametrize("T", [1, 7, 100])
@pytest.mark.parametrize("dtype", [O.TYPE_Q4_K, O.TYPE_Q6_K], ids=["q4k_down", "q6k_down"])
def test_nemotron_relu_sqr_shared(T, dtype):
    v = Variant(1024, 32, 6, 512, M.ACT_RELU_SQR, M.GATING_SIGMOID_BIAS, dtype=dtype, sh_I=1024,
                sh_act=M.ACT_RELU_SQR, seed=40 + dtype)
    _run(v, T, PATHS, f"nemotron relu^2 + shared (down {dtype})")


def test_nemotron_f32_model_dims():
    # the model's own inner dims: 1856 routed, 3712 shared (not 256-value rows)
    v = Variant(256, 16, 6, 1856, M.ACT_RELU_SQR, M.GATING_SIGMOID_BIAS, qtype=O.TYPE_F32, dtype=O.TYPE_F32,
                sh_I=3712, sh_act=M.ACT_RELU_SQR, seed=41)
    _run(v, 5, [("default", 0)], "nemotron F32 I=1856 shared 3712")


@pytest.mark.parametrize("T", [1, 9, 64])
def test_talker_sigmoid_gated_shared(T):
    v = Variant(1024, 32, 6, 256, M.ACT_SILU, M.GATING_SOFTMAX_TOPK, sh_I=768, sh_act=M.ACT_SILU, sh_gate=True,
                seed=42)
    _run(v, T, PATHS, "talker SwiGLU + sigmoid-gated shared")


def test_talker_f32_model_dims():
    v = Variant(256, 16, 6, 384, M.ACT_SILU, M.GATING_SOFTMAX_TOPK, qtype=O.TYPE_F32, dtype=O.TYPE_F32, sh_I=768,
                sh_act=M.ACT_SILU, sh_gate=True, seed=43)
    _run(v, 7, [("default", 0)], "talker F32 I=384")


@pytest.mark.parametrize("T", [1, 33, 200])
def test_diffusiongemma_softmax_all(T):
    v = Variant(512, 128, 8, 256, M.ACT_GELU_TANH, M.GATING_SOFTMAX_ALL, seed=44)
    _run(v, T, PATHS, "diffusiongemma softmax-all")


def test_softmax_all_underflow_ties():
    # router logits spread over hundreds: most probabilities underflow to 0,
    # and the K picks include ties at 0 broken by the lower id
    v = Variant(256, 64, 8, 256, M.ACT_GELU_TANH, M.GATING_SOFTMAX_ALL, router_std=3.0, seed=45)
    dbg = _run(v, 50, [("default", 0)], "softmax-all underflow ties", x_scale=4.0)
    logit_rank = np.argsort(-dbg["logits"].astype(np.float64), axis=1, kind="stable")[:, :8]
    differs = int((logit_rank != dbg["sel"]).any(axis=1).sum())
    log(f"underflow ties: {differs} of 50 tokens pick differently from the logits' own ranking")
    assert differs > 0


def _router_input_case(v: Variant, T, paths, name, seed):
    """diffusiongemma's layer: the router reads xr = rms_norm(res) * router_scale
    * s (diffusiongemma_model.cpp:919-922), the experts x = rms_norm(res) *
    ffn_norm2 (:937); softmax over all experts, top-k of the probabilities,
    renorm, per-expert scale (:923-935).  The oracle side is the reference's
    graph in the oracle's ops: router logits of xr, the gating, then the
    experts on x with that routing."""
    D, E, K = v.o["D"], v.o["E"], v.o["K"]
    rng = np.random.default_rng(seed)
    res = rng.standard_normal((T, D)).astype(np.float32)
    r64 = res.astype(np.float64)
    nrm = r64 / np.sqrt((r64 * r64).mean(axis=1, keepdims=True) + 1e-6)
    router_scale = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    ffn_norm2 = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    xr = ((nrm.astype(np.float32) * router_scale) * np.float32(D ** -0.5)).astype(np.float32)
    x = (nrm.astype(np.float32) * ffn_norm2).astype(np.float32)
    logits = O.router_logits(v.o["router_w"], None, xr)
    sel, w = O.route_gated(logits, K, O.GATING_SOFTMAX_ALL, expert_scale=v.o["expert_scale"])
    ref, dbg = O.moe_forward(v.o, x, res, sel_in=sel, w_in=w)
    counts, offsets, perm = O.dispatch(sel, E)
    # the logits of x differ from those of xr, so the bit-exact logit check below tells them apart
    assert not np.array_equal(O.router_logits(v.o["router_w"], None, x), logits)
    ctx = M.Context(0)
    ctx.reserve(max(T, 1), D, v.o["I"], E, K)
    xd, xrd, rd = M.to_device(x), M.to_device(xr), M.to_device(res)
    for pname, thr in paths:
        ctx.set_gemm_threshold(thr)
        out = M.DeviceBuffer(4 * T * D)
        bufs, r = _routing_buffers(T, E, K)
        M.check("forward_router_input", ctx.forward_router_input(v.L, xd, xrd, T, rd, out, r))
        got = out.download(np.float32, (T, D))
        gl = bufs["logits"].download(np.float32, (T, E))
        assert np.array_equal(gl.view(np.uint32), logits.view(np.uint32)), f"{name}: logits"
        assert np.array_equal(bufs["sel"].download(np.int32, (T, K)), sel), f"{name} {pname}: ids"
        assert np.allclose(bufs["weights"].download(np.float32, (T, K)), w, rtol=1e-6, atol=1e-7), name
        assert np.array_equal(bufs["counts"].download(np.int32, (E,)), counts), f"{name}: counts"
        assert np.array_equal(bufs["offsets"].download(np.int32, (E + 1,)), offsets), f"{name}: offsets"
        assert np.array_equal(bufs["perm"].download(np.int32, (T * K,)), perm), f"{name}: permutation"
        e = rel_l2(got - res, ref - res)
        log(f"{name} {pname} T={T}: rel-L2 {e:.3e} max-abs {max_abs(got, ref):.3e}")
        assert e <= TOL, (name, pname, T)
    # x_router == x is the plain forward, bit for bit
    out1, out2 = M.DeviceBuffer(4 * T * D), M.DeviceBuffer(4 * T * D)
    ctx.set_gemm_threshold(0)
    M.check("forward_router_input", ctx.forward_router_input(v.L, xd, xd, T, rd, out1))
    M.check("forward", ctx.forward(v.L, xd, T, rd, out2))
    assert np.array_equal(out1.download(np.uint32, (T, D)), out2.download(np.uint32, (T, D)))
    ctx.close()


@pytest.mark.parametrize("T", [1, 12, 150])
def test_diffusiongemma_router_input(T):
    v = Variant(512, 128, 8, 256, M.ACT_GELU_TANH, M.GATING_SOFTMAX_ALL, seed=46)
    _router_input_case(v, T, PATHS, "diffusiongemma router input", 100 + T)


def test_diffusiongemma_router_input_model_dims():
    # the model's own widths (n_embd 2816, expert n_ff 704: no 256-value k-quant
    # row fits 704) with F32 tables, 16 of the 128 experts
    v = Variant(2816, 16, 8, 704, M.ACT_GELU_TANH, M.GATING_SOFTMAX_ALL, qtype=O.TYPE_F32, dtype=O.TYPE_F32,
                seed=47)
    _router_input_case(v, 5, [("default", 0)], "diffusiongemma router input, model widths", 200)
