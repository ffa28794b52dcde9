"""Expert tables in Q8_0, Q5_0, Q4_0 and F16 (the types the reference's
converters write by default: Q8_0 convert/convert_hf_to_gguf.py:55-57 and
convert/convert_qwen3omni.py:60-61,135; Q5_0 convert/convert_nemotronomni.py:
113-114; F16 / Q4_0 convert/convert_diffusiongemma.py:62), through the C ABI
against the CPU oracle.

  * mi_quantize of the four types byte-exact against the oracle's ggml _ref
    quantizers (zero blocks, ties, large and tiny scales);
  * whole layers at the moondream3 and qwen3omni shapes in Q8_0 and F16, at
    the default product path of each token count and the other one;
  * diffusiongemma's expert widths (n_embd 2816, n_ff 704: no k-quant row
    fits 704) in F16 with its own router input, all 128 experts;
  * Q4_0 / Q5_0 layers, gated and nemotronomni's relu^2 with the sigmoid
    router, on both paths;
  * mi_mul_mat_id of each type (b broadcast and per slot).
Bars: logits, ids, counts, offsets, permutation bit-exact; weights within
1e-6; output rel-L2 <= 1e-2 (rel-L2 and max-abs logged).  The GEMV path
quantizes the activations exactly as the oracle does (Q8_0 codes and scales
bit for bit, F16 by the same rounding) and sums exact integer / fp16
products, so it sits near 1e-6; the GEMM path rounds the dequantized
operands to fp16.
"""
import sys

import numpy as np
import pytest

import mimoe as M
import pyoracle as O
import workloads as W
from _util import max_abs, oracle_layer_dict, rel_l2
from test_gpu_configs import _check_routing, _routing_buffers

pytestmark = pytest.mark.gpu

TOL = 1e-2
NEW_TYPES = [M.TYPE_Q8_0, M.TYPE_Q5_0, M.TYPE_Q4_0, M.TYPE_F16]
NAMES = {M.TYPE_Q8_0: "q8_0", M.TYPE_Q5_0: "q5_0", M.TYPE_Q4_0: "q4_0", M.TYPE_F16: "f16"}


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = M.Context(0)
    c.reserve(256, 2816, 1024, 128, 8)
    yield c
    c.close()


@pytest.mark.parametrize("type_", NEW_TYPES, ids=[NAMES[t] for t in NEW_TYPES])
def test_quantize_bit_exact(ctx, type_):
    rng = np.random.default_rng(31 + type_)
    rows = [(rng.standard_normal((200, 96)) * 0.02).astype(np.float32),
            (rng.standard_normal((50, 96)) * rng.uniform(1e-6, 1e3, (50, 1))).astype(np.float32),
            np.zeros((2, 96), np.float32),
            np.tile(np.array([1.0, -1.0, 0.5, -0.5], np.float32), (3, 24)),      # ties of |max|
            np.round(rng.standard_normal((20, 96)) * 8).astype(np.float32) / 8]   # values on half steps
    rows = np.concatenate(rows)
    src = M.to_device(rows)
    rs = M.row_size(type_, 96)
    dst = M.DeviceBuffer(rows.shape[0] * rs)
    M.check("quantize", ctx.quantize(type_, src, dst, rows.shape[0], 96))
    got = dst.download(np.uint8, (rows.shape[0], rs))
    ref = O.quantize(type_, rows) if type_ != M.TYPE_F16 else rows.astype(np.float16).view(np.uint8)
    bad = np.nonzero((got != ref).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} rows differ, first {bad[:8]}"


def _spec(name, D, E, K, I, fused, t, act, seed, gating=M.GATING_SOFTMAX_TOPK):
    return W.LayerSpec(name, D, E, K, I, fused, t, t, act, "none", seed)


_layers = {}


def _layer(spec, cap_T=1024):
    if spec.name not in _layers:
        for k in list(_layers):            # one big layer resident at a time
            c, g, _ = _layers.pop(k)
            c.close()
        c = M.Context(0)
        c.reserve(cap_T, spec.D, spec.I, spec.E, spec.K)
        g = W.GpuLayer(c, spec)
        OL = oracle_layer_dict(g.download_tables(), spec, g.download_router(), None)
        _layers[spec.name] = (c, g, OL)
    return _layers[spec.name]


@pytest.fixture(scope="module", autouse=True)
def _close_layers():
    yield
    for c, g, _ in _layers.values():
        c.close()
    _layers.clear()


def _run_layer(spec, T, paths, xr=None):
    c, g, OL = _layer(spec)
    x = W.gen_x(c, spec, T)
    res = W.gen_x(c, spec, T, stream=W.S_RES)
    xh = x.download(np.float32, (T, spec.D))
    rh = res.download(np.float32, (T, spec.D))
    ref, dbg = O.moe_forward(OL, xh, rh)
    errs = {}
    for pname in paths:
        c.set_gemm_threshold({"default": 0, "gemv": 1 << 30, "gemm": 1}[pname])
        out = M.DeviceBuffer(4 * T * spec.D)
        bufs, r = _routing_buffers(T, spec.E, spec.K)
        M.check("forward", c.forward(g.layer, x, T, res, out, r))
        got = out.download(np.float32, (T, spec.D))
        _check_routing(bufs, dbg, T, spec.E, spec.K, f"{spec.name} T={T} {pname}")
        e = rel_l2(got - rh, ref - rh)
        errs[pname] = e
        log(f"{spec.name} T={T} {pname}: rel-L2 {e:.3e} max-abs {max_abs(got, ref):.3e}, "
            f"experts used {int((dbg['counts'] > 0).sum())}/{spec.E}")
        assert e <= TOL
    c.set_gemm_threshold(0)
    assert c.take_errors() == (0, 0)
    return errs


MD = {t: _spec(f"md_{NAMES[t]}", 2048, 64, 8, 1024, True, t, M.ACT_GELU_ERF_GP1, 0x5EED0800 + t)
      for t in (M.TYPE_Q8_0, M.TYPE_F16)}
QO = {t: _spec(f"qo_{NAMES[t]}", 2048, 128, 8, 768, False, t, M.ACT_SILU, 0x5EED0900 + t)
      for t in (M.TYPE_Q8_0, M.TYPE_F16)}


@pytest.mark.parametrize("type_", [M.TYPE_Q8_0, M.TYPE_F16], ids=["q8_0", "f16"])
@pytest.mark.parametrize("T,paths", [(1, ["default"]), (8, ["default", "gemm"]), (300, ["default", "gemv"]),
                                     (1024, ["default"])])
def test_moondream3_shape(type_, T, paths):
    """moondream3 with the converter's default Q8_0 tables (and F16): fused
    [h | g] ffn_up_exps ne=[2048, 2048, 64], gelu_erf(h) * (g + 1)"""
    errs = _run_layer(MD[type_], T, paths)
    if "gemv" in errs or T <= 8:
        assert errs.get("gemv", errs["default"]) <= 1e-4


@pytest.mark.parametrize("type_", [M.TYPE_Q8_0, M.TYPE_F16], ids=["q8_0", "f16"])
@pytest.mark.parametrize("T,paths", [(1, ["default"]), (64, ["default", "gemv"])])
def test_qwen3omni_shape(type_, T, paths):
    """qwen3omni with its converter's default Q8_0 tables (and --outtype f16):
    E 128, I 768, separate gate / up, SwiGLU"""
    _run_layer(QO[type_], T, paths)


@pytest.mark.parametrize("type_", [M.TYPE_Q5_0, M.TYPE_Q4_0], ids=["q5_0", "q4_0"])
@pytest.mark.parametrize("T", [5, 100])
def test_small_gated(type_, T):
    spec = _spec(f"small_{NAMES[type_]}", 512, 16, 4, 256, False, type_, M.ACT_GELU_TANH, 0x5EED0A00 + type_)
    _run_layer(spec, T, ["gemv", "gemm"])


def test_diffusiongemma_f16_model_widths():
    """diffusiongemma's experts at its own widths and default F16 tables
    (n_embd 2816, expert n_ff 704, 128 experts, top-8, GeGLU), softmax over
    all experts with a per-expert scale, the router on its own input
    (diffusiongemma_model.cpp:917-945)"""
    spec = _spec("dg_f16", 2816, 128, 8, 704, False, M.TYPE_F16, M.ACT_GELU_TANH, 0x5EED0B00)
    c, g, OL = _layer(spec, cap_T=256)
    rng = np.random.default_rng(5)
    es = (0.5 + rng.random(spec.E)).astype(np.float32)
    esd = M.to_device(es)
    g.layer.gating = M.GATING_SOFTMAX_ALL
    g.layer.expert_scale = esd.addr
    for T in (3, 150):
        x = (rng.standard_normal((T, spec.D)) * 0.5).astype(np.float32)
        xr = (rng.standard_normal((T, spec.D)) * 0.02).astype(np.float32)
        res = rng.standard_normal((T, spec.D)).astype(np.float32)
        logits = O.router_logits(OL["router_w"], None, xr)
        sel, w = O.route_gated(logits, spec.K, O.GATING_SOFTMAX_ALL, expert_scale=es)
        ref, _ = O.moe_forward(OL, x, res, sel_in=sel, w_in=w)
        out = M.DeviceBuffer(4 * T * spec.D)
        bufs, r = _routing_buffers(T, spec.E, spec.K)
        M.check("forward_router_input", c.forward_router_input(g.layer, M.to_device(x), M.to_device(xr), T,
                                                               M.to_device(res), out, r))
        assert np.array_equal(bufs["logits"].download(np.float32, (T, spec.E)).view(np.uint32),
                              logits.view(np.uint32))
        assert np.array_equal(bufs["sel"].download(np.int32, (T, spec.K)), sel)
        got = out.download(np.float32, (T, spec.D))
        e = rel_l2(got - res, ref - res)
        log(f"dg_f16 T={T}: rel-L2 {e:.3e} max-abs {max_abs(got, ref):.3e}")
        assert e <= TOL
    g.layer.gating = M.GATING_SOFTMAX_TOPK
    g.layer.expert_scale = None


@pytest.mark.parametrize("T", [3, 70])
def test_nemotron_q5_0_relu_sqr(T):
    """nemotronomni's expert stacks are Q5_0 in its mixed tier: non-gated
    relu^2 experts (the gate slot holds ffn_up_exps) with the sigmoid router,
    selection bias and renorm x 2.5 (nemotronomni_model.cpp:344-367)"""
    from test_gpu_variants import Variant, _run, PATHS
    v = Variant(1024, 32, 6, 512, M.ACT_RELU_SQR, M.GATING_SIGMOID_BIAS, qtype=O.TYPE_Q5_0, dtype=O.TYPE_Q5_0,
                sh_I=1024, sh_act=M.ACT_RELU_SQR, seed=48)
    _run(v, T, PATHS, "nemotron Q5_0 relu^2 + shared")


@pytest.mark.parametrize("type_", NEW_TYPES, ids=[NAMES[t] for t in NEW_TYPES])
@pytest.mark.parametrize("ne11,T", [(1, 6), (3, 6), (1, 200)])
def test_mul_mat_id(ctx, type_, ne11, T):
    rng = np.random.default_rng(400 + type_ + ne11 + T)
    E, N, Kin, n_used = 16, 160, 704, 3
    wf = (rng.standard_normal((E * N, Kin)) * 0.05).astype(np.float32)
    wq = O.quantize(type_, wf) if type_ != M.TYPE_F16 else wf.astype(np.float16).view(np.uint8)
    b = rng.standard_normal((T, ne11, Kin)).astype(np.float32)
    ids = np.stack([rng.permutation(E)[:n_used] for _ in range(T)]).astype(np.int32)
    ref = O.mul_mat_id(type_, wq, Kin, N, E, b, ids)
    asd, bd, idd = M.to_device(wq), M.to_device(b), M.to_device(ids)
    dst = M.DeviceBuffer(4 * T * n_used * N)
    rc = ctx.mul_mat_id(M.tensor(asd, type_, [Kin, N, E]), M.tensor(bd, M.TYPE_F32, [Kin, ne11, T]),
                        M.tensor(idd, M.TYPE_I32, [n_used, T]), M.tensor(dst, M.TYPE_F32, [N, n_used, T]))
    M.check("mul_mat_id", rc)
    got = dst.download(np.float32, (T, n_used, N))
    e = rel_l2(got, ref)
    log(f"mul_mat_id {NAMES[type_]} ne11={ne11} T={T}: rel-L2 {e:.3e}")
    assert e <= (1e-5 if T < 50 else TOL)
