"""Layer stack pieces (h_{l+1} = h_l + MoE_l(RMSNorm(h_l)),
attention as identity) through the C ABI.

* mi_rmsnorm against a float64 numpy restatement (rtol 2e-6), in place and
  out of place, on a width that is not a multiple of the 256-thread stride.
* Two layers of a small moondream-shape stack on the GPU (norm on the GPU,
  MoE with the residual pointer) against the CPU oracle fed the GPU's own
  normalized input per layer: routing bit-exact, outputs rel-L2 <= 1e-2.
"""
import ctypes as C
import sys

import numpy as np
import pytest

import mimoe as M
import pyoracle as O
import workloads as W
from _util import cpu_layer, max_abs, oracle_layer_dict, rel_l2, small_spec

pytestmark = pytest.mark.gpu

EPS = 1e-6


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rmsnorm_ref(x: np.ndarray, eps: float) -> np.ndarray:
    x64 = x.astype(np.float64)
    return (x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + eps)).astype(np.float32)


@pytest.mark.parametrize("T,D", [(37, 2048), (5, 300), (1, 1)])
def test_rmsnorm(T, D):
    ctx = M.Context(0)
    rng = np.random.default_rng(T * 1000 + D)
    x = (rng.standard_normal((T, D)) * 3.0).astype(np.float32)
    xd, yd = M.to_device(x), M.DeviceBuffer(4 * T * D)
    M.check("rmsnorm", ctx.rmsnorm(xd, T, D, EPS, yd))
    ref = rmsnorm_ref(x, EPS)
    got = yd.download(np.float32, (T, D))
    assert np.allclose(got, ref, rtol=2e-6, atol=1e-7), float(np.abs(got - ref).max())
    # in place
    M.check("rmsnorm", ctx.rmsnorm(xd, T, D, EPS, xd))
    assert np.array_equal(xd.download(np.float32, (T, D)), got)
    assert ctx.rmsnorm(None, T, D, EPS, yd) == -1   # MI_MOE_ERR_NULL
    ctx.close()


def test_stack_two_layers():
    spec = small_spec("stack", D=512, E=8, K=2, I=256, fused=True, down_type=O.TYPE_Q6_K,
                      act=O.ACT_GELU_TANH, seed=0x5EED2000)
    T = 6
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    layers = [W.GpuLayer(ctx, spec, copy=c) for c in range(2)]
    cpus = [cpu_layer(spec, copy=c) for c in range(2)]
    h = W.gen_x(ctx, spec, T)
    n = M.DeviceBuffer(4 * T * spec.D)
    out = M.DeviceBuffer(4 * T * spec.D)
    for li, (g, cl) in enumerate(zip(layers, cpus)):
        M.check("rmsnorm", ctx.rmsnorm(h, T, spec.D, EPS, n))
        M.check("forward", ctx.forward(g.layer, n, T, h, out))
        h_in = h.download(np.float32, (T, spec.D))
        n_in = n.download(np.float32, (T, spec.D))
        assert np.allclose(n_in, rmsnorm_ref(h_in, EPS), rtol=2e-6, atol=1e-7)
        got = out.download(np.float32, (T, spec.D))
        ref, _ = O.moe_forward(oracle_layer_dict(cl, spec, cl["router_w"], None), n_in, h_in)
        e = rel_l2(got - h_in, ref - h_in)
        log(f"stack layer {li}: rel-L2 {e:.3e} max-abs {max_abs(got, ref):.3e}")
        assert e <= 1e-2
        h, out = out, h
    ctx.close()


# ------------------------------------------------------------------ pre-MoE norms
def norm_ref(x: np.ndarray, kind: int, eps: float, w=None, b=None) -> np.ndarray:
    """fp64 restatement of ggml_rms_norm / ggml_norm, then * w, + b."""
    x64 = x.astype(np.float64)
    if kind == M.NORM_RMS:
        y = x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + eps)
    else:
        c = x64 - x64.mean(axis=1, keepdims=True)
        y = c / np.sqrt((c * c).mean(axis=1, keepdims=True) + eps)
    if w is not None:
        y = y * w.astype(np.float64)
    if b is not None and kind == M.NORM_LAYER:
        y = y + b.astype(np.float64)
    return y


NORMS = [("rms", M.NORM_RMS, False, False), ("rms_w", M.NORM_RMS, True, False),
         ("layer", M.NORM_LAYER, False, False), ("layer_wb", M.NORM_LAYER, True, True)]


def _norm_tensors(D, with_w, with_b, seed):
    rng = np.random.default_rng(seed)
    w = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32) if with_w else None
    b = (0.1 * rng.standard_normal(D)).astype(np.float32) if with_b else None
    return w, b


@pytest.mark.parametrize("name,kind,with_w,with_b", NORMS)
@pytest.mark.parametrize("T,D", [(37, 2048), (5, 300), (3, 4096), (2, 1)])
def test_norm_op(name, kind, with_w, with_b, T, D):
    """mi_norm against the fp64 restatement: |err| <= 2e-6 * (|y| + scale of
    the row), covering the LayerNorm cancellation near the mean; in place
    gives the same bits; D > 4096 is refused."""
    ctx = M.Context(0)
    rng = np.random.default_rng(T * 7919 + D)
    x = (rng.standard_normal((T, D)) * 3.0 + 0.5).astype(np.float32)
    w, b = _norm_tensors(D, with_w, with_b, D)
    wd = M.to_device(w) if w is not None else None
    bd = M.to_device(b) if b is not None else None
    nrm = M.make_norm(kind, EPS, wd, bd)
    xd, yd = M.to_device(x), M.DeviceBuffer(4 * T * D)
    M.check("norm", ctx.norm(nrm, xd, T, D, yd))
    got = yd.download(np.float32, (T, D)).astype(np.float64)
    ref = norm_ref(x, kind, EPS, w, b)
    scale = np.abs(ref).max(axis=1, keepdims=True) + 1e-30
    err = np.abs(got - ref) / (np.abs(ref) + scale)
    assert err.max() <= 2e-6, (name, float(err.max()))
    M.check("norm in place", ctx.norm(nrm, xd, T, D, xd))
    assert np.array_equal(xd.download(np.float32, (T, D)), yd.download(np.float32, (T, D)))
    big = M.DeviceBuffer(4 * 4097)
    assert ctx.norm(nrm, big, 1, 4097, big) == -6   # MI_MOE_ERR_UNSUPPORTED
    ctx.close()


def _fused_vs_separate(ctx, layer, spec, T, nrm, seed):
    """forward_norm(h, res=h) against norm(h) -> forward(n, res=h): outputs and
    routing bit-identical."""
    rng = np.random.default_rng(seed)
    h = (rng.standard_normal((T, spec.D)) * 2.0 + 0.3).astype(np.float32)
    hd = M.to_device(h)
    nd = M.DeviceBuffer(4 * T * spec.D)
    out_f, out_s = M.DeviceBuffer(4 * T * spec.D), M.DeviceBuffer(4 * T * spec.D)
    rt = []
    for _ in range(2):
        bufs = dict(logits=M.DeviceBuffer(4 * T * spec.E), sel=M.DeviceBuffer(4 * T * spec.K),
                    weights=M.DeviceBuffer(4 * T * spec.K))
        r = M.Routing()
        for k, v in bufs.items():
            setattr(r, k, C.c_void_p(v.addr))
        rt.append((bufs, r))
    M.check("forward_norm", ctx.forward_norm(layer, nrm, hd, T, hd, out_f, rt[0][1]))
    M.check("norm", ctx.norm(nrm, hd, T, spec.D, nd))
    M.check("forward", ctx.forward(layer, nd, T, hd, out_s, rt[1][1]))
    M.synchronize()
    a, b = out_f.download(np.float32, (T, spec.D)), out_s.download(np.float32, (T, spec.D))
    assert np.isfinite(a).all()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), "outputs"
    for k, shape, dt in (("logits", (T, spec.E), np.float32), ("sel", (T, spec.K), np.int32),
                         ("weights", (T, spec.K), np.float32)):
        ga, gb = rt[0][0][k].download(dt, shape), rt[1][0][k].download(dt, shape)
        assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32)), k


@pytest.mark.parametrize("name,kind,with_w,with_b", [NORMS[1], NORMS[3]])
def test_forward_norm_small(name, kind, with_w, with_b):
    """Small moondream-shape layer: T = 1 and 5 (single-token kernel or GEMV
    chain, by the planner) and 300 (GEMM path)."""
    spec = small_spec("norm_small", D=512, E=8, K=2, I=256, fused=True, down_type=O.TYPE_Q6_K,
                      act=O.ACT_GELU_ERF_GP1, seed=0x5EED4000)
    ctx = M.Context(0)
    ctx.reserve(300, spec.D, spec.I, spec.E, spec.K)
    g = W.GpuLayer(ctx, spec)
    w, b = _norm_tensors(spec.D, with_w, with_b, 11)
    nrm = M.make_norm(kind, EPS, M.to_device(w) if w is not None else None,
                      M.to_device(b) if b is not None else None)
    for T in (1, 5, 300):
        _fused_vs_separate(ctx, g.layer, spec, T, nrm, T)
        log(f"forward_norm {name} small T={T}: fused == norm + forward")
    ctx.close()


@pytest.mark.parametrize("name,kind,with_w,with_b", [NORMS[0], NORMS[3]])
@pytest.mark.parametrize("T", [1, 1024])
def test_forward_norm_config(name, kind, with_w, with_b, T):
    """The config-1 layer: the single-token fused kernel (T = 1) and the
    1024-token GEMM path normalize on load exactly as the norm op does."""
    spec = W.CONFIGS[1]["spec"]
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    g = W.GpuLayer(ctx, spec)
    w, b = _norm_tensors(spec.D, with_w, with_b, 12)
    nrm = M.make_norm(kind, EPS, M.to_device(w) if w is not None else None,
                      M.to_device(b) if b is not None else None)
    _fused_vs_separate(ctx, g.layer, spec, T, nrm, 1000 + T)
    log(f"forward_norm {name} md_cfg1 T={T}: fused == norm + forward")
    ctx.close()


@pytest.mark.parametrize("T", [1, 5])
@pytest.mark.parametrize("rescue", [64, 0])
def test_forward_norm_in_place(T, rescue):
    """forward_norm with out == res == h (the header allows out to alias res,
    and res is h here): bit-identical to norm(h) -> forward(n, res=h) into a
    separate buffer.  T = 1 runs the single-token kernel, which must then
    normalize into the workspace first (a work-group that recomputes a late
    router row re-reads h); rescue 0 makes every work-group recompute what
    is not ready at its first look."""
    spec = W.CONFIGS[1]["spec"]
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    ctx.set_decode_rescue(rescue)
    g = W.GpuLayer(ctx, spec)
    nrm = M.make_norm(M.NORM_RMS, EPS)
    rng = np.random.default_rng(77 + T)
    h = (rng.standard_normal((T, spec.D)) * 2.0).astype(np.float32)
    hd, nd, ref = M.to_device(h), M.DeviceBuffer(4 * T * spec.D), M.DeviceBuffer(4 * T * spec.D)
    M.check("norm", ctx.norm(nrm, hd, T, spec.D, nd))
    M.check("forward", ctx.forward(g.layer, nd, T, hd, ref))
    for rep in range(3):
        hd2 = M.to_device(h)
        M.check("forward_norm in place", ctx.forward_norm(g.layer, nrm, hd2, T, hd2, hd2))
        a = hd2.download(np.float32, (T, spec.D))
        assert np.array_equal(a.view(np.uint32), ref.download(np.float32, (T, spec.D)).view(np.uint32)), rep
    assert ctx.take_errors() == (0, 0)
    log(f"forward_norm in place T={T} rescue={rescue}: == norm + forward")
    ctx.close()
