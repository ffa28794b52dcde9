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
