"""Layers whose gate/up tables are Q6_K, as the reference's converters write
them on request (moondream3 `--q6`: convert/convert_hf_to_gguf.py:56,74-76;
qwen3omni `--outtype q6_k`: convert/convert_qwen3omni.py:60-61,135), through
the C ABI against the CPU oracle.

Shapes:
  md_q6  moondream3: fused [h | g] ffn_up_exps ne=[2048, 2048, 64] Q6_K,
         ffn_down_exps Q6_K, gelu_erf(h) * (g + 1) (moondream.cpp:509-544)
  qo_q6  qwen3omni: E 128, I 768, separate gate / up, SwiGLU, all Q6_K
         (qwen3omni_model.cpp:755-780)

Every token count runs on the path the default rule picks (T = 1: the
single-token chain, the fused kernel takes Q4_K gate/up only; small T: the
grouped GEMV with its Q6_K GLU epilogue; large T: the 16x16x32 MFMA GEMM with
its fused GLU + Q8_K epilogue), and the middle sizes also on the other
product path.  Bars: logits, ids, counts, offsets and permutation bit-exact;
weights within 1e-6; output rel-L2 <= 1e-2, rel-L2 and max-abs logged.
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

MD_Q6 = W.LayerSpec("md_q6", 2048, 64, 8, 1024, True, M.TYPE_Q6_K, M.TYPE_Q6_K, M.ACT_GELU_ERF_GP1,
                    "none", 0x5EED0600)
QO_Q6 = W.LayerSpec("qo_q6", 2048, 128, 8, 768, False, M.TYPE_Q6_K, M.TYPE_Q6_K, M.ACT_SILU, "none",
                    0x5EED0601)

# (spec, T, forced product paths beside the default: "gemv" / "gemm")
CASES = [
    (MD_Q6, 1, []),
    (MD_Q6, 8, ["gemm"]),
    (MD_Q6, 300, ["gemv"]),
    (MD_Q6, 1024, []),
    (QO_Q6, 1, []),
    (QO_Q6, 64, ["gemv"]),
]


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


_layers = {}


def _layer(spec):
    """one context + device layer + oracle tables per spec for the module"""
    if spec.name not in _layers:
        ctx = M.Context(0)
        ctx.reserve(1024, spec.D, spec.I, spec.E, spec.K)
        g = W.GpuLayer(ctx, spec)
        OL = oracle_layer_dict(g.download_tables(), spec, g.download_router(), None)
        _layers[spec.name] = (ctx, g, OL)
    return _layers[spec.name]


@pytest.fixture(scope="module", autouse=True)
def _close_layers():
    yield
    for ctx, g, _ in _layers.values():
        ctx.close()
    _layers.clear()


@pytest.mark.parametrize("spec,T,forced", CASES, ids=[f"{s.name}-T{t}" for s, t, _ in CASES])
def test_q6k_gate_up_layer(spec, T, forced):
    log(f"case {spec.name} T={T} paths default+{forced}")
    ctx, g, OL = _layer(spec)
    x = W.gen_x(ctx, spec, T)
    res = W.gen_x(ctx, spec, T, stream=W.S_RES)
    xh = x.download(np.float32, (T, spec.D))
    rh = res.download(np.float32, (T, spec.D))
    ref, dbg = O.moe_forward(OL, xh, rh)
    for pname in ["default"] + forced:
        ctx.set_gemm_threshold({"default": 0, "gemv": 1 << 30, "gemm": 1}[pname])
        out = M.DeviceBuffer(4 * T * spec.D)
        bufs, r = _routing_buffers(T, spec.E, spec.K)
        M.check("forward", ctx.forward(g.layer, x, T, res, out, r))
        got = out.download(np.float32, (T, spec.D))
        _check_routing(bufs, dbg, T, spec.E, spec.K, f"{spec.name} T={T} {pname}")
        # the residual is N(0,1) like the MoE sum's inputs: hold the MoE part to the bar
        e = rel_l2(got - rh, ref - rh)
        log(f"{spec.name} T={T} {pname}: rel-L2 {e:.3e} max-abs {max_abs(got, ref):.3e}, "
            f"experts used {int((dbg['counts'] > 0).sum())}/{spec.E}")
        assert e <= TOL
    ctx.set_gemm_threshold(0)
    _, waits, sat = ctx.take_all_errors()
    assert waits == 0 and sat == 0
