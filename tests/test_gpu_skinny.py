"""The skinny grouped products (k_gs.hip: 16-row tiles of a balanced
dispatch, each wave's weight stream held several blocks ahead in registers,
v_mfma_f32_16x16x32_f16) through the C ABI, against the CPU oracle and
against the 4-wave GEMMs (32-row tiles) on the same inputs.

Bars: router logits, ids, weights and the permutation bit-exact; layer
output rel-L2 <= 1e-2 against the oracle, rel-L2 and
max-abs logged; the two GPU product paths within 2e-3 of each other (the
same fp16 operands, the products summed in another order, then the fp16
and Q8_K roundings of the activation rows); no range saturation.

Shapes: qwen3omni (E 128, top-8, I 768, separate gate / up, SwiGLU) from 8
to 128 tokens - at 128 several experts receive more than 16 rows, which
take several tiles - and the moondream3 layer with Q4_K down (fused [h | g]
up_exps, E 64, I 1024) with tanh-GELU and with moondream3's own
gelu_erf(h) * (g + 1), up to 64 tokens (multi-tile experts again).
"""
import ctypes as C
import sys

import numpy as np
import pytest

import mimoe as M
import pyoracle as O
import workloads as W
from _util import max_abs, oracle_layer_dict, rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-2
PATH_TOL = 2e-3
TILES_SKINNY, TILES_32 = 3, 2


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _routing_buffers(T, E, K):
    bufs = dict(logits=M.DeviceBuffer(4 * T * E), sel=M.DeviceBuffer(4 * T * K),
                weights=M.DeviceBuffer(4 * T * K), counts=M.DeviceBuffer(4 * E),
                offsets=M.DeviceBuffer(4 * (E + 1)), perm=M.DeviceBuffer(4 * T * K))
    r = M.Routing()
    for k, v in bufs.items():
        setattr(r, k, C.c_void_p(v.addr))
    return bufs, r


def _check_routing(bufs, dbg, T, E, K, what):
    gl = bufs["logits"].download(np.float32, (T, E))
    assert np.array_equal(gl.view(np.uint32), dbg["logits"].view(np.uint32)), f"{what}: router logits"
    assert np.array_equal(bufs["sel"].download(np.int32, (T, K)), dbg["sel"]), f"{what}: expert ids"
    assert np.allclose(bufs["weights"].download(np.float32, (T, K)), dbg["w"], rtol=1e-6, atol=1e-7), \
        f"{what}: weights"
    assert np.array_equal(bufs["perm"].download(np.int32, (T * K,)), dbg["perm"]), f"{what}: permutation"


def _spec(name):
    if name == "qo_cfg3":
        return W.CONFIGS[3]["spec"]
    if name == "md_q4down":
        return W.CONFIGS[0]["spec"]
    return W.md_spec(0, M.TYPE_Q4_K, act=M.ACT_GELU_ERF_GP1)


CASES = [("qo_cfg3", 8), ("qo_cfg3", 21), ("qo_cfg3", 32), ("qo_cfg3", 64), ("qo_cfg3", 128),
         ("md_q4down", 8), ("md_q4down", 40), ("md_q4down", 64), ("md_gelu_erf", 40)]


@pytest.mark.parametrize("name,T", CASES)
def test_skinny_products(name, T):
    spec = _spec(name)
    log(f"case {name} T={T}: skinny products vs 32-row GEMM tiles vs oracle")
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    g = W.GpuLayer(ctx, spec)
    x = W.gen_x(ctx, spec, T)
    xh = x.download(np.float32, (T, spec.D))
    ref, dbg = O.moe_forward(oracle_layer_dict(g.download_tables(), spec, g.download_router(), None), xh)
    counts = np.bincount(dbg["sel"].ravel(), minlength=spec.E)
    log(f"{name} T={T}: rows per expert max {counts.max()}, experts with rows {int((counts > 0).sum())}, "
        f"tiles of 16 {int(np.ceil(counts / 16).sum())}")
    ctx.set_fused_decode(M.DECODE_CHAIN)
    ctx.set_gemm_threshold(1)
    outs = {}
    for kind in (TILES_SKINNY, TILES_32):
        ctx.set_gemm_tiles(kind)
        out = M.DeviceBuffer(4 * T * spec.D)
        bufs, r = _routing_buffers(T, spec.E, spec.K)
        M.check("forward", ctx.forward(g.layer, x, T, None, out, r))
        got = out.download(np.float32, (T, spec.D))
        what = "skinny" if kind == TILES_SKINNY else "32-row tiles"
        _check_routing(bufs, dbg, T, spec.E, spec.K, f"{name} T={T} {what}")
        e = rel_l2(got, ref)
        log(f"{name} T={T} {what}: rel-L2 {e:.3e} max-abs {max_abs(got, ref):.3e} vs oracle")
        assert np.isfinite(got).all()
        assert e <= TOL
        outs[kind] = got
    d = rel_l2(outs[TILES_SKINNY], outs[TILES_32])
    log(f"{name} T={T}: skinny vs 32-row tiles rel-L2 {d:.3e} max-abs "
        f"{max_abs(outs[TILES_SKINNY], outs[TILES_32]):.3e}")
    assert d <= PATH_TOL
    ctx.set_gemm_tiles(0)
    ctx.set_gemm_threshold(0)
    assert ctx.take_all_errors() == (0, 0, 0)
    ctx.close()


def test_skinny_refused_where_it_does_not_apply():
    """Forcing the skinny kind on a layer it does not take (Q6_K down)
    leaves the layer on the shape rule's GEMM: same bits as kind 0."""
    spec = W.CONFIGS[1]["spec"]
    T = 40
    log(f"case md_cfg1 T={T}: skinny kind on a Q6_K-down layer")
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    g = W.GpuLayer(ctx, spec)
    x = W.gen_x(ctx, spec, T)
    ctx.set_gemm_threshold(1)
    outs = []
    for kind in (0, TILES_SKINNY):
        ctx.set_gemm_tiles(kind)
        out = M.DeviceBuffer(4 * T * spec.D)
        M.check("forward", ctx.forward(g.layer, x, T, None, out, None))
        outs.append(out.download(np.float32, (T, spec.D)))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert ctx.take_all_errors() == (0, 0, 0)
    ctx.close()
