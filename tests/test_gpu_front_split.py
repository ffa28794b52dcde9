"""Small calls on the kernel chain, through the C ABI, against the CPU
oracle: the router split over its chunks (k_front_parts + k_topk_parts) and
the 32-row GEMMs without a dispatch launch (each work-group finds its tile).

Below T x E = 8192 logits, and where the (16-token, 16-expert) tiles alone
would leave half of the CUs idle, the kernel chain computes each 64-value
chunk's fp64 partial in its own wave, stores the partials, and the top-k
launch adds them in chunk order before rounding: the same order as the
one-launch front, so the logits stay bit-identical to the oracle's.  The
cases straddle the switch (qwen3omni T = 64 / 65, moondream3 T = 128 / 129),
include a router bias (the Zipf-skewed config-2 layer: the bias is added
after the rounding, in the top-k launch) and the three gating kinds (the
sigmoid kind reads the selected experts' logits back across lanes), and run
the chain (fused decode off), so T = 1 takes the split router as well.

Bars: logits, ids, counts, offsets, permutation bit-exact; weights within
1e-6; output rel-L2 <= 1e-2 (logged with max-abs).
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


CASES = [("qo", 3, T) for T in (1, 5, 16, 33, 64, 65)] + [("md_skew", 2, T) for T in (2, 40, 128, 129)]


@pytest.mark.parametrize("name,cfg,T", CASES, ids=[f"{n}-T{t}" for n, _, t in CASES])
def test_front_split_routing(name, cfg, T):
    spec = W.CONFIGS[cfg]["spec"]
    log(f"case {name} T={T}")
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    ctx.set_fused_decode(M.DECODE_CHAIN)
    g = W.GpuLayer(ctx, spec)
    OL = oracle_layer_dict(g.download_tables(), g.spec, g.download_router(), g.bias_host)
    x = W.gen_x(ctx, spec, T, copy=1)
    xh = x.download(np.float32, (T, spec.D))
    ref, dbg = O.moe_forward(OL, xh)
    out = M.DeviceBuffer(4 * T * spec.D)
    bufs, r = _routing_buffers(T, spec.E, spec.K)
    M.check("forward", ctx.forward(g.layer, x, T, None, out, r))
    got = out.download(np.float32, (T, spec.D))
    gl = bufs["logits"].download(np.float32, (T, spec.E))
    assert np.array_equal(gl.view(np.uint32), dbg["logits"].view(np.uint32)), f"{name} T={T}: logits"
    assert np.array_equal(bufs["sel"].download(np.int32, (T, spec.K)), dbg["sel"]), f"{name} T={T}: ids"
    assert np.allclose(bufs["weights"].download(np.float32, (T, spec.K)), dbg["w"], rtol=1e-6, atol=1e-7)
    assert np.array_equal(bufs["counts"].download(np.int32, (spec.E,)), dbg["counts"])
    assert np.array_equal(bufs["offsets"].download(np.int32, (spec.E + 1,)), dbg["offsets"])
    assert np.array_equal(bufs["perm"].download(np.int32, (T * spec.K,)), dbg["perm"])
    e = rel_l2(got, ref)
    log(f"{name} T={T}: rel-L2 {e:.3e} max-abs {max_abs(got, ref):.3e}")
    assert e <= TOL
    ctx.close()


@pytest.mark.parametrize("gating", [M.GATING_SIGMOID_BIAS, M.GATING_SOFTMAX_ALL], ids=["sigmoid_bias", "softmax_all"])
@pytest.mark.parametrize("T", [1, 24])
def test_front_split_gating_kinds(gating, T):
    # qwen3omni widths with the other two gating kinds (oracle: route_gated on
    # the oracle's logits)
    D, E, K = 2048, 128, 8
    rng = np.random.default_rng(7 + T + gating)
    Wr = (rng.standard_normal((E, D)) * 0.05).astype(np.float32)
    x = rng.standard_normal((T, D)).astype(np.float32)
    sel_bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
    scale = (0.5 + rng.random(E)).astype(np.float32)
    logits = O.router_logits(Wr, None, x)
    if gating == M.GATING_SIGMOID_BIAS:
        sel, w = O.route_gated(logits, K, O.GATING_SIGMOID_BIAS, sel_bias=sel_bias, scaling=2.5, eps=1e-20)
    else:
        sel, w = O.route_gated(logits, K, O.GATING_SOFTMAX_ALL, expert_scale=scale)
    # a layer whose experts do not matter here: tiny Q4_K tables, routing only
    I = 256
    spec_tables = {nm: O.quantize(O.TYPE_Q4_K, (rng.standard_normal((E * rows, cols)) * 0.02).astype(np.float32))
                   for nm, rows, cols in (("gate", I, D), ("up", I, D), ("down", D, I))}
    keep = []

    def dev(a):
        b = M.to_device(np.ascontiguousarray(a))
        keep.append(b)
        return b

    L = M.Layer()
    L.n_embd, L.n_expert, L.n_expert_used, L.n_ff = D, E, K, I
    L.router_w = dev(Wr).addr
    L.gate = M.tensor(dev(spec_tables["gate"]), M.TYPE_Q4_K, [D, I, E])
    L.up = M.tensor(dev(spec_tables["up"]), M.TYPE_Q4_K, [D, I, E])
    L.down = M.tensor(dev(spec_tables["down"]), M.TYPE_Q4_K, [I, D, E])
    L.fused_gate_up, L.act, L.gating = 0, M.ACT_SILU, gating
    if gating == M.GATING_SIGMOID_BIAS:
        L.sel_bias, L.routed_scaling, L.gate_eps = dev(sel_bias).addr, 2.5, 1e-20
    else:
        L.expert_scale = dev(scale).addr
    ctx = M.Context(0)
    ctx.reserve(T, D, I, E, K)
    ctx.set_fused_decode(M.DECODE_CHAIN)
    out = M.DeviceBuffer(4 * T * D)
    bufs, r = _routing_buffers(T, E, K)
    M.check("forward", ctx.forward(L, M.to_device(x), T, None, out, r))
    gl = bufs["logits"].download(np.float32, (T, E))
    assert np.array_equal(gl.view(np.uint32), logits.view(np.uint32)), "logits"
    assert np.array_equal(bufs["sel"].download(np.int32, (T, K)), sel), "ids"
    assert np.allclose(bufs["weights"].download(np.float32, (T, K)), w, rtol=1e-6, atol=1e-7), "weights"
    log(f"gating {gating} T={T}: routing bit-exact")
    ctx.close()


SD_CASES = [("qo", 3, T) for T in (8, 16, 32, 64)] + [("md", 0, T) for T in (4, 16, 40, 64)]


@pytest.mark.parametrize("name,cfg,T", SD_CASES, ids=[f"{n}-T{t}" for n, _, t in SD_CASES])
def test_gemm_self_dispatch(name, cfg, T):
    """Small calls on the 32-row GEMM tiles skip the dispatch launch when the
    caller asks for no dispatch outputs: each GEMM work-group derives its
    tile from the ids.  Its output must equal the dispatched call's bit for
    bit (same tiles, same rows, same K order), and the oracle's to 1e-2."""
    spec = W.CONFIGS[cfg]["spec"]
    log(f"case {name} T={T}")
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    ctx.set_fused_decode(M.DECODE_CHAIN)
    g = W.GpuLayer(ctx, spec)
    OL = oracle_layer_dict(g.download_tables(), g.spec, g.download_router(), g.bias_host)
    x = W.gen_x(ctx, spec, T, copy=2)
    ref, dbg = O.moe_forward(OL, x.download(np.float32, (T, spec.D)))
    outs = []
    for with_routing in (True, False):
        out = M.DeviceBuffer(4 * T * spec.D)
        bufs, r = _routing_buffers(T, spec.E, spec.K)
        M.check("forward", ctx.forward(g.layer, x, T, None, out, r if with_routing else None))
        outs.append(out.download(np.float32, (T, spec.D)))
        if with_routing:
            assert np.array_equal(bufs["perm"].download(np.int32, (T * spec.K,)), dbg["perm"])
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), f"{name} T={T}: self-dispatch differs"
    e = rel_l2(outs[1], ref)
    log(f"{name} T={T} self-dispatch: bit-identical to the dispatched call; rel-L2 {e:.3e} "
        f"max-abs {max_abs(outs[1], ref):.3e}, experts used {int((dbg['counts'] > 0).sum())}/{spec.E}")
    assert e <= TOL
    ctx.close()
