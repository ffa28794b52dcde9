"""BASELINE.json configs at their own sizes, through the C ABI, against the CPU
oracle (ggml-semantics restatement, oracle/moe_oracle.c).

Bars: router logits, expert ids, counts, offsets and the permutation
bit-exact for every token; routing weights within 1e-6; layer output rel-L2
<= 1e-2, rel-L2 and max-abs logged.

  config 1  moondream3 layer, 1024-token prefill, gate/up Q4_K, down Q6_K
            (also with moondream3's own gelu_erf(h) * (g + 1))
  config 2  the same with the Zipf(1.2) router bias: 16 experts receive none
  config 3  qwen3omni layer (E 128, I 768, SwiGLU) at 1, 8, 32, 64 tokens on
            the path the default rule picks (fused single-token kernel, GEMV,
            GEMM) and at 8 tokens on both product paths
  config 4  the 24-layer stack's layer shape (Q4_K down): one layer at 2048
            tokens through mi_moe_forward_norm (RMSNorm), a 3-layer stack,
            and 4 decode steps each fed the RMSNorm of the previous step's
            final hidden; each layer checked on its own GPU input
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
EPS = 1e-6


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
    assert np.array_equal(bufs["counts"].download(np.int32, (E,)), dbg["counts"]), f"{what}: counts"
    assert np.array_equal(bufs["offsets"].download(np.int32, (E + 1,)), dbg["offsets"]), f"{what}: offsets"
    assert np.array_equal(bufs["perm"].download(np.int32, (T * K,)), dbg["perm"]), f"{what}: permutation"


def _oracle_dict(g: W.GpuLayer) -> dict:
    return oracle_layer_dict(g.download_tables(), g.spec, g.download_router(), g.bias_host)


PREFILL = {
    "md_cfg1": W.CONFIGS[1]["spec"],
    "md_cfg2_skew": W.CONFIGS[2]["spec"],
    "md_cfg1_geglu_erf_gp1": W.md_spec(1, M.TYPE_Q6_K, act=M.ACT_GELU_ERF_GP1),
}


@pytest.mark.parametrize("name", list(PREFILL))
def test_config_prefill_1024(name):
    spec = PREFILL[name]
    T = 1024
    log(f"case {name} T={T}")
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    g = W.GpuLayer(ctx, spec)
    x = W.gen_x(ctx, spec, T)
    out = M.DeviceBuffer(4 * T * spec.D)
    bufs, r = _routing_buffers(T, spec.E, spec.K)
    M.check("forward", ctx.forward(g.layer, x, T, None, out, r))
    got = out.download(np.float32, (T, spec.D))
    xh = x.download(np.float32, (T, spec.D))
    ref, dbg = O.moe_forward(_oracle_dict(g), xh)
    _check_routing(bufs, dbg, T, spec.E, spec.K, name)
    e = rel_l2(got, ref)
    c = dbg["counts"]
    log(f"{name}: T={T} rel-L2 {e:.3e} max-abs {max_abs(got, ref):.3e}; experts used {int((c > 0).sum())}/{spec.E}, "
        f"rows per expert {int(c[c > 0].min())}..{int(c.max())}")
    if spec.router_bias == "zipf":
        assert int((c == 0).sum()) >= W.N_DEAD
    assert e <= TOL
    ctx.close()


@pytest.mark.parametrize("T", [1, 8, 32, 64])
def test_config3_batched_decode(T):
    spec = W.CONFIGS[3]["spec"]
    log(f"case qo_cfg3 T={T}")
    ctx = M.Context(0)
    ctx.reserve(64, spec.D, spec.I, spec.E, spec.K)
    g = W.GpuLayer(ctx, spec)
    OL = _oracle_dict(g)
    x = W.gen_x(ctx, spec, T)
    xh = x.download(np.float32, (T, spec.D))
    ref, dbg = O.moe_forward(OL, xh)
    paths = [("default", 0)]
    if T == 8:
        paths += [("gemv", 1 << 30), ("gemm", 1)]
    for pname, thr in paths:
        ctx.set_gemm_threshold(thr)
        # default: the fused kernels where they apply; gemv / gemm: the chain on that path
        ctx.set_fused_decode(M.DECODE_FUSED if pname == "default" else M.DECODE_CHAIN)
        out = M.DeviceBuffer(4 * T * spec.D)
        bufs, r = _routing_buffers(T, spec.E, spec.K)
        M.check("forward", ctx.forward(g.layer, x, T, None, out, r))
        got = out.download(np.float32, (T, spec.D))
        _check_routing(bufs, dbg, T, spec.E, spec.K, f"qo T={T} {pname}")
        e = rel_l2(got, ref)
        log(f"qo_cfg3 T={T} {pname}: rel-L2 {e:.3e} max-abs {max_abs(got, ref):.3e}, "
            f"touched experts {int((dbg['counts'] > 0).sum())}")
        assert e <= TOL
    ctx.close()


def _rmsnorm_ref(x, eps):
    x64 = x.astype(np.float64)
    return (x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + eps)).astype(np.float32)


def _check_layer_norm(ctx, g, OL, h, T, what, nbuf, out):
    """out = h + MoE(RMSNorm(h)) by mi_moe_forward_norm, against the oracle on
    the GPU's own normalized rows (mi_norm, bit-identical to the norm inside
    the forward) with residual h"""
    spec = g.spec
    nrm = M.make_norm(M.NORM_RMS, EPS)
    bufs, r = _routing_buffers(T, spec.E, spec.K)
    M.check("forward_norm", ctx.forward_norm(g.layer, nrm, h, T, h, out, r))
    M.check("norm", ctx.norm(nrm, h, T, spec.D, nbuf))
    h_in = h.download(np.float32, (T, spec.D))
    n_in = nbuf.download(np.float32, (T, spec.D))
    assert np.allclose(n_in, _rmsnorm_ref(h_in, EPS), rtol=2e-6, atol=1e-7), f"{what}: norm"
    got = out.download(np.float32, (T, spec.D))
    ref, dbg = O.moe_forward(OL, n_in, h_in)
    _check_routing(bufs, dbg, T, spec.E, spec.K, what)
    e = rel_l2(got - h_in, ref - h_in)
    log(f"{what}: rel-L2 {e:.3e} max-abs {max_abs(got, ref):.3e}")
    assert e <= TOL


def test_config4_layer_2048():
    spec = W.md_spec(4, M.TYPE_Q4_K)
    T = 2048
    log(f"case md_cfg4 layer T={T}")
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    g = W.GpuLayer(ctx, spec)
    h = W.gen_x(ctx, spec, T)
    nbuf, out = M.DeviceBuffer(4 * T * spec.D), M.DeviceBuffer(4 * T * spec.D)
    _check_layer_norm(ctx, g, _oracle_dict(g), h, T, "md_cfg4 layer 0 T=2048", nbuf, out)
    ctx.close()


def test_config4_stack_and_fed_back_decode():
    spec = W.md_spec(4, M.TYPE_Q4_K)
    T, n_layers, n_steps = 256, 3, 4
    log(f"case md_cfg4 stack: {n_layers} layers, prefill T={T}, {n_steps} decode steps")
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    layers = [W.GpuLayer(ctx, spec, copy=c) for c in range(n_layers)]
    OLs = [_oracle_dict(g) for g in layers]
    h = W.gen_x(ctx, spec, T)
    h2, nbuf = M.DeviceBuffer(4 * T * spec.D), M.DeviceBuffer(4 * T * spec.D)
    cur, nxt = h, h2
    for li, g in enumerate(layers):
        _check_layer_norm(ctx, g, OLs[li], cur, T, f"md_cfg4 stack prefill layer {li}", nbuf, nxt)
        cur, nxt = nxt, cur
    # decode: the token is the RMSNorm of the last prefill row of the final hidden
    tok, tok2, n1 = M.DeviceBuffer(4 * spec.D), M.DeviceBuffer(4 * spec.D), M.DeviceBuffer(4 * spec.D)
    M.check("copy", M.load().mi_memcpy_d2d(tok.ptr, C.c_void_p(cur.addr + 4 * (T - 1) * spec.D), 4 * spec.D))
    M.check("rmsnorm", ctx.rmsnorm(tok, 1, spec.D, EPS, tok))
    a, b = tok, tok2
    for step in range(n_steps):
        for li, g in enumerate(layers):
            _check_layer_norm(ctx, g, OLs[li], a, 1, f"md_cfg4 decode step {step} layer {li}", n1, b)
            a, b = b, a
        fin = a.download(np.float32, (1, spec.D))
        M.check("rmsnorm", ctx.rmsnorm(a, 1, spec.D, EPS, a))
        assert np.allclose(a.download(np.float32, (1, spec.D)), _rmsnorm_ref(fin, EPS), rtol=2e-6, atol=1e-7)
    b_ids, waits = ctx.take_errors()
    assert (b_ids, waits) == (0, 0)
    ctx.close()


@pytest.mark.parametrize("name,T", [("qo_cfg3", 32), ("qo_cfg3", 64), ("qo_cfg3", 128), ("md_cfg1", 300), ("md_cfg1", 40),
                                    ("qo_cfg3_tiled", 8), ("qo_cfg3_tiled", 16), ("qo_cfg3_tiled", 64),
                                    ("md_cfg1_tiled", 24), ("md_cfg1_tiled", 64)])
def test_gemm_row_tiles(name, T):
    """Every row-tile size of the 4-wave GEMMs at one size: 8-, 32- and 64-row
    tiles (two to four work-groups per CU; 32 rows the default up to 8
    dispatched rows per expert) and 192-row balanced tiles give the same bits (each output's K
    order is the same), and match the oracle.  `_tiled`: the layers carry
    tiled copies of their tables."""
    spec = W.CONFIGS[3]["spec"] if name.startswith("qo_cfg3") else W.CONFIGS[1]["spec"]
    log(f"case {name} T={T} row tiles 32 / 192")
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    g = W.GpuLayer(ctx, spec)
    if name.endswith("_tiled"):
        g.add_tiled(ctx)
    x = W.gen_x(ctx, spec, T)
    xh = x.download(np.float32, (T, spec.D))
    ref, dbg = O.moe_forward(_oracle_dict(g), xh)
    ctx.set_fused_decode(M.DECODE_CHAIN)
    ctx.set_gemm_threshold(1)
    outs = []
    for kind in (1, 2, 4, 5):   # 192-row, 32-row, 8-row (without a dispatch launch), 64-row tiles
        ctx.set_gemm_tiles(kind)
        out = M.DeviceBuffer(4 * T * spec.D)
        bufs, r = _routing_buffers(T, spec.E, spec.K)
        # 192- and 64-row tiles with the dispatch's outputs; 32- and 8-row
        # tiles without (their work-groups find their tiles from the ids, up
        # to 1024 of them)
        M.check("forward", ctx.forward(g.layer, x, T, None, out, r if kind in (1, 5) else None))
        got = out.download(np.float32, (T, spec.D))
        if kind in (1, 5):
            _check_routing(bufs, dbg, T, spec.E, spec.K, f"{name} T={T} tiles {kind}")
        e = rel_l2(got, ref)
        log(f"{name} T={T} row tiles {({1: '192', 2: '32', 4: '8', 5: '64'})[kind]}: rel-L2 {e:.3e} "
            f"max-abs {max_abs(got, ref):.3e}")
        assert e <= TOL
        outs.append(got)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert np.array_equal(outs[0].view(np.uint32), outs[2].view(np.uint32))
    assert np.array_equal(outs[0].view(np.uint32), outs[3].view(np.uint32))
    assert ctx.take_all_errors() == (0, 0, 0)
    ctx.close()
