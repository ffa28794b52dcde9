"""The largest router widths the ABI accepts (E = 256 experts; K = 16 slots
on the kernel chain), through the C ABI, against the CPU oracle, on every
path a call of that size takes: the fused single-token and batched decode
kernels, the chain's GEMV, its 32-row GEMMs without a dispatch launch, and
the 192-row GEMMs; and rows that start 4 bytes past a 16-byte boundary.

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


CASES = [  # (K, T, decode mode, routing outputs wanted)
    (8, 1, M.DECODE_FUSED, True), (8, 5, M.DECODE_FUSED, True), (8, 40, M.DECODE_CHAIN, False),
    (8, 40, M.DECODE_CHAIN, True), (8, 300, M.DECODE_CHAIN, True), (16, 3, M.DECODE_CHAIN, True),
    (16, 20, M.DECODE_CHAIN, False),
]


@pytest.mark.parametrize("K,T,mode,want", CASES, ids=[f"K{k}-T{t}-{'fused' if m == M.DECODE_FUSED else 'chain'}-"
                                                       f"{'routing' if w else 'plain'}" for k, t, m, w in CASES])
def test_e256(K, T, mode, want):
    spec = W.LayerSpec(f"e256_k{K}", 512, 256, K, 256, False, M.TYPE_Q4_K, M.TYPE_Q4_K, M.ACT_SILU, "none",
                       0x5EED7000 + K)
    log(f"case E=256 K={K} T={T}")
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    ctx.set_fused_decode(mode)
    g = W.GpuLayer(ctx, spec)
    OL = oracle_layer_dict(g.download_tables(), g.spec, g.download_router(), g.bias_host)
    x = W.gen_x(ctx, spec, T)
    ref, dbg = O.moe_forward(OL, x.download(np.float32, (T, spec.D)))
    out = M.DeviceBuffer(4 * T * spec.D)
    bufs, r = _routing_buffers(T, spec.E, spec.K)
    M.check("forward", ctx.forward(g.layer, x, T, None, out, r if want else None))
    got = out.download(np.float32, (T, spec.D))
    if want:
        gl = bufs["logits"].download(np.float32, (T, spec.E))
        assert np.array_equal(gl.view(np.uint32), dbg["logits"].view(np.uint32)), "logits"
        assert np.array_equal(bufs["sel"].download(np.int32, (T, K)), dbg["sel"]), "ids"
        assert np.allclose(bufs["weights"].download(np.float32, (T, K)), dbg["w"], rtol=1e-6, atol=1e-7)
        assert np.array_equal(bufs["counts"].download(np.int32, (spec.E,)), dbg["counts"]), "counts"
        assert np.array_equal(bufs["offsets"].download(np.int32, (spec.E + 1,)), dbg["offsets"]), "offsets"
        assert np.array_equal(bufs["perm"].download(np.int32, (T * K,)), dbg["perm"]), "permutation"
    e = rel_l2(got, ref)
    log(f"E=256 K={K} T={T}: rel-L2 {e:.3e} max-abs {max_abs(got, ref):.3e}, "
        f"experts used {int((dbg['counts'] > 0).sum())}/256")
    assert np.isfinite(got).all()
    assert e <= TOL
    ctx.close()


@pytest.mark.parametrize("T", [3, 40, 300])
def test_unaligned_rows(T):
    """x and res 4 bytes past a 16-byte boundary take the routers' and the
    Q8_K passes' element-wise load forms: outputs bit-identical to the same
    rows at an aligned address."""
    spec = W.qo_spec()
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    ctx.set_fused_decode(M.DECODE_CHAIN)
    g = W.GpuLayer(ctx, spec)
    rng = np.random.default_rng(T)
    x = rng.standard_normal((T, spec.D)).astype(np.float32)
    res = rng.standard_normal((T, spec.D)).astype(np.float32)
    outs = []
    for shift in (0, 1):
        xb = M.to_device(np.concatenate([np.zeros(shift, np.float32), x.ravel()]))
        rb = M.to_device(np.concatenate([np.zeros(shift, np.float32), res.ravel()]))
        ob = M.DeviceBuffer(4 * (T * spec.D + 1))
        M.check("forward", ctx.forward(g.layer, C.c_void_p(xb.addr + 4 * shift), T, C.c_void_p(rb.addr + 4 * shift),
                                       C.c_void_p(ob.addr + 4 * shift)))
        outs.append(ob.download(np.float32, (T * spec.D + 1,))[shift:shift + T * spec.D])
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), f"T={T}: unaligned rows differ"
    log(f"T={T}: unaligned x / res / out bit-identical to aligned")
    ctx.close()
