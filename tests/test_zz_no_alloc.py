"""mi_moe_forward_noalloc (no context, no allocation: the library's per-GPU
file-scope workspace) through the C ABI, against mi_moe_forward on a context
in MI_DECODE_CHAIN mode - the path the no-allocation entry point takes - on
two calls in a row, the second with fewer tokens: outputs and routing bit
for bit, plus the oracle's bar on the first call.  Calls beyond the stated
limits (MI_NOALLOC_MAX_TOKENS tokens, n_expert <= 128, n_ff <= 1024) are
refused with MI_MOE_ERR_CAPACITY and write nothing.
"""
import ctypes as C
import sys

import numpy as np
import pytest

import mimoe as M
import pyoracle as O
import workloads as W
from _util import oracle_layer_dict, rel_l2

pytestmark = pytest.mark.gpu


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _routing(T, E, K):
    bufs = dict(logits=M.DeviceBuffer(4 * T * E), sel=M.DeviceBuffer(4 * T * K), weights=M.DeviceBuffer(4 * T * K),
                counts=M.DeviceBuffer(4 * E), offsets=M.DeviceBuffer(4 * (E + 1)), perm=M.DeviceBuffer(4 * T * K))
    r = M.Routing()
    for k, v in bufs.items():
        setattr(r, k, C.c_void_p(v.addr))
    return bufs, r


def _download(bufs, T, E, K):
    return dict(logits=bufs["logits"].download(np.uint32, (T, E)), sel=bufs["sel"].download(np.int32, (T, K)),
                weights=bufs["weights"].download(np.uint32, (T, K)), counts=bufs["counts"].download(np.int32, (E,)),
                offsets=bufs["offsets"].download(np.int32, (E + 1,)), perm=bufs["perm"].download(np.int32, (T * K,)))


@pytest.mark.parametrize("name,spec,calls", [("md_cfg0", W.CONFIGS[0]["spec"], [40, 7]),
                                             ("qo_cfg3", W.CONFIGS[3]["spec"], [64, 1])])
def test_noalloc_matches_forward(name, spec, calls):
    ctx = M.Context(0)
    ctx.reserve(64, spec.D, spec.I, spec.E, spec.K)
    ctx.set_fused_decode(M.DECODE_CHAIN)
    g = W.GpuLayer(ctx, spec)
    rng = np.random.default_rng(7)
    for i, T in enumerate(calls):
        log(f"case {name} call {i}: T={T}")
        x = rng.standard_normal((T, spec.D)).astype(np.float32)
        res = rng.standard_normal((T, spec.D)).astype(np.float32)
        xd, rd = M.to_device(x), M.to_device(res)
        o1, o2 = M.DeviceBuffer(4 * T * spec.D), M.DeviceBuffer(4 * T * spec.D)
        b1, r1 = _routing(T, spec.E, spec.K)
        b2, r2 = _routing(T, spec.E, spec.K)
        M.check("forward_noalloc", M.forward_noalloc(g.layer, xd, T, rd, o1, r1))
        M.check("forward", ctx.forward(g.layer, xd, T, rd, o2, r2))
        a, b = o1.download(np.float32, (T, spec.D)), o2.download(np.float32, (T, spec.D))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{name} T={T}: output"
        ra, rb = _download(b1, T, spec.E, spec.K), _download(b2, T, spec.E, spec.K)
        for k in ra:
            assert np.array_equal(ra[k], rb[k]), f"{name} T={T}: {k}"
        if i == 0:
            ref, dbg = O.moe_forward(oracle_layer_dict(g.download_tables(), spec, g.download_router(), None), x, res)
            assert np.array_equal(ra["sel"], dbg["sel"])
            e = rel_l2(a - res, ref - res)
            log(f"{name} T={T}: no-alloc = forward bit for bit; vs oracle rel-L2 {e:.3e}")
            assert e <= 1e-2
        else:
            log(f"{name} T={T}: no-alloc = forward bit for bit")
    ctx.close()


def test_noalloc_refuses_beyond_limits():
    spec = W.CONFIGS[0]["spec"]
    ctx = M.Context(0)
    g = W.GpuLayer(ctx, spec)
    T = M.NOALLOC_MAX_TOKENS + 1
    x = M.to_device(np.ones((T, spec.D), np.float32))
    sentinel = np.full((T, spec.D), 3.0, np.float32)
    out = M.DeviceBuffer(4 * T * spec.D).upload(sentinel)
    assert M.forward_noalloc(g.layer, x, T, None, out) == M.ERR_CAPACITY
    L = g.layer
    assert M.forward_noalloc(L, None, 4, None, out) == M.ERR_NULL
    # 200 experts: a valid layer beyond n_expert <= 128 (tiny F32 tables)
    D, E, K, I = 64, 200, 2, 8
    rng = np.random.default_rng(3)
    keep = [M.to_device((rng.standard_normal(n) * 0.1).astype(np.float32)) for n in (E * D, E * 2 * I * D, E * D * I)]
    Lb = M.make_layer(D, E, K, I, keep[0], None, M.tensor(keep[1], M.TYPE_F32, [D, 2 * I, E]), None,
                      M.tensor(keep[2], M.TYPE_F32, [I, D, E]), True, M.ACT_SILU)
    assert M.forward_noalloc(Lb, x, 4, None, out) == M.ERR_CAPACITY
    assert np.array_equal(out.download(np.float32, (T, spec.D)), sentinel), "a refused call wrote output"
    M.check("forward_noalloc", M.forward_noalloc(L, x, 0, None, out))   # empty batch: no-op
    ctx.close()
