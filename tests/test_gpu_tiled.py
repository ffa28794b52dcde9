"""Tiled copies of the Q4_K expert tables (mi_moe_tile_q4k) through the C ABI.

The copy holds the table's bytes in the grouped GEMMs' order: for every
matrix and every 32-row group, block b of the group's 32 rows as 4608
contiguous bytes, then block b + 1.  A layer that carries the copies
(mi_moe_layer.gate_tiled / up_tiled / down_tiled) has its grouped GEMMs read
them, with the same LDS image per column tile as the rows give, so the
forward must equal the one without copies bit for bit; the oracle bounds
both (rel-L2 <= 1e-2).

Bars: the layout equals a numpy reorder of the source bytes exactly; the
forward with copies is bit-identical to the forward without; the argument
checks return the documented status codes.
"""
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


def np_tiled(src: np.ndarray) -> np.ndarray:
    """src: [E, N, row bytes] of Q4_K rows -> the tiled byte order"""
    E, N, rb = src.shape
    nb = rb // 144
    return src.reshape(E, N // 32, 32, nb, 144).transpose(0, 1, 3, 2, 4).reshape(E, N, rb)


@pytest.mark.parametrize("E,N,K", [(1, 32, 256), (3, 64, 512), (5, 96, 2048), (2, 768, 2048)])
def test_tile_layout(E, N, K):
    log(f"tile layout E={E} N={N} K={K}")
    rb = M.row_size(M.TYPE_Q4_K, K)
    rng = np.random.default_rng(E * 1000 + N + K)
    src = rng.integers(0, 256, size=(E, N, rb), dtype=np.uint8)
    ctx = M.Context(0)
    s = M.to_device(src)
    d = M.DeviceBuffer(src.nbytes).zero()
    M.check("mi_moe_tile_q4k", ctx.tile_q4k(M.tensor(s, M.TYPE_Q4_K, [K, N, E]), d))
    M.synchronize()
    got = d.download(np.uint8, (E, N, rb))
    assert np.array_equal(got, np_tiled(src))
    ctx.close()


def test_tile_rejects():
    ctx = M.Context(0)
    K, N, E = 512, 64, 2
    rb = M.row_size(M.TYPE_Q4_K, K)
    s = M.DeviceBuffer(rb * N * E)
    d = M.DeviceBuffer(rb * N * E)
    assert ctx.tile_q4k(M.tensor(s, M.TYPE_Q6_K, [K, N, E]), d) == M.ERR_TYPE
    assert ctx.tile_q4k(M.tensor(s, M.TYPE_Q4_K, [K, 48, E]), d) == M.ERR_SHAPE      # not whole 32-row groups
    padded = M.tensor(s, M.TYPE_Q4_K, [K, 32, E], nb=[144, rb, rb * 64, rb * 64 * E])
    assert ctx.tile_q4k(padded, d) == M.ERR_SHAPE                                   # gap between matrices
    assert ctx.tile_q4k(M.tensor(s, M.TYPE_Q4_K, [K, N, E]), s) == M.ERR_ARG        # in place
    assert ctx.tile_q4k(M.tensor(s, M.TYPE_Q4_K, [K, N, E]), d.addr + 8) == M.ERR_UNSUPPORTED
    ctx.close()


# (name, config, T, chain, GEMM tiles: 0 by shape, 3 the skinny 16-row products)
CASES = ([("qo", 3, 8, True, 0)] + [("qo", 3, T, False, 0) for T in (32, 64, 300)]
         + [("md_q4", 0, T, False, 0) for T in (16, 64, 1024)]
         + [("md_q6down", 1, T, False, 0) for T in (64, 1024)]
         + [("qo_skinny", 3, T, True, 3) for T in (8, 32, 64)] + [("md_q4_skinny", 0, 40, True, 3)])


@pytest.mark.parametrize("name,cfg,T,chain,tiles", CASES, ids=[f"{c[0]}-T{c[2]}" for c in CASES])
def test_forward_tiled_bit_identical(name, cfg, T, chain, tiles):
    spec = W.CONFIGS[cfg]["spec"]
    log(f"case {name} T={T} chain={chain} gemm_tiles={tiles}")
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    if chain:
        ctx.set_fused_decode(M.DECODE_CHAIN)
    if tiles:
        ctx.set_gemm_threshold(1)
        ctx.set_gemm_tiles(tiles)
    g = W.GpuLayer(ctx, spec)
    x = W.gen_x(ctx, spec, T, copy=3)
    outs = []
    for tiled in (False, True):
        if tiled:
            g.add_tiled(ctx)
            assert g.tiled, "no Q4_K table"
        out = M.DeviceBuffer(4 * T * spec.D)
        M.check("forward", ctx.forward(g.layer, x, T, None, out))
        outs.append(out.download(np.float32, (T, spec.D)))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), f"{name} T={T}: tiled differs"
    if T <= 64:
        OL = oracle_layer_dict(g.download_tables(), g.spec, g.download_router(), g.bias_host)
        ref, _ = O.moe_forward(OL, x.download(np.float32, (T, spec.D)))
        e = rel_l2(outs[1], ref)
        log(f"{name} T={T}: tiled bit-identical; rel-L2 {e:.3e} max-abs {max_abs(outs[1], ref):.3e}")
        assert e <= TOL
    else:
        log(f"{name} T={T}: tiled bit-identical")
    ctx.close()


def test_layer_tiled_checks():
    spec = W.CONFIGS[3]["spec"]
    T = 4
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    g = W.GpuLayer(ctx, spec)
    x = W.gen_x(ctx, spec, T)
    out = M.DeviceBuffer(4 * T * spec.D)
    g.add_tiled(ctx)
    keep = M.Tensor.from_buffer_copy(g.layer.up_tiled)   # (the field itself is a view into the layer)
    g.layer.up_tiled = M.Tensor()                    # gate without up
    assert ctx.forward(g.layer, x, T, None, out) == M.ERR_ARG
    g.layer.up_tiled = keep
    q, ttype, Kin, N = g.tables["down"]
    g.layer.down_tiled = M.tensor(g.tiled["down"], ttype, [Kin, N // 2, spec.E])   # other shape than down
    assert ctx.forward(g.layer, x, T, None, out) == M.ERR_SHAPE
    g.layer.down_tiled = M.tensor(g.tiled["down"], M.TYPE_Q6_K, [Kin, N, spec.E])
    assert ctx.forward(g.layer, x, T, None, out) == M.ERR_TYPE
    g.layer.down_tiled = M.tensor(g.tiled["down"], ttype, [Kin, N, spec.E])
    M.check("forward", ctx.forward(g.layer, x, T, None, out))
    ctx.close()
