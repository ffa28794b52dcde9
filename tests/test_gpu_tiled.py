"""Tiled copies of the expert tables (mi_moe_tile) through the C ABI.

Q4_K: the table's bytes in the grouped GEMMs' order (for every matrix and
every 32-row group, block b of the group's 32 rows as 4608 contiguous bytes,
then block b + 1).  Q6_K (down tables): per 32-row group and block, 8 KB of
the 6-bit codes merged into bytes in the order the GEMM's lanes take them
and 1 KB of fp16 d * scale.  A layer that carries the copies
(mi_moe_layer.gate_tiled / up_tiled / down_tiled) has its grouped GEMMs read
them, building the same fp16 operands as from the rows, so the forward must
equal the one without copies bit for bit; the oracle bounds both (rel-L2 <=
1e-2).

Bars: the layouts equal numpy models of them exactly (the Q6_K model
decodes the codes from the block fields, the copy must match); the forward
with copies is bit-identical to the forward without; the argument checks
return the documented status codes.
"""
import sys

import numpy as np
import pytest

import mimoe as M
import pyoracle as O
import workloads as W
from _tiled_model import np_tiled, np_tiled_q6k
from _util import max_abs, oracle_layer_dict, rel_l2, small_spec

pytestmark = pytest.mark.gpu

TOL = 1e-2


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("E,N,K", [(1, 32, 256), (3, 64, 512), (5, 96, 2048), (2, 768, 2048)])
def test_tile_layout(E, N, K):
    log(f"tile layout Q4_K E={E} N={N} K={K}")
    rb = M.row_size(M.TYPE_Q4_K, K)
    rng = np.random.default_rng(E * 1000 + N + K)
    src = rng.integers(0, 256, size=(E, N, rb), dtype=np.uint8)
    ctx = M.Context(0)
    s = M.to_device(src)
    t = M.tensor(s, M.TYPE_Q4_K, [K, N, E])
    assert M.tiled_bytes(t) == src.nbytes
    d = M.DeviceBuffer(src.nbytes).zero()
    desc = M.Tensor()
    M.check("mi_moe_tile", ctx.tile(t, d, desc))
    M.synchronize()
    got = d.download(np.uint8, (E, N, rb))
    assert np.array_equal(got, np_tiled(src))
    assert desc.data == d.addr and desc.type == M.TYPE_Q4_K and list(desc.ne) == [K, N, E, 1]
    assert list(desc.nb)[:3] == [144, rb, rb * N]
    ctx.close()


@pytest.mark.parametrize("E,N,K,off", [(1, 32, 256, 0), (2, 64, 1024, 2), (3, 96, 512, 4)])
def test_tile_layout_q6k(E, N, K, off):
    """random blocks with finite d (the scale chunk compares fp16 bits); off:
    the table starts 2 / 4 bytes into its buffer (Q6_K rows are 2-byte aligned)"""
    log(f"tile layout Q6_K E={E} N={N} K={K} offset {off}")
    rb = M.row_size(M.TYPE_Q6_K, K)
    rng = np.random.default_rng(E * 100 + N + K)
    src = rng.integers(0, 256, size=(E, N, rb // 210, 210), dtype=np.uint8)
    src[..., 208:210] = rng.uniform(-0.01, 0.01, size=src.shape[:-1] + (1,)).astype(np.float16).view(np.uint8)
    src = src.reshape(E, N, rb)
    ctx = M.Context(0)
    buf = M.DeviceBuffer(src.nbytes + 16)
    buf.upload(src, offset=off)
    t = M.tensor(buf, M.TYPE_Q6_K, [K, N, E], offset=off)
    nbytes = M.tiled_bytes(t)
    assert nbytes == E * N * (K // 256) * 288
    d = M.DeviceBuffer(nbytes).zero()
    desc = M.Tensor()
    M.check("mi_moe_tile", ctx.tile(t, d, desc))
    M.synchronize()
    got = d.download(np.uint8, (E, N // 32, K // 256, 9216))
    want = np_tiled_q6k(src)
    assert np.array_equal(got, want)
    assert list(desc.nb)[:3] == [288, 288 * (K // 256), 288 * (K // 256) * N]
    ctx.close()


def test_tile_rejects():
    ctx = M.Context(0)
    K, N, E = 512, 64, 2
    rb = M.row_size(M.TYPE_Q4_K, K)
    s = M.DeviceBuffer(rb * N * E)
    d = M.DeviceBuffer(2 * rb * N * E)
    assert ctx.tile(M.tensor(s, M.TYPE_Q8_0, [K, N, E]), d) == M.ERR_TYPE
    assert M.tiled_bytes(M.tensor(s, M.TYPE_F32, [K, N, E])) == M.ERR_TYPE
    assert ctx.tile(M.tensor(s, M.TYPE_Q4_K, [K, 48, E]), d) == M.ERR_SHAPE      # not whole 32-row groups
    padded = M.tensor(s, M.TYPE_Q4_K, [K, 32, E], nb=[144, rb, rb * 64, rb * 64 * E])
    assert ctx.tile(padded, d) == M.ERR_SHAPE                                   # gap between matrices
    assert ctx.tile(M.tensor(s, M.TYPE_Q4_K, [K, N, E]), s) == M.ERR_ARG        # in place
    assert ctx.tile(M.tensor(s, M.TYPE_Q4_K, [K, N, E]), d.addr + 8) == M.ERR_UNSUPPORTED
    assert ctx.tile(M.tensor(s, M.TYPE_Q4_K, [K, N, E], offset=4), d) == M.ERR_UNSUPPORTED
    q6 = M.tensor(s, M.TYPE_Q6_K, [K, N // 2, E])
    assert ctx.tile(q6, s.addr + 16) == M.ERR_ARG                               # the copy overlaps its source
    ctx.close()


# (name, config, T, chain, GEMM tiles: 0 by shape, 3 the skinny 16-row products)
CASES = ([("qo", 3, 8, True, 0)] + [("qo", 3, T, False, 0) for T in (32, 64, 300)]
         + [("md_q4", 0, T, False, 0) for T in (16, 64, 1024)]
         + [("md_q6down", 1, T, False, 0) for T in (64, 300, 1024)] + [("md_q6down_skew", 2, 1024, False, 0)]
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
    dbuf = g.tiled["down"]._buf
    g.layer.down_tiled = M.tensor(dbuf, ttype, [Kin, N // 2, spec.E])   # other shape than down
    assert ctx.forward(g.layer, x, T, None, out) == M.ERR_SHAPE
    g.layer.down_tiled = M.tensor(dbuf, M.TYPE_Q6_K, [Kin, N, spec.E])   # other type than down
    assert ctx.forward(g.layer, x, T, None, out) == M.ERR_TYPE
    g.layer.down_tiled = M.tensor(dbuf, ttype, [Kin, N, spec.E])
    M.check("forward", ctx.forward(g.layer, x, T, None, out))
    g.layer.gate_tiled = M.tensor(dbuf, M.TYPE_Q6_K, [spec.D, spec.I, spec.E])   # Q6_K copies: down only
    assert ctx.forward(g.layer, x, T, None, out) == M.ERR_TYPE
    ctx.close()


@pytest.mark.parametrize("down_type", [M.TYPE_Q4_K, M.TYPE_Q6_K], ids=["q4k_down", "q6k_down"])
def test_expert_ffn_tiled_bit_identical(down_type):
    """The table form (caller's ids, gate/up and down ids different) on the
    grouped GEMMs reads the copies too: bit-identical to the rows."""
    spec = small_spec(f"tiled_tbl_{down_type}", D=512, E=8, K=3, I=256, fused=False, down_type=down_type,
                      act=O.ACT_SILU, seed=0x5EED3200 + down_type)
    T = 96
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    ctx.set_gemm_threshold(1)
    g = W.GpuLayer(ctx, spec)
    rng = np.random.default_rng(down_type)
    x = M.to_device(rng.standard_normal((T, spec.D)).astype(np.float32))
    res = M.to_device(rng.standard_normal((T, spec.D)).astype(np.float32))
    gu = M.to_device(rng.integers(0, spec.E, size=(T, spec.K)).astype(np.int32))
    dn = M.to_device(rng.integers(0, spec.E, size=(T, spec.K)).astype(np.int32))
    w = M.to_device(rng.random((T, spec.K)).astype(np.float32))
    outs = []
    for tiled in (False, True):
        if tiled:
            g.add_tiled(ctx)
            assert set(g.tiled) == {"gate", "up", "down"}
        out = M.DeviceBuffer(4 * T * spec.D)
        M.check("expert_ffn", ctx.expert_ffn(g.layer, x, T, res, gu, dn, w, out))
        outs.append(out.download(np.float32, (T, spec.D)))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    log(f"expert_ffn down type {down_type}: tiled bit-identical")
    ctx.close()


EDGE = [  # (name, D, E, K, I, fused, down type, T)
    ("e256_k8", 512, 256, 8, 256, False, M.TYPE_Q4_K, 40),
    ("e256_k16", 512, 256, 16, 256, False, M.TYPE_Q4_K, 300),
    ("d256_fused_q6", 256, 16, 4, 256, True, M.TYPE_Q6_K, 96),
    ("d256_fused_q6_small", 256, 16, 4, 256, True, M.TYPE_Q6_K, 5),
]


@pytest.mark.parametrize("name,D,E,K,I,fused,dt,T", EDGE, ids=[e[0] for e in EDGE])
def test_tiled_edge_shapes(name, D, E, K, I, fused, dt, T):
    """Tiled copies at the widest router (E = 256, K up to 16) and at rows
    of one 256-value block (D = 256: one Q4_K / Q6_K block per row, the
    tile's block stride is the whole group), on the kernel chain: the output
    equals the rows' bit for bit and the oracle's to 1e-2."""
    spec = W.LayerSpec(name, D, E, K, I, fused, M.TYPE_Q4_K, dt, M.ACT_SILU if not fused else M.ACT_GELU_ERF_GP1,
                       "none", 0x5EED7400 + E + K + D)
    log(f"case {name} T={T}")
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    ctx.set_fused_decode(M.DECODE_CHAIN)
    ctx.set_gemm_threshold(1)
    g = W.GpuLayer(ctx, spec)
    x = W.gen_x(ctx, spec, T, copy=5)
    outs = []
    for tiled in (False, True):
        if tiled:
            g.add_tiled(ctx)
        out = M.DeviceBuffer(4 * T * spec.D)
        M.check("forward", ctx.forward(g.layer, x, T, None, out))
        outs.append(out.download(np.float32, (T, spec.D)))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), name
    OL = oracle_layer_dict(g.download_tables(), g.spec, g.download_router(), g.bias_host)
    ref, _ = O.moe_forward(OL, x.download(np.float32, (T, spec.D)))
    e = rel_l2(outs[1], ref)
    log(f"{name} T={T}: tiled bit-identical; rel-L2 {e:.3e} max-abs {max_abs(outs[1], ref):.3e}")
    assert e <= TOL
    ctx.close()
