"""Batched decode (2..16 tokens) in one kernel (k_decodeb, k_decode.hip) against
the CPU oracle and against the separate-kernel chain.

Bars, as for every forward path: router logits, expert ids and the dispatch of
the T*K ids (counts / offsets / permutation) bit-exact; routing weights within
1e-6 relative; MoE output rel-L2 <= 1e-2 against the oracle.  The kernel and
the GEMV chain (forced: the default rule takes the GEMMs from half a row per
expert) use the same integer dots and Q8_K code but sum the fp32 dot
partials in different orders, so an activation on a Q8_K rounding boundary can
land on either side: the two must agree to a few such flips (rel-L2 <= 5e-3).

Launches on one context share the epoch-tagged hand-off words with the
single-token kernel, so one case runs batches of different sizes interleaved
with single tokens and the chain; the rescue case forces the fallback that
makes the plain launch safe (a work-group computes any unit it waited too long
for) and checks the bits against the default schedule.
"""
import ctypes as C
import sys

import numpy as np
import pytest

import mimoe as M
import pyoracle as O
import workloads as W
from _util import cpu_x, max_abs, oracle_layer_dict, rel_l2, small_spec

pytestmark = pytest.mark.gpu

TOL_REL_L2 = 1e-2
TOL_PATHS = 5e-3
TMAX = 16


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


CASES = {
    "md_small_q6": small_spec("md_small_q6", D=512, E=8, K=2, I=256, fused=True, down_type=O.TYPE_Q6_K,
                              act=O.ACT_GELU_ERF_GP1),
    "qo_small": small_spec("qo_small", D=512, E=16, K=4, I=256, fused=False, act=O.ACT_SILU,
                           seed=0x5EED1001),
    "md_d256_k3": small_spec("md_d256_k3", D=256, E=8, K=3, I=512, fused=True, act=O.ACT_GELU_TANH,
                             seed=0x5EED1002),
    "md_d1024_q6": small_spec("md_d1024_q6", D=1024, E=32, K=8, I=768, fused=True, down_type=O.TYPE_Q6_K,
                              act=O.ACT_GELU_ERF, seed=0x5EED1003),
    "md_cfg0": W.CONFIGS[0]["spec"],
    "qo_cfg3": W.CONFIGS[3]["spec"],
}


def _routing_buffers(T, E, K):
    bufs = dict(logits=M.DeviceBuffer(4 * T * E), sel=M.DeviceBuffer(4 * T * K),
                weights=M.DeviceBuffer(4 * T * K), counts=M.DeviceBuffer(4 * E),
                offsets=M.DeviceBuffer(4 * (E + 1)), perm=M.DeviceBuffer(4 * T * K))
    r = M.Routing()
    for k, v in bufs.items():
        setattr(r, k, C.c_void_p(v.addr))
    return bufs, r


def _run(ctx, layer, spec, x, res, mode):
    T = x.shape[0]
    ctx.set_fused_decode(mode)
    # the chain on the integer-dot GEMV (the kernel's arithmetic; the default
    # rule would take the fp16 GEMMs from half a row per expert)
    ctx.set_gemm_threshold(1 << 30 if mode == M.DECODE_CHAIN else 0)
    ctx.set_profiling(True)
    xd, rd = M.to_device(x), M.to_device(res)
    out = M.DeviceBuffer(4 * T * spec.D)
    bufs, r = _routing_buffers(T, spec.E, spec.K)
    M.check("forward", ctx.forward(layer, xd, T, rd, out, r))
    stages = [n for n, _ in ctx.stage_times()]
    ctx.set_profiling(False)
    got = out.download(np.float32, (T, spec.D))
    rt = dict(logits=bufs["logits"].download(np.float32, (T, spec.E)),
              sel=bufs["sel"].download(np.int32, (T, spec.K)),
              weights=bufs["weights"].download(np.float32, (T, spec.K)),
              counts=bufs["counts"].download(np.int32, (spec.E,)),
              offsets=bufs["offsets"].download(np.int32, (spec.E + 1,)),
              perm=bufs["perm"].download(np.int32, (T * spec.K,)))
    return got, rt, stages


def _check(tag, got, rt, ref, res, dbg):
    assert np.array_equal(rt["logits"].view(np.uint32), dbg["logits"].view(np.uint32)), f"{tag}: logits"
    assert np.array_equal(rt["sel"], dbg["sel"]), f"{tag}: ids"
    assert np.allclose(rt["weights"], dbg["w"], rtol=1e-6, atol=1e-7), f"{tag}: weights"
    assert np.array_equal(rt["counts"], dbg["counts"]), f"{tag}: counts"
    assert np.array_equal(rt["offsets"], dbg["offsets"]), f"{tag}: offsets"
    assert np.array_equal(rt["perm"], dbg["perm"]), f"{tag}: permutation"
    assert np.isfinite(got).all(), f"{tag}: non-finite output"
    e = rel_l2(got - res, ref - res)
    assert e <= TOL_REL_L2, (tag, e)
    return e


def _setup(spec, T):
    ctx = M.Context(0)
    ctx.reserve(TMAX, spec.D, spec.I, spec.E, spec.K)
    g = W.GpuLayer(ctx, spec)
    L = oracle_layer_dict(g.download_tables(), spec, g.download_router(), g.bias_host)
    x = cpu_x(spec, T)
    res = cpu_x(spec, T, stream=W.S_RES)
    ref, dbg = O.moe_forward(L, x, res)
    return ctx, g, L, x, res, ref, dbg


def _expert_bytes(spec):
    row = lambda t, k: k // 256 * (144 if t == O.TYPE_Q4_K else 210)  # noqa: E731
    gu = (2 if spec.fused else 1) * spec.I * row(spec.gate_type, spec.D)
    return gu + (0 if spec.fused else spec.I * row(spec.gate_type, spec.D)) + spec.D * row(spec.down_type, spec.I)


def _batched_kernel_expected(spec, T):
    # experts above 2 MiB: only at most one dispatched row per expert on average
    return not (_expert_bytes(spec) > 2 << 20 and T * spec.K > spec.E)


@pytest.mark.parametrize("name", list(CASES))
def test_decodeb_parity(name):
    spec = CASES[name]
    ctx, g, L, x, res, ref, dbg = _setup(spec, TMAX)
    for T in (2, 3, 8, 16):
        log(f"case {name} T={T}")
        xs, rs = x[:T], res[:T]
        r_ref, r_dbg = O.moe_forward(L, xs, rs)
        got_f, rt_f, st_f = _run(ctx, g.layer, spec, xs, rs, M.DECODE_FUSED)
        if not _batched_kernel_expected(spec, T):
            assert "decodeb" not in st_f, f"batched kernel taken past one row per expert: {st_f}"
            e_f = _check(f"{name} T={T} fused mode (chain)", got_f, rt_f, r_ref, rs, r_dbg)
            log(f"{name} T={T}: {T * spec.K} rows over {spec.E} experts: chain, rel-L2 {e_f:.3e}")
            continue
        assert "decodeb" in st_f, f"batched kernel not taken: {st_f}"
        got_c, rt_c, st_c = _run(ctx, g.layer, spec, xs, rs, M.DECODE_CHAIN)
        assert "decodeb" not in st_c
        e_f = _check(f"{name} T={T} fused", got_f, rt_f, r_ref, rs, r_dbg)
        e_c = _check(f"{name} T={T} chain", got_c, rt_c, r_ref, rs, r_dbg)
        e_p = rel_l2(got_f - rs, got_c - rs)
        log(f"{name} T={T}: fused rel-L2 {e_f:.3e} (max-abs {max_abs(got_f, r_ref):.3e}), chain {e_c:.3e}, "
            f"fused vs chain {e_p:.3e}, touched experts {int((r_dbg['counts'] > 0).sum())}")
        assert e_p <= TOL_PATHS, e_p
    assert ctx.take_errors() == (0, 0)
    ctx.close()


@pytest.mark.parametrize("polls", [0, 1])
def test_decodeb_rescue(polls):
    """With 0 polls nearly every work-group recomputes every unit it does not
    see complete at its first look; the output must be the default
    schedule's, bit for bit."""
    spec = CASES["md_d1024_q6"]
    T = 8
    ctx, g, L, x, res, ref, dbg = _setup(spec, T)
    for rep in range(2):
        ctx.set_decode_rescue(64)
        base, _, st = _run(ctx, g.layer, spec, x, res, M.DECODE_FUSED)
        assert "decodeb" in st
        ctx.set_decode_rescue(polls)
        got, rt, st = _run(ctx, g.layer, spec, x, res, M.DECODE_FUSED)
        assert "decodeb" in st
        _check(f"rescue_{polls}", got, rt, ref, res, dbg)
        assert np.array_equal(got.view(np.uint32), base.view(np.uint32)), "rescued units changed the bits"
    ctx.set_decode_rescue(64)
    assert ctx.take_errors() == (0, 0)
    log(f"batched rescue after {polls} polls: bit-identical to the default schedule")
    ctx.close()


def test_decodeb_sequence():
    """One context: batches of 8, 3, 16 and 2 tokens interleaved with single
    tokens (the single-token kernel) and the chain, twice over: the epoch-
    tagged words of one launch never satisfy a wait of the next."""
    spec = CASES["md_cfg0"]
    ctx, g, L, x, res, ref, dbg = _setup(spec, TMAX)
    for rep in range(2):
        for T, mode in ((8, M.DECODE_FUSED), (1, M.DECODE_FUSED), (3, M.DECODE_FUSED), (16, M.DECODE_CHAIN),
                        (16, M.DECODE_FUSED), (1, M.DECODE_FUSED), (2, M.DECODE_FUSED)):
            xs, rs = x[:T], res[:T]
            r_ref, r_dbg = O.moe_forward(L, xs, rs)
            got, rt, st = _run(ctx, g.layer, spec, xs, rs, mode)
            fused_b = mode == M.DECODE_FUSED and _batched_kernel_expected(spec, T)
            want = "decode1" if T == 1 else "decodeb" if fused_b else None
            if want:
                assert want in st, (T, st)
            elif T > 1:
                assert "decodeb" not in st, (T, st)
            e = _check(f"seq rep {rep} T={T}", got, rt, r_ref, rs, r_dbg)
            log(f"sequence rep {rep} T={T} {'fused' if mode == M.DECODE_FUSED else 'chain'}: rel-L2 {e:.3e}")
    assert ctx.take_errors() == (0, 0)
    ctx.close()
