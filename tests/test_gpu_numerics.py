"""Numerics of the grouped-GEMM path on inputs that stress its fp16 MFMA
operands, through the C ABI, against the CPU oracle.

The GEMM path multiplies fp16 operands: the activations as fp16(d * q) of
their Q8_K codes, the weights dequantized to fp16 in registers, with fp32
accumulation.  The down product's input is quantized to Q8_K again (ggml's
mul_mat_id quantizes its F32 input), so any difference in the gate/up values
moves some of those codes by one step; that re-quantization, not the fp16
rounding itself, sets most of the error against the integer-exact oracle.
The integer GEMV path runs beside each case as the exact reference point.

Cases (moondream3 widths D 2048 / I 1024, Q4_K gate/up, Q6_K down):
  baseline        N(0, 1) rows, N(0, 0.02) expert weights
  outliers        four channels of every row x 100 (one 256-block per row
                  dominated by its outlier, as in LLM hidden states)
  small weights   expert weights N(0, 0.001): Q4_K scales near 1e-4
  large rows      rows x 30 (|x| up to ~150; gate/up values up to ~130, GLU
                  values up to ~2e4, still inside the fp16 range)
  beyond fp16     one token carries 1e6: its Q8_K block exceeds the fp16
                  range; the operands saturate, the call counts the block
                  (mi_moe_ctx_take_errors fp16_saturated), every output
                  stays finite and the other tokens keep the tolerance; the
                  integer GEMV path (the fallback the header names for such
                  calls) counts nothing and meets it on every token

Bars: logits, ids, permutation bit-exact; output rel-L2 <= 1e-2 (the
north_star tolerance), logged with max-abs for each path; the GEMV path
within 1e-3 (its dots are integer-exact; only the GLU's last-ulp differences
and the Q8_K codes they move remain).  No residual is added, so the measure
is the MoE output itself (with small weights it is far below a residual's
ulp).
"""
import ctypes as C
import sys

import numpy as np
import pytest

import mimoe as M
import pyoracle as O
import workloads as W
from _util import max_abs, rel_l2, small_spec

pytestmark = pytest.mark.gpu

TOL = 1e-2
D, I, E, K, T = 2048, 1024, 16, 4, 256


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _layer(w_std, seed):
    spec = small_spec(f"num_{w_std}", D=D, E=E, K=K, I=I, fused=True, down_type=O.TYPE_Q6_K,
                      act=O.ACT_GELU_TANH, seed=seed, w_std=w_std)
    ctx = M.Context(0)
    ctx.reserve(T, D, I, E, K)
    g = W.GpuLayer(ctx, spec)
    t = g.download_tables()
    OL = dict(D=D, E=E, K=K, I=I, router_w=g.download_router(), router_b=None, gate_type=spec.gate_type,
              gate=t["gate"], fused=True, down_type=spec.down_type, down=t["down"], act=spec.act)
    return ctx, g, OL


def _routing():
    bufs = dict(logits=M.DeviceBuffer(4 * T * E), sel=M.DeviceBuffer(4 * T * K),
                weights=M.DeviceBuffer(4 * T * K), counts=M.DeviceBuffer(4 * E),
                offsets=M.DeviceBuffer(4 * (E + 1)), perm=M.DeviceBuffer(4 * T * K))
    r = M.Routing()
    for k, v in bufs.items():
        setattr(r, k, C.c_void_p(v.addr))
    return bufs, r


def _x(kind, rng):
    x = rng.standard_normal((T, D)).astype(np.float32)
    if kind == "outliers":
        x[:, rng.choice(D, 4, replace=False)] *= 100.0
    elif kind == "large rows":
        x *= 30.0
    elif kind == "beyond fp16":
        x[17, 300] = 1.0e6
    return x


CASES = [("baseline", 0.02), ("outliers", 0.02), ("small weights", 0.001), ("large rows", 0.02),
         ("beyond fp16", 0.02)]


@pytest.mark.parametrize("kind,w_std", CASES, ids=[c[0].replace(" ", "_") for c in CASES])
def test_gemm_numerics(kind, w_std):
    ctx, g, OL = _layer(w_std, 0x5EED4000 + int(1e4 * w_std))
    rng = np.random.default_rng(len(kind))
    x = _x(kind, rng)
    ref, dbg = O.moe_forward(OL, x)
    xd = M.to_device(x)
    errs = {}
    for pname, thr in [("gemv", 1 << 30), ("gemm", 1)]:
        ctx.set_gemm_threshold(thr)
        assert ctx.take_all_errors() == (0, 0, 0)
        out = M.DeviceBuffer(4 * T * D)
        bufs, r = _routing()
        M.check("forward", ctx.forward(g.layer, xd, T, None, out, r))
        got = out.download(np.float32, (T, D))
        sat = ctx.take_all_errors()[2]
        assert np.array_equal(bufs["logits"].download(np.float32, (T, E)).view(np.uint32),
                              dbg["logits"].view(np.uint32)), f"{kind}: logits"
        assert np.array_equal(bufs["sel"].download(np.int32, (T, K)), dbg["sel"]), f"{kind}: ids"
        assert np.array_equal(bufs["perm"].download(np.int32, (T * K,)), dbg["perm"]), f"{kind}: permutation"
        assert np.isfinite(got).all(), f"{kind} {pname}: non-finite output"
        keep = np.ones(T, bool)
        if kind == "beyond fp16" and pname == "gemm":
            assert sat >= 1, "the out-of-range block was not counted"
            keep[17] = False
        else:
            assert sat == 0, f"{kind} {pname}: {sat} blocks counted as saturated"
        e = rel_l2(got[keep], ref[keep])
        errs[pname] = e
        log(f"{kind} (w_std {w_std}) {pname}: rel-L2 {e:.3e} max-abs {max_abs(got[keep], ref[keep]):.3e}"
            f"{f', {sat} fp16-saturated blocks' if sat else ''}")
        assert e <= TOL, (kind, pname)
    assert errs["gemv"] < 1e-3, "the integer path should be exact up to the GLU's last ulp"
    ctx.close()
