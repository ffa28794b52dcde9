"""Prefill GEMMs (k_gemm4.hip) through the C ABI.

* mi_mul_mat_id (ggml_mul_mat_id, moondream.cpp:519,537) on Q4_K / Q6_K
  expert tables against the CPU oracle: broadcast (ne11 = 1) and per-slot
  (ne11 = n_used) activations, Q6_K rows of 210 and 630 bytes (odd rows start
  2 bytes past a dword), weight row counts that are not multiples of the
  512-row work-group tile, experts with more than one 128-row tile and
  experts with none.  The GEMM path multiplies fp16-dequantized weights with
  fp16 d*q of the Q8_K activations (fp32 accumulation); the oracle is the
  fp64 dot of the dequantized weights with the dequantized Q8_K rows, so the
  difference is fp16 rounding only: rel-L2 <= 2e-3 (measured ~3e-4).  The
  GEMV path (exact integer dots) is checked beside it.
* Ids repeated inside a token (legal for mul_mat_id) take the dispatch's
  ballot path; T * n_used above one staged chunk of ids (8192) takes several
  chunks.
* Full BASELINE layers at T = 1024 on the GEMM path against the same layer
  on the GEMV path (bit-exact routing, outputs within 5e-3: the two differ by
  fp16 rounding plus the few Q8_K rounding flips of the activations that it
  causes).  The GEMV path is itself held to the oracle by test_gpu_parity.
"""
import ctypes as C
import sys

import numpy as np
import pytest

import mimoe as M
import pyoracle as O
import workloads as W
from _util import cpu_x, max_abs, rel_l2

pytestmark = pytest.mark.gpu

TOL_GEMM_OP = 2e-3
TOL_PATHS = 1e-2


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


MMID_CASES = [
    # type, Kin, N, E, n_used, T, ne11[, ids repeated inside a token]
    (O.TYPE_Q4_K, 512, 300, 8, 4, 300, 1),
    (O.TYPE_Q4_K, 512, 300, 8, 6, 700, 6, True),
    (O.TYPE_Q6_K, 256, 520, 8, 4, 2300, 1, True),
    (O.TYPE_Q4_K, 1024, 2048, 16, 4, 257, 4),
    (O.TYPE_Q6_K, 1024, 2048, 10, 8, 64, 8),
    (O.TYPE_Q6_K, 256, 520, 8, 3, 301, 3),
    (O.TYPE_Q6_K, 768, 2048, 12, 2, 200, 1),
]


@pytest.mark.parametrize("case", MMID_CASES,
                         ids=lambda c: f"t{c[0]}_k{c[1]}_n{c[2]}_e{c[3]}_u{c[4]}_T{c[5]}_b{c[6]}" + ("_rep" if c[7:] else ""))
def test_mul_mat_id_gemm(case):
    type_, Kin, N, E, nu, T, ne11 = case[:7]
    rep = bool(case[7:])
    rng = np.random.default_rng(1000 + Kin + N + T)
    w = (rng.standard_normal((E * N, Kin)) * 0.02).astype(np.float32)
    raw = O.quantize(type_, w).ravel()
    b = rng.standard_normal((T, ne11, Kin)).astype(np.float32)
    # skewed ids: expert 0 takes most rows (several 128-row tiles), the last
    # expert none
    p = np.linspace(3.0, 1.0, E)
    p[-1] = 0.0
    p = p / p.sum()
    ids = np.stack([rng.choice(E, size=nu, replace=rep, p=p) for _ in range(T)]).astype(np.int32)
    if rep:
        assert any(len(set(r)) < nu for r in ids.tolist())
    ref = O.mul_mat_id(type_, raw, Kin, N, E, b, ids)

    ctx = M.Context(0)
    ctx.reserve(T, Kin, Kin, E, nu)
    rd, bd, idd = M.to_device(raw), M.to_device(b), M.to_device(ids)
    dst = M.DeviceBuffer(4 * T * nu * N)
    t_as = M.tensor(rd, type_, [Kin, N, E])
    t_b = M.tensor(bd, M.TYPE_F32, [Kin, ne11, T])
    t_ids = M.tensor(idd, M.TYPE_I32, [nu, T])
    t_dst = M.tensor(dst, M.TYPE_F32, [N, nu, T])
    for path, thr in (("gemm", 1), ("gemv", 1 << 30)):
        ctx.set_gemm_threshold(thr)
        M.check("mul_mat_id", ctx.mul_mat_id(t_as, t_b, t_ids, t_dst))
        got = dst.download(np.float32, (T, nu, N))
        e = rel_l2(got, ref)
        log(f"mul_mat_id {case} {path}: rel-L2 {e:.3e} max-abs {max_abs(got, ref):.3e}")
        assert e <= (TOL_GEMM_OP if path == "gemm" else 1e-4), (path, e)
    ctx.close()


FULL = {
    "md_cfg1": W.CONFIGS[1]["spec"],
    "md_cfg2_skew": W.CONFIGS[2]["spec"],
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


@pytest.mark.parametrize("T", [1, 63, 1024, 1500, 4133])
def test_dispatch_chunks(T):
    """Dispatch (counts / offsets / permutation) against the oracle's stable
    counting sort of the GPU's own top-k ids, across one and several staged
    chunks of ids (8192 ids per chunk)."""
    spec = FULL["qo_cfg3"]
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    g = W.GpuLayer(ctx, spec)
    x = cpu_x(spec, T)
    xd = M.to_device(x)
    out = M.DeviceBuffer(4 * T * spec.D)
    bufs, r = _routing_buffers(T, spec.E, spec.K)
    M.check("forward", ctx.forward(g.layer, xd, T, None, out, r))
    sel = bufs["sel"].download(np.int32, (T, spec.K))
    counts, offsets, perm = O.dispatch(sel, spec.E)
    assert np.array_equal(bufs["counts"].download(np.int32, (spec.E,)), counts)
    assert np.array_equal(bufs["offsets"].download(np.int32, (spec.E + 1,)), offsets)
    assert np.array_equal(bufs["perm"].download(np.int32, (T * spec.K,)), perm)
    log(f"dispatch T={T}: max count {int(counts.max())}")
    ctx.close()


@pytest.mark.parametrize("name", list(FULL))
def test_prefill_gemm_vs_gemv(name):
    spec = FULL[name]
    T = 1024
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    g = W.GpuLayer(ctx, spec)
    x = cpu_x(spec, T)
    res = cpu_x(spec, T, stream=W.S_RES)
    xd, rd = M.to_device(x), M.to_device(res)
    outs, routs = {}, {}
    for path, thr in (("gemm", 1), ("gemv", 1 << 30)):
        ctx.set_gemm_threshold(thr)
        out = M.DeviceBuffer(4 * T * spec.D)
        bufs, r = _routing_buffers(T, spec.E, spec.K)
        M.check("forward", ctx.forward(g.layer, xd, T, rd, out, r))
        outs[path] = out.download(np.float32, (T, spec.D))
        routs[path] = {k: v.download(np.int32, (v.nbytes // 4,)) for k, v in bufs.items()}
    for k in routs["gemm"]:
        assert np.array_equal(routs["gemm"][k], routs["gemv"][k]), k
    counts = routs["gemm"]["counts"]
    e = rel_l2(outs["gemm"] - res, outs["gemv"] - res)
    log(f"{name}: T={T} gemm vs gemv rel-L2 {e:.3e} max-abs {max_abs(outs['gemm'], outs['gemv']):.3e} "
        f"max count {int(counts.max())} empty experts {int((counts == 0).sum())}")
    assert e <= TOL_PATHS
    ctx.close()


def test_prefill_repeatable():
    """Three forwards of the config-1 layer give the same bits: no kernel of
    the prefill path depends on scheduling order or on workspace contents
    left by the previous call (fixed-order sums, dispatch rebuilt, counters
    cleared)."""
    spec = FULL["md_cfg1"]
    T = 1024
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    g = W.GpuLayer(ctx, spec)
    xd = M.to_device(cpu_x(spec, T))
    outs = []
    for _ in range(3):
        out = M.DeviceBuffer(4 * T * spec.D)
        M.check("forward", ctx.forward(g.layer, xd, T, None, out))
        outs.append(out.download(np.float32, (T, spec.D)))
    assert np.isfinite(outs[0]).all()
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))
    ctx.close()

