"""The drop-in boundary's caller-routed entry points on k-quant tables,
through the C ABI and through the C++ vqa::moe mirror, against the CPU
oracle.

  mi_moe_expert_ffn        the table form build_expert_ffn_table_res
                           (moe_compute.hpp:66-71, moe_compute.cpp:93-136) and
                           the expert-cache driver's default graph B, which
                           always passes two ids tensors
                           (moe_decode_driver.hpp:505-509): Q4_K gate/up with
                           Q4_K or Q6_K down, on the GEMV and the GEMM paths,
                           with one ids pointer, two buffers of equal contents,
                           and two buffers of different contents (the oracle's
                           separate down ids)
  vqa::moe mirror          build_expert_ffn_table_res in C++ on the same
                           tables with two ids buffers (its self-test binary's
                           table mode)
  ids outside [0, E)       ids E and -1: the slot contributes nothing (the
                           oracle with that slot's weight 0), mi_mul_mat_id
                           writes zero rows, mi_moe_ctx_take_errors counts them
  mi_top_k                 ggml_top_k through the ABI on rows with padded
                           strides, against np.argsort(-x, kind="stable")
                           (the reference's own oracle convention,
                           scripts/parity_nemotronomni_seg.py:228,363,376)

Bars: rel-L2 <= 1e-2 against the oracle (measured values logged); ids and
zero rows exact; the padding of strided outputs untouched.
"""
import pathlib
import subprocess
import sys

import numpy as np
import pytest

import mimoe as M
import pyoracle as O
import workloads as W
from _util import max_abs, rel_l2, small_spec

pytestmark = pytest.mark.gpu

ROOT = pathlib.Path(__file__).resolve().parents[1]
SELFTEST = ROOT / "skyvision.cpp_amd" / "host" / "vqa_moe_selftest"
TOL = 1e-2


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _layer(down_type, seed, D=512, E=8, K=3, I=256):
    spec = small_spec(f"tbl_{down_type}", D=D, E=E, K=K, I=I, fused=False, down_type=down_type,
                      act=O.ACT_SILU, seed=seed)
    ctx = M.Context(0)
    ctx.reserve(128, D, I, E, K)
    g = W.GpuLayer(ctx, spec)
    t = g.download_tables()
    OL = dict(D=D, E=E, K=K, I=I, router_w=None, router_b=None, gate_type=spec.gate_type, gate=t["gate"],
              up=t["up"], fused=False, down_type=down_type, down=t["down"], act=spec.act)
    return ctx, g, spec, OL, t


def _routing(rng, T, E, K):
    gu = rng.integers(0, E, size=(T, K)).astype(np.int32)        # repeats inside a token allowed
    dn = rng.integers(0, E, size=(T, K)).astype(np.int32)
    w = rng.random((T, K)).astype(np.float32)
    return gu, dn, w


@pytest.mark.parametrize("down_type", [M.TYPE_Q4_K, M.TYPE_Q6_K], ids=["q4k_down", "q6k_down"])
@pytest.mark.parametrize("path", ["gemv", "gemm"])
def test_expert_ffn_kquant_two_ids(down_type, path):
    ctx, g, spec, OL, _ = _layer(down_type, 0x5EED3000 + down_type)
    ctx.set_gemm_threshold(1 if path == "gemm" else 1 << 30)
    rng = np.random.default_rng(down_type * 10 + (path == "gemm"))
    for T in [5, 96]:
        x = rng.standard_normal((T, spec.D)).astype(np.float32)
        res = rng.standard_normal((T, spec.D)).astype(np.float32)
        gu, dn, w = _routing(rng, T, spec.E, spec.K)
        xd, rd, wd = M.to_device(x), M.to_device(res), M.to_device(w)
        gud, gud2, dnd = M.to_device(gu), M.to_device(gu), M.to_device(dn)
        out = M.DeviceBuffer(4 * T * spec.D)
        for mode, a, b, dsel in [("one pointer", gud, gud, gu), ("two equal buffers", gud, gud2, gu),
                                 ("two different buffers", gud, dnd, dn)]:
            M.check("expert_ffn", ctx.expert_ffn(g.layer, xd, T, rd, a, b, wd, out))
            got = out.download(np.float32, (T, spec.D))
            ref, _ = O.moe_forward(OL, x, res, sel_in=gu, down_sel_in=dsel, w_in=w)
            e = rel_l2(got - res, ref - res)
            log(f"expert_ffn {path} down type {down_type} T={T} {mode}: rel-L2 {e:.3e} max-abs {max_abs(got, ref):.3e}")
            assert e <= TOL, mode
        # the down ids really drive the down product
        ref_same, _ = O.moe_forward(OL, x, res, sel_in=gu, w_in=w)
        assert rel_l2(got - res, ref_same - res) > 0.1
    assert ctx.take_errors() == (0, 0)
    ctx.close()


def test_mirror_table_form_two_ids(tmp_path):
    if not SELFTEST.exists():
        pytest.fail(f"{SELFTEST} is not built: run __graft_entry__.build()")
    ctx, g, spec, OL, t = _layer(M.TYPE_Q6_K, 0x5EED3100)
    ctx.close()
    rng = np.random.default_rng(31)
    T = 40
    x = rng.standard_normal((T, spec.D)).astype(np.float32)
    res = rng.standard_normal((T, spec.D)).astype(np.float32)
    gu, dn, w = _routing(rng, T, spec.E, spec.K)
    for thr, pname in [(1 << 30, "gemv"), (1, "gemm")]:
        d = tmp_path / pname
        d.mkdir()
        (d / "meta.txt").write_text(f"{T} {spec.D} {spec.I} {spec.E} {spec.K} {spec.gate_type} {spec.down_type} "
                                    f"0 0 {thr}\n")
        for name, a in [("x", x), ("res", res), ("gate", t["gate"]), ("up", t["up"]), ("down", t["down"]),
                        ("ids_gu", gu), ("ids_dn", dn), ("w", w)]:
            (d / f"{name}.bin").write_bytes(np.ascontiguousarray(a).tobytes())
        r = subprocess.run([str(SELFTEST), "--table", str(d)], capture_output=True, text=True, timeout=120)
        log(r.stderr.strip())
        assert r.returncode == 0, r.stderr
        got = np.fromfile(d / "out.bin", np.float32).reshape(T, spec.D)
        ref, _ = O.moe_forward(OL, x, res, sel_in=gu, down_sel_in=dn, w_in=w)
        e = rel_l2(got - res, ref - res)
        log(f"vqa::moe::build_expert_ffn_table_res {pname}, two ids buffers: rel-L2 {e:.3e}")
        assert e <= TOL


@pytest.mark.parametrize("path", ["gemv", "gemm"])
def test_out_of_range_ids(path):
    ctx, g, spec, OL, t = _layer(M.TYPE_Q4_K, 0x5EED3200)
    ctx.set_gemm_threshold(1 if path == "gemm" else 1 << 30)
    assert ctx.take_errors() == (0, 0)
    rng = np.random.default_rng(32)
    T, E, K = 24, spec.E, spec.K
    x = rng.standard_normal((T, spec.D)).astype(np.float32)
    res = rng.standard_normal((T, spec.D)).astype(np.float32)
    gu, dn, w = _routing(rng, T, E, K)
    gu_bad, dn_bad = gu.copy(), dn.copy()
    gu_bad[0, 1], gu_bad[5, 0], dn_bad[7, 2], dn_bad[5, 0] = E, -1, E + 3, -7
    dead = (gu_bad < 0) | (gu_bad >= E) | (dn_bad < 0) | (dn_bad >= E)
    w_live = np.where(dead, 0.0, w).astype(np.float32)
    out = M.DeviceBuffer(4 * T * spec.D)
    M.check("expert_ffn", ctx.expert_ffn(g.layer, M.to_device(x), T, M.to_device(res), M.to_device(gu_bad),
                                         M.to_device(dn_bad), M.to_device(w), out))
    got = out.download(np.float32, (T, spec.D))
    assert np.isfinite(got).all()
    ref, _ = O.moe_forward(OL, x, res, sel_in=np.where(dead, 0, gu), down_sel_in=np.where(dead, 0, dn),
                           w_in=w_live)
    e = rel_l2(got - res, ref - res)
    log(f"bad ids {path}: {int(dead.sum())} dead slots, rel-L2 {e:.3e} vs the oracle with their weights 0")
    assert e <= TOL
    assert ctx.take_errors() == (4, 0)      # two in each ids buffer
    assert ctx.take_errors() == (0, 0)      # taking clears
    # mul_mat_id: the rows of bad ids are zeros, the others are the oracle's
    ids = gu.copy()
    ids[3, 0], ids[10, 2] = -1, E
    bad = (ids < 0) | (ids >= E)
    Kin, N = spec.D, spec.I
    b = rng.standard_normal((T, 1, Kin)).astype(np.float32)
    dst = M.DeviceBuffer(4 * T * K * N).upload(np.full((T, K, N), 9.0, np.float32))
    rc = ctx.mul_mat_id(g.tensor("gate"), M.tensor(M.to_device(b), M.TYPE_F32, [Kin, 1, T]),
                        M.tensor(M.to_device(ids), M.TYPE_I32, [K, T]), M.tensor(dst, M.TYPE_F32, [N, K, T]))
    M.check("mul_mat_id", rc)
    gotm = dst.download(np.float32, (T, K, N))
    assert np.all(gotm[bad] == 0.0)
    refm = O.mul_mat_id(spec.gate_type, t["gate"], Kin, N, E, b, np.where(bad, 0, ids))
    assert rel_l2(gotm[~bad], refm[~bad]) <= TOL
    assert ctx.take_errors() == (2, 0)
    ctx.close()


@pytest.mark.parametrize("E,k", [(64, 8), (128, 8), (5, 5), (256, 16)])
def test_top_k_strided(E, k):
    ctx = M.Context(0)
    rng = np.random.default_rng(E + k)
    T = 1000
    lda, ldd = E + 13, k + 3                       # padded row strides (elements)
    a = rng.standard_normal((T, lda)).astype(np.float32)
    a[0, :E] = 0.5                                  # all equal -> ids 0..k-1
    a[1, :E] = np.round(a[1, :E] * 2) / 2           # many ties
    a[2, :E] = -np.inf
    a[2, E - 1] = np.inf
    sentinel = np.full((T, ldd), -77, np.int32)
    ad, dd = M.to_device(a), M.DeviceBuffer(4 * T * ldd).upload(sentinel)
    ta = M.tensor(ad, M.TYPE_F32, [E, T], nb=[4, 4 * lda, 4 * lda * T, 4 * lda * T])
    td = M.tensor(dd, M.TYPE_I32, [k, T], nb=[4, 4 * ldd, 4 * ldd * T, 4 * ldd * T])
    M.check("top_k", ctx.top_k(ta, k, td))
    got = dd.download(np.int32, (T, ldd))
    ref = np.argsort(-a[:, :E].astype(np.float64), axis=1, kind="stable")[:, :k]
    assert np.array_equal(got[:, :k], ref)
    assert np.all(got[:, k:] == -77), "padding written"
    # refused: k > E, a wrong dst shape
    assert ctx.top_k(ta, E + 1, td) == M.ERR_SHAPE
    td_bad = M.tensor(dd, M.TYPE_I32, [k, T + 1], nb=[4, 4 * ldd, 4 * ldd * T, 4 * ldd * T])
    assert ctx.top_k(ta, k, td_bad) == M.ERR_SHAPE
    log(f"top_k E={E} k={k}: {T} rows with strides {lda}/{ldd} match the stable argsort")
    ctx.close()
