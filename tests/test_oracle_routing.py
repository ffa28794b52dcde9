"""Pins the oracle's routing, product and layer functions independently of
the GPU: each check below uses a closed form, a textbook routine, an
invariant or brute force, chosen so that a dropped term, a wrong index or a
transposed operand in the C restatement fails it.

  router_logits    fp64 dot (numpy) rounded to fp32; exact on integer data
  top_k            np.argsort(-x, kind="stable") (the reference's own oracle,
                   scripts/parity_nemotronomni_seg.py:228,363,376); ties, +-inf, K = E
  softmax_selected fp64 closed form; sums to 1; equivariant under slot order
  dispatch         integer invariants (sum, exclusive scan, bijection, order)
  mul_mat_id       F32: fp64 matmul; k-quants: fp64 dot of the dequantized
                   weight and Q8_K activation rows (formats pinned in
                   test_oracle_formats.py); ne11 = 1 broadcast vs ne11 = K
  act_pair         math.erf / math.exp / math.tanh in double
  moe_forward      known answer of moe_compute.cpp:156-214 and an fp64 numpy
                   composition of the whole layer on a small random layer
"""
import math

import numpy as np
import pytest

import pyoracle as O

RNG = np.random.default_rng(7)


# ------------------------------------------------------------------ router
def test_router_logits_exact_on_integer_data():
    # integer-valued inputs: every partial sum is exact in fp64, the result is
    # an exact integer -> any reduction order gives the same bits
    E, D, T = 16, 384, 5
    W = RNG.integers(-8, 9, size=(E, D)).astype(np.float32)
    x = RNG.integers(-8, 9, size=(T, D)).astype(np.float32)
    b = RNG.integers(-4, 5, size=E).astype(np.float32)
    got = O.router_logits(W, b, x)
    ref = (x.astype(np.float64) @ W.astype(np.float64).T + b).astype(np.float32)
    assert np.array_equal(got, ref)


def test_router_logits_fp64_rounding():
    E, D, T = 64, 2048, 7
    W = (RNG.standard_normal((E, D)) * 0.02).astype(np.float32)
    x = RNG.standard_normal((T, D)).astype(np.float32)
    got = O.router_logits(W, None, x).astype(np.float64)
    ref64 = x.astype(np.float64) @ W.astype(np.float64).T
    # one fp32 rounding of an fp64 sum: within 1 ulp of the exact value
    ulp = np.spacing(np.abs(ref64).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - ref64) <= ulp)
    # a transposed operand would not be close
    assert not np.allclose(got, (x.astype(np.float64) @ W.astype(np.float64).T)[:, ::-1])


# ------------------------------------------------------------------ top-k
@pytest.mark.parametrize("E,K", [(64, 8), (128, 8), (8, 8), (5, 1)])
def test_top_k_matches_stable_argsort(E, K):
    T = 50
    logits = RNG.standard_normal((T, E)).astype(np.float32)
    logits[0, :] = 0.25                              # all equal -> ids 0..K-1
    logits[1, :] = np.round(logits[1, :] * 2) / 2    # many ties
    logits[2, 3 % E] = np.inf
    logits[2, 1 % E] = -np.inf
    got = O.top_k(logits, K)
    ref = np.argsort(-logits, axis=1, kind="stable")[:, :K].astype(np.int32)
    assert np.array_equal(got, ref)
    assert np.array_equal(got[0], np.arange(K))


# ------------------------------------------------------------------ softmax over the selected
def test_softmax_selected_closed_form_and_invariants():
    T, E, K = 40, 64, 8
    logits = (RNG.standard_normal((T, E)) * 3).astype(np.float32)
    sel = O.top_k(logits, K)
    w = O.softmax_selected(logits, sel)
    z = np.take_along_axis(logits.astype(np.float64), sel, axis=1)
    ref = np.exp(z - z.max(axis=1, keepdims=True))
    ref /= ref.sum(axis=1, keepdims=True)
    assert np.allclose(w, ref, rtol=2e-6, atol=1e-8)
    assert np.allclose(w.sum(axis=1), 1.0, atol=2e-6)
    # permuting the selected slots permutes the weights
    perm = RNG.permutation(K)
    w2 = O.softmax_selected(logits, np.ascontiguousarray(sel[:, perm]))
    assert np.allclose(w2, w[:, perm], rtol=1e-6, atol=1e-9)


# ------------------------------------------------------------------ dispatch
@pytest.mark.parametrize("T,K,E", [(1, 8, 64), (37, 8, 64), (300, 4, 16), (64, 8, 128)])
def test_dispatch_invariants(T, K, E):
    sel = np.stack([RNG.choice(E, size=K, replace=False) for _ in range(T)]).astype(np.int32)
    if T > 3:
        sel[3, :] = np.arange(K)           # a row hitting the lowest experts
    counts, offsets, perm = O.dispatch(sel, E)
    assert counts.sum() == T * K
    assert np.array_equal(counts, np.bincount(sel.ravel(), minlength=E))
    assert offsets[0] == 0 and np.array_equal(np.diff(offsets), counts)
    assert np.array_equal(np.sort(perm), np.arange(T * K))
    for e in range(E):
        lst = perm[offsets[e]:offsets[e + 1]]
        assert np.all(sel.ravel()[lst] == e)
        assert np.all(np.diff(lst) > 0)    # token-ascending (then slot)


# ------------------------------------------------------------------ mul_mat_id
def _dequant_rows(type_, raw, n_rows, kin):
    rs = O.row_size(type_, kin)
    return np.stack([O.dequantize(type_, raw[r * rs:(r + 1) * rs], kin) for r in range(n_rows)])


def test_mul_mat_id_f32_matches_fp64():
    E, N, Kin, T, nu = 6, 24, 40, 9, 3
    as_ = RNG.standard_normal((E, N, Kin)).astype(np.float32)
    b = RNG.standard_normal((T, nu, Kin)).astype(np.float32)
    ids = np.stack([RNG.choice(E, size=nu, replace=False) for _ in range(T)]).astype(np.int32)
    got = O.mul_mat_id(O.TYPE_F32, as_, Kin, N, E, b, ids)
    ref = np.stack([[as_[ids[t, k]].astype(np.float64) @ b[t, k].astype(np.float64)
                     for k in range(nu)] for t in range(T)])
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("type_", [O.TYPE_Q4_K, O.TYPE_Q6_K])
@pytest.mark.parametrize("ne11", [1, 4])
def test_mul_mat_id_kquant_matches_dequantized_fp64(type_, ne11):
    E, N, Kin, T, nu = 5, 12, 512, 6, 4
    w = (RNG.standard_normal((E * N, Kin)) * 0.02).astype(np.float32)
    raw = O.quantize(type_, w).ravel()
    b = RNG.standard_normal((T, ne11, Kin)).astype(np.float32)
    ids = np.stack([RNG.choice(E, size=nu, replace=False) for _ in range(T)]).astype(np.int32)
    got = O.mul_mat_id(type_, raw, Kin, N, E, b, ids)
    wd = _dequant_rows(type_, raw, E * N, Kin).reshape(E, N, Kin).astype(np.float64)
    ref = np.zeros((T, nu, N))
    for t in range(T):
        for k in range(nu):
            xq = O.quantize(O.TYPE_Q8_K, b[t, k % ne11][None, :])
            xd = O.dequantize(O.TYPE_Q8_K, xq.ravel(), Kin).astype(np.float64)
            ref[t, k] = wd[ids[t, k]] @ xd
    scale = np.abs(ref).max()
    assert np.max(np.abs(got - ref)) <= 1e-5 * scale


# ------------------------------------------------------------------ activation
def test_act_pair_closed_forms():
    for a in [-6.0, -2.5, -0.3, 0.0, 0.7, 3.1]:
        for b in [-1.5, 0.0, 2.0]:
            silu = a / (1 + math.exp(-a)) * b
            gelu = 0.5 * a * (1 + math.erf(a / math.sqrt(2)))
            tanh = 0.5 * a * (1 + math.tanh(math.sqrt(2 / math.pi) * a * (1 + 0.044715 * a * a)))
            for act, ref in [(0, silu), (1, gelu * (b + 1)), (2, tanh * b), (3, gelu * b)]:
                got = O.act_pair(act, np.float32(a), np.float32(b))
                assert abs(got - ref) <= 2e-6 * max(1.0, abs(ref)), (act, a, b, got, ref)


# ------------------------------------------------------------------ whole layer
def test_known_answer_f32_silu():
    """moe_compute.cpp:156-214: D=2, I=3, K=2, F32 SiLU, table form."""
    gate = np.array([[[0, 1], [1, 0], [0, 0]], [[1, 0], [0, 1], [0, 0]]], np.float32)   # [E][I][D]
    up = np.array([[[1, 0], [0, 1], [1, 1]], [[0, 1], [1, 0], [0, 0]]], np.float32)
    down = np.array([[[1, 0, 0], [0, 1, 0]], [[0, 1, 0], [1, 0, 0]]], np.float32)        # [E][D][I]
    layer = dict(E=2, K=2, I=3, router_w=None, router_b=None, gate_type=O.TYPE_F32, gate=gate,
                 up=up, fused=False, down_type=O.TYPE_F32, down=down, act=0)
    x = np.array([[1.0, 2.0]], np.float32)
    out, _ = O.moe_forward(layer, x, res=x, sel_in=np.array([[0, 1]], np.int32),
                           w_in=np.array([[0.5, 1.0]], np.float32))
    assert np.allclose(out[0], [3.6423913, 4.1931758], atol=1e-6)


def test_layer_matches_fp64_composition():
    D, E, K, I, T = 512, 8, 3, 256, 11
    q4, q6 = O.TYPE_Q4_K, O.TYPE_Q6_K
    rw = (RNG.standard_normal((E, D)) * 0.05).astype(np.float32)
    rb = (RNG.standard_normal(E) * 0.1).astype(np.float32)
    gu = O.quantize(q4, (RNG.standard_normal((E * 2 * I, D)) * 0.02).astype(np.float32)).ravel()
    dn = O.quantize(q6, (RNG.standard_normal((E * D, I)) * 0.02).astype(np.float32)).ravel()
    x = RNG.standard_normal((T, D)).astype(np.float32)
    layer = dict(E=E, K=K, I=I, router_w=rw, router_b=rb, gate_type=q4, gate=gu, up=None,
                 fused=True, down_type=q6, down=dn, act=1)
    out, dbg = O.moe_forward(layer, x)
    # fp64 composition: same routing decisions, every product in fp64 on
    # dequantized operands, activations quantized to Q8_K like ggml-cpu
    sel = dbg["sel"]
    logits = x.astype(np.float64) @ rw.astype(np.float64).T + rb
    assert np.array_equal(sel, np.argsort(-logits.astype(np.float32), axis=1, kind="stable")[:, :K])
    z = np.take_along_axis(logits, sel, axis=1)
    w = np.exp(z - z.max(1, keepdims=True))
    w /= w.sum(1, keepdims=True)
    Wg = _dequant_rows(q4, gu, E * 2 * I, D).reshape(E, 2 * I, D).astype(np.float64)
    Wd = _dequant_rows(q6, dn, E * D, I).reshape(E, D, I).astype(np.float64)
    ref = np.zeros((T, D))
    for t in range(T):
        xq = O.dequantize(O.TYPE_Q8_K, O.quantize(O.TYPE_Q8_K, x[t][None, :]).ravel(), D)
        for k in range(K):
            hg = Wg[sel[t, k]] @ xq.astype(np.float64)
            h, g = hg[:I], hg[I:]
            a = 0.5 * h * (1 + np.vectorize(math.erf)(h / math.sqrt(2))) * (g + 1)
            aq = O.dequantize(O.TYPE_Q8_K, O.quantize(O.TYPE_Q8_K, a.astype(np.float32)[None, :]).ravel(), I)
            ref[t] += w[t, k] * (Wd[sel[t, k]] @ aq.astype(np.float64))
    rel = np.linalg.norm(out - ref) / np.linalg.norm(ref)
    # measured 1.9e-7 (fp32 vs fp64 summation); one Q8_K rounding flip of an
    # activation would already cost ~1e-4, a wrong term far more
    assert rel < 1e-5, rel


# ------------------------------------------------------------------ gating variants
def test_route_gated_hand_case():
    """nemotronomni gating (sigmoid, selection bias, renorm x scaling) and the
    per-expert scale on a case worked by hand."""
    l = np.array([[0.0, 1.0, -1.0, 2.0]], np.float32)
    sel, w = O.route_gated(l, 2, 1, sel_bias=np.array([0, 0, 5, 0], np.float32), scaling=2.5)
    assert sel.tolist() == [[2, 3]]   # sig(-1) + 5 first, then sig(2) = 0.881 over sig(1) = 0.731
    s = 1 / (1 + np.exp(-np.array([-1.0, 2.0])))
    assert np.allclose(w[0], s / s.sum() * 2.5, rtol=1e-6)
    sel, w = O.route_gated(l, 2, 0, expert_scale=np.array([1, 2, 3, 4], np.float32))
    assert sel.tolist() == [[3, 1]]
    p = np.exp([2.0, 1.0]) / np.exp([2.0, 1.0]).sum()
    assert np.allclose(w[0], p * [4, 2], rtol=1e-6)


def test_route_gated_properties():
    rng = np.random.default_rng(3)
    T, E, K = 200, 64, 8
    l = (rng.standard_normal((T, E)) * 2).astype(np.float32)
    b = (rng.standard_normal(E) * 0.5).astype(np.float32)
    sc = (1 + rng.random(E)).astype(np.float32)
    # kind 1: the ranking is that of fp64 sigmoid + bias (distinct values here)
    sel, w = O.route_gated(l, K, 1, sel_bias=b, scaling=2.5, eps=0.0)
    score = (1 / (1 + np.exp(-l.astype(np.float64)))).astype(np.float32) + b
    ref = np.argsort(-score.astype(np.float64), axis=1, kind="stable")[:, :K]
    assert np.array_equal(sel, ref)
    assert np.allclose(w.astype(np.float64).sum(axis=1), 2.5, rtol=2e-6)
    # kind 1 without a bias selects the top-k logits (sigmoid is monotonic)
    sel0, _ = O.route_gated(l, K, 1)
    assert np.array_equal(sel0, O.top_k(l, K))
    # eps enters the denominator once
    _, we = O.route_gated(l, K, 1, sel_bias=b, scaling=1.0, eps=0.5)
    s_sel = (1 / (1 + np.exp(-np.take_along_axis(l, sel, 1).astype(np.float64))))
    assert np.allclose(we, s_sel / (s_sel.sum(axis=1, keepdims=True) + 0.5), rtol=2e-6)
    # kind 0 with a per-expert scale: the default weights times scale[sel], exactly
    s0, w0 = O.route_gated(l, K, 0, expert_scale=sc)
    assert np.array_equal(s0, O.top_k(l, K))
    wd = O.softmax_selected(l, s0)
    assert np.array_equal(w0, (wd * sc[s0]).astype(np.float32))
