"""Pins the oracle's layer variants independently of the GPU:

  route_gated kind 2   diffusiongemma's softmax over all E -> top-k on the
                       probabilities -> renorm over the K
                       (diffusiongemma_model.cpp:923-932): a sequential fp64
                       restatement in numpy, a hand case, and a case where
                       probabilities underflow to equal zeros so the ranking of
                       the probabilities differs from the ranking of the logits
  act RELU_SQR         relu(u)^2 closed form (nemotronomni_model.cpp:366-367)
  moe_forward          fp64 numpy compositions of: separate down ids
                       (moe_compute.hpp:45, the down_ids of the table form);
                       non-gated relu^2 experts; a shared expert, unscaled
                       (nemotronomni_model.cpp:371-376) and sigmoid-gated
                       (qwen3omni_talker.cpp:396-402); the gating kinds
"""
import math

import numpy as np
import pytest

import pyoracle as O

RNG = np.random.default_rng(11)


def _dequant_rows(type_, raw, n_rows, kin):
    if type_ == O.TYPE_F32:
        return np.asarray(raw, np.float32).reshape(n_rows, kin)
    rs = O.row_size(type_, kin)
    raw = np.asarray(raw).ravel()
    return np.stack([O.dequantize(type_, raw[r * rs:(r + 1) * rs], kin) for r in range(n_rows)])


def _softmax_all_ref(l: np.ndarray, K: int, scale=None):
    """kind 2 restated with Python loops: max, e = fl32(exp(fl32(l - max))),
    sequential fp64 sum, p = e * fl32(1 / sum); stable descending argsort of p;
    w = p_sel / fl32(sequential fp64 sum of p_sel) [* scale]."""
    T, E = l.shape
    sel = np.zeros((T, K), np.int32)
    w = np.zeros((T, K), np.float32)
    for t in range(T):
        mx = np.float32(l[t].max())
        e = np.array([np.float32(math.exp(float(np.float32(l[t, i] - mx)))) for i in range(E)], np.float32)
        s = 0.0
        for i in range(E):
            s += float(e[i])
        p = (e * np.float32(1.0 / s)).astype(np.float32)
        sel[t] = np.argsort(-p.astype(np.float64), kind="stable")[:K]
        ps = 0.0
        for k in range(K):
            ps += float(p[sel[t, k]])
        w[t] = p[sel[t]] / np.float32(ps)
        if scale is not None:
            w[t] = w[t] * scale[sel[t]]
    return sel, w


def test_softmax_all_matches_restatement():
    T, E, K = 64, 128, 8
    l = (RNG.standard_normal((T, E)) * 3).astype(np.float32)
    sc = (0.5 + RNG.random(E)).astype(np.float32)
    sel, w = O.route_gated(l, K, O.GATING_SOFTMAX_ALL, expert_scale=sc)
    rs, rw = _softmax_all_ref(l, K, sc)
    assert np.array_equal(sel, rs)
    assert np.array_equal(w, rw)
    # with distinct probabilities the ids are those of the logits (softmax is monotonic)
    assert np.array_equal(O.route_gated(l, K, O.GATING_SOFTMAX_ALL)[0], O.top_k(l, K))


def test_softmax_all_hand_case_and_underflow_ties():
    # hand case: p ~ softmax([0, 1, 2, -1]); top-2 = {2, 1}; renormalized over the two
    l = np.array([[0.0, 1.0, 2.0, -1.0]], np.float32)
    sel, w = O.route_gated(l, 2, O.GATING_SOFTMAX_ALL)
    assert sel.tolist() == [[2, 1]]
    assert np.allclose(w[0], [math.e / (math.e + 1), 1 / (math.e + 1)], rtol=1e-6)
    # logits far below the maximum underflow to probability 0: ties at 0 rank
    # the lower id first, while the logits themselves are distinct and rank
    # the larger logit first (a restatement ranking logits would fail here)
    l = np.array([[0.0, -300.0, -200.0, -250.0, 1.0]], np.float32)
    sel, w = O.route_gated(l, 4, O.GATING_SOFTMAX_ALL)
    assert sel.tolist() == [[4, 0, 1, 2]]
    assert O.top_k(l, 4).tolist() == [[4, 0, 2, 3]]
    assert w[0, 2] == 0.0 and w[0, 3] == 0.0
    assert abs(float(w[0, :2].sum()) - 1.0) < 1e-6


def test_act_relu_sqr():
    for a in [-3.0, -1e-30, 0.0, 1e-3, 0.5, 7.25]:
        got = O.act_pair(O.ACT_RELU_SQR, np.float32(a), np.float32(123.0))
        assert got == np.float32(max(a, 0.0)) * np.float32(max(a, 0.0))


def _q8_round_trip(v: np.ndarray) -> np.ndarray:
    n = v.shape[-1]
    return O.dequantize(O.TYPE_Q8_K, O.quantize(O.TYPE_Q8_K, v.astype(np.float32)[None, :]).ravel(), n)


def _act64(act, a, b):
    if act == O.ACT_RELU_SQR:
        return np.where(a > 0, a * a, 0.0)
    if act == 0:
        return a / (1 + np.exp(-a)) * b
    if act == 1:
        return 0.5 * a * (1 + np.vectorize(math.erf)(a / math.sqrt(2))) * (b + 1)
    if act == 2:
        return 0.5 * a * (1 + np.tanh(math.sqrt(2 / math.pi) * a * (1 + 0.044715 * a * a))) * b
    return 0.5 * a * (1 + np.vectorize(math.erf)(a / math.sqrt(2))) * b


def _expert64(Wg, Wu, Wd, act, x64):
    """one expert on one token, fp64 products on dequantized weights with the
    Q8_K activations of ggml-cpu (both products)"""
    xq = _q8_round_trip(x64.astype(np.float32)).astype(np.float64)
    g = Wg @ xq
    u = Wu @ xq if Wu is not None else None
    a = _act64(act, g, u)
    aq = _q8_round_trip(a.astype(np.float32)).astype(np.float64)
    return Wd @ aq


def _make_layer(D, E, K, I, act, gating=0, sh_I=0, sh_act=0, sh_gate=False, qt=O.TYPE_Q4_K, dt=O.TYPE_Q6_K):
    gated = act != O.ACT_RELU_SQR
    L = dict(D=D, E=E, K=K, I=I, router_w=(RNG.standard_normal((E, D)) * 0.05).astype(np.float32),
             router_b=None, gate_type=qt, down_type=dt, fused=False, act=act, gating=gating)
    f = lambda rows, k: (RNG.standard_normal((rows, k)) * 0.02).astype(np.float32)  # noqa: E731
    L["gate_f"] = f(E * I, D)
    L["gate"] = O.quantize(qt, L["gate_f"]).ravel()
    L["up"] = O.quantize(qt, f(E * I, D)).ravel() if gated else None
    L["down"] = O.quantize(dt, f(E * D, I)).ravel()
    if gating == O.GATING_SIGMOID_BIAS:
        L.update(sel_bias=(RNG.standard_normal(E) * 0.1).astype(np.float32), routed_scaling=2.5, gate_eps=1e-3)
    if gating == O.GATING_SOFTMAX_ALL:
        L["expert_scale"] = (0.5 + RNG.random(E)).astype(np.float32)
    if sh_I:
        act_gated = sh_act != O.ACT_RELU_SQR
        L.update(sh_I=sh_I, sh_act=sh_act, sh_type=qt, sh_down_type=dt,
                 sh_gate=O.quantize(qt, f(sh_I, D)).ravel(),
                 sh_up=O.quantize(qt, f(sh_I, D)).ravel() if act_gated else None,
                 sh_down=O.quantize(dt, f(D, sh_I)).ravel(),
                 sh_gate_inp=(RNG.standard_normal(D) * 0.05).astype(np.float32) if sh_gate else None)
    return L


def _compose(L, x, sel, dsel, w):
    D, E, I = L["D"], L["E"], L["I"]
    qt, dt = L["gate_type"], L["down_type"]
    Wg = _dequant_rows(qt, L["gate"], E * I, D).reshape(E, I, D).astype(np.float64)
    Wu = _dequant_rows(qt, L["up"], E * I, D).reshape(E, I, D).astype(np.float64) if L["up"] is not None else None
    Wd = _dequant_rows(dt, L["down"], E * D, I).reshape(E, D, I).astype(np.float64)
    T, K = sel.shape
    ref = np.zeros((T, D))
    for t in range(T):
        xq = _q8_round_trip(x[t]).astype(np.float64)
        for k in range(K):
            g = Wg[sel[t, k]] @ xq
            u = Wu[sel[t, k]] @ xq if Wu is not None else None
            a = _act64(L["act"], g, u)
            aq = _q8_round_trip(a.astype(np.float32)).astype(np.float64)
            ref[t] += float(w[t, k]) * (Wd[dsel[t, k]] @ aq)
    if L.get("sh_I"):
        sI = L["sh_I"]
        Sg = _dequant_rows(qt, L["sh_gate"], sI, D).astype(np.float64)
        Su = _dequant_rows(qt, L["sh_up"], sI, D).astype(np.float64) if L["sh_up"] is not None else None
        Sd = _dequant_rows(dt, L["sh_down"], D, sI).astype(np.float64)
        for t in range(T):
            s = _expert64(Sg, Su, Sd, L["sh_act"], x[t].astype(np.float64))
            if L.get("sh_gate_inp") is not None:
                s = s / (1 + math.exp(-float(L["sh_gate_inp"].astype(np.float64) @ x[t].astype(np.float64))))
            ref[t] += s
    return ref


@pytest.mark.parametrize("case", ["down_ids", "relu_sqr", "shared_relu_sqr", "shared_silu_gated",
                                  "sigmoid_gating", "softmax_all_gating"])
def test_layer_variants_match_fp64_composition(case):
    D, E, K, I, T = 512, 8, 3, 256, 7
    x = RNG.standard_normal((T, D)).astype(np.float32)
    kw = {}
    if case == "relu_sqr":
        L = _make_layer(D, E, K, I, O.ACT_RELU_SQR)
    elif case == "shared_relu_sqr":
        L = _make_layer(D, E, K, I, O.ACT_RELU_SQR, sh_I=512, sh_act=O.ACT_RELU_SQR)
    elif case == "shared_silu_gated":
        L = _make_layer(D, E, K, I, 0, sh_I=256, sh_act=0, sh_gate=True)
    elif case == "sigmoid_gating":
        L = _make_layer(D, E, K, I, 2, gating=O.GATING_SIGMOID_BIAS)
    elif case == "softmax_all_gating":
        L = _make_layer(D, E, K, I, 2, gating=O.GATING_SOFTMAX_ALL)
    else:
        L = _make_layer(D, E, K, I, 0)
        sel = np.stack([RNG.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
        dsel = np.stack([RNG.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
        w = RNG.random((T, K)).astype(np.float32)
        kw = dict(sel_in=sel, down_sel_in=dsel, w_in=w)
    res = RNG.standard_normal((T, D)).astype(np.float32)
    out, dbg = O.moe_forward(L, x, res, **kw)
    if case == "down_ids":
        sel, dsel, w = kw["sel_in"], kw["down_sel_in"], kw["w_in"]
        # the same call with the gate/up ids for the down product differs: the
        # ids really reach the down product
        out_same, _ = O.moe_forward(L, x, res, sel_in=sel, w_in=w)
        assert np.linalg.norm(out_same - out) > 0.1 * np.linalg.norm(out - res)
    else:
        sel, w = dbg["sel"], dbg["w"]
        dsel = sel
        ref_sel, ref_w = O.route_gated(dbg["logits"], K, L["gating"], sel_bias=L.get("sel_bias"),
                                       expert_scale=L.get("expert_scale"),
                                       scaling=L.get("routed_scaling", 1.0) or 1.0, eps=L.get("gate_eps", 0.0))
        assert np.array_equal(sel, ref_sel) and np.array_equal(w, ref_w)
    ref = _compose(L, x, sel, dsel, w)
    got = out.astype(np.float64) - res
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    # fp32 vs fp64 summation only (~1e-7); a Q8_K rounding flip costs ~1e-4,
    # a dropped or mis-indexed term far more
    assert rel < 1e-5, (case, rel)
    if L.get("sh_I"):
        # the shared part alone is the composition's shared part
        sh = dbg["sh"].astype(np.float64)
        L0 = dict(L, sh_I=0)
        ref0 = _compose(L0, x, sel, dsel, w)
        assert np.linalg.norm(sh - (ref - ref0)) / np.linalg.norm(ref - ref0) < 1e-5
