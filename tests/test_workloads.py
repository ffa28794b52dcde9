"""The synthetic workloads are what BASELINE.json describes: config 2's
router bias sends about 40 % of the 8192 assignments to the 4 hottest
experts and none to 16 experts; config 1's load is near uniform (every
expert between about 64 and 200 rows).  Computed on the CPU with the
oracle's bit-exact RNG and router."""
import numpy as np

import pyoracle as O
import workloads as W


def routing_counts(cfg):
    spec = W.CONFIGS[cfg]["spec"]
    T = W.CONFIGS[cfg]["tokens"][0]
    rw = O.fill_normal(spec.E * spec.D, spec.seed, W.S_ROUTER_W, 0.0, spec.router_std).reshape(spec.E, spec.D)
    x = O.fill_normal(T * spec.D, spec.seed, W.S_X, 0.0, 1.0).reshape(T, spec.D)
    b = W.zipf_bias(spec.E, spec.seed) if spec.router_bias == "zipf" else None
    sel = O.top_k(O.router_logits(rw, b, x), spec.K)
    return np.bincount(sel.ravel(), minlength=spec.E), T * spec.K


def test_config2_skew():
    c, n = routing_counts(2)
    top4 = np.sort(c)[::-1][:4].sum() / n
    assert 0.37 <= top4 <= 0.43, top4
    assert (c == 0).sum() == 16


def test_config1_near_uniform():
    c, n = routing_counts(1)
    assert c.sum() == n and c.min() >= 64 and c.max() <= 200, (c.min(), c.max())
