"""HIP graph capture of the forward.  The C ABI takes a stream, so a serving
loop may capture mi_moe_forward once and replay it: every replay must give the
eager forward's bits.  Covered: the prefill path (router + Q8_K of x, top-k,
dispatch, grouped MFMA GEMMs, Q8_K of the GLU rows, combine), the small-batch
GEMV chain, and the single-token fused kernel in its plain-launch mode (its
epoch-tagged logits and monotonic barrier counters carry over between
replays).  Each replay reads a new input written into the captured buffer,
with eager forwards and synchronizations between replays, so graph nodes that
replay stale state or depend on the first replay's memory show up as a
mismatch on a later replay.  Capture and replay go through the library's own
mi_stream_begin_capture / mi_stream_end_capture / mi_graph_launch.
"""
import sys

import numpy as np
import pytest

import mimoe as M
import pyoracle as O
import workloads as W
from _util import small_spec

pytestmark = pytest.mark.gpu

REPLAYS = 4


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _x(spec, T, r):
    return (np.random.default_rng(1000 * T + r).standard_normal((T, spec.D))).astype(np.float32)


def _graph_vs_eager(ctx, layer, spec, T, res=True):
    D = spec.D
    xd = M.DeviceBuffer(4 * T * D).upload(_x(spec, T, 0))
    rd = M.DeviceBuffer(4 * T * D).upload(_x(spec, T, 99)) if res else None
    out_g, out_e = M.DeviceBuffer(4 * T * D), M.DeviceBuffer(4 * T * D)
    M.check("warm forward", ctx.forward(layer, xd, T, rd, out_e))
    M.synchronize()
    s = M.Stream()
    g = M.Graph(s, lambda st: M.check("forward under capture", ctx.forward(layer, xd, T, rd, out_g, stream=st.h)))
    for r in range(1, REPLAYS + 1):
        xd.upload(_x(spec, T, r))
        g.launch(s)
        s.synchronize()
        got = out_g.download(np.float32, (T, D))
        M.check("eager forward", ctx.forward(layer, xd, T, rd, out_e))
        M.synchronize()
        ref = out_e.download(np.float32, (T, D))
        assert np.isfinite(ref).all()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"replay {r}"
    g.destroy()
    s.destroy()


@pytest.mark.parametrize("T", [1, 4, 300])
def test_graph_small_layer(T):
    """Small moondream-shape layer: T = 300 on the GEMM path, T = 4 on the
    GEMV chain (4 T K < 5 E), T = 1 on the chain (the layer is outside the fused kernel's
    shapes or the fused kernel, whichever the planner picks)."""
    spec = small_spec("md_graph", D=512, E=8, K=2, I=256, fused=True, down_type=O.TYPE_Q6_K,
                      act=O.ACT_GELU_TANH, seed=0x5EED3000)
    ctx = M.Context(0)
    ctx.reserve(300, spec.D, spec.I, spec.E, spec.K)
    g = W.GpuLayer(ctx, spec)
    _graph_vs_eager(ctx, g.layer, spec, T)
    log(f"graph md_graph T={T}: {REPLAYS} replays bit-identical to eager")
    ctx.close()


@pytest.mark.parametrize("T", [1, 1024])
def test_graph_config_layer(T):
    """The config-1 layer: 1024-token prefill and the single-token fused
    kernel in plain-launch mode."""
    spec = W.CONFIGS[1]["spec"]
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    ctx.set_fused_decode(M.DECODE_FUSED)
    g = W.GpuLayer(ctx, spec)
    _graph_vs_eager(ctx, g.layer, spec, T, res=False)
    log(f"graph md_cfg1 T={T}: {REPLAYS} replays bit-identical to eager")
    ctx.close()
