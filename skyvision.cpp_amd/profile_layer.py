"""Runs one BASELINE layer configuration at a chosen token count, for a
profiler to trace: the layer (16 rotated synthetic copies, seeded like the
bench) forwarded `--iters` times, captured once into a HIP graph and
replayed (or issued call by call with --no-graph), on the default product
paths (the kernel chain with --chain; the tables' tiled copies with --tiled).  Prints the time per call.

    rocprofv3 --kernel-trace --stats -- python3 skyvision.cpp_amd/profile_layer.py --config 3 --tokens 32
"""
import argparse
import os
import sys
import time

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import mimoe as M  # noqa: E402
import workloads as W  # noqa: E402


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", type=int, default=3, choices=[0, 1, 2, 3])
    ap.add_argument("--tokens", type=int, default=32)
    ap.add_argument("--iters", type=int, default=64)
    ap.add_argument("--copies", type=int, default=16)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--chain", action="store_true", help="the kernel chain also where a fused decode kernel applies")
    ap.add_argument("--tiled", action="store_true", help="tiled copies of the Q4_K tables for the grouped GEMMs")
    ap.add_argument("--gemm-tiles", type=int, default=0, choices=[0, 1, 2, 3, 4, 5],
                    help="GEMM row tiles (mi_moe_ctx_set_gemm_tiles): 0 by shape, 1 192 rows, 2 32 rows, "
                         "3 the skinny products, 4 8 rows, 5 64 rows")
    ap.add_argument("--stages", action="store_true", help="also the per-stage averages of 32 profiled calls")
    a = ap.parse_args()
    spec = W.CONFIGS[a.config]["spec"]
    T = a.tokens
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    if a.chain:
        ctx.set_fused_decode(M.DECODE_CHAIN)
    if a.gemm_tiles:
        ctx.set_gemm_tiles(a.gemm_tiles)
    layers = [W.GpuLayer(ctx, spec, copy=c) for c in range(a.copies)]
    if a.tiled:
        for g in layers:
            g.add_tiled(ctx)
    xs = [W.gen_x(ctx, spec, T, copy=c) for c in range(a.copies)]
    out = M.DeviceBuffer(4 * T * spec.D)
    n = len(layers)
    M.synchronize()
    if a.no_graph:
        t0 = time.perf_counter()
        for i in range(a.iters):
            M.check("forward", ctx.forward(layers[i % n].layer, xs[i % n], T, None, out))
        M.synchronize()
        us = (time.perf_counter() - t0) / a.iters * 1e6
        print(f"config {a.config} T={T}: {us:.1f} us per call (issued call by call, host clock)", flush=True)
    else:
        s = M.Stream()

        def record(st):
            for i in range(a.iters):
                M.check("forward (capture)", ctx.forward(layers[i % n].layer, xs[i % n], T, None, out, stream=st.h))

        g = M.Graph(s, record)
        g.launch(s)
        s.synchronize()
        e0, e1 = M.Event(), M.Event()
        e0.record(s.h)
        g.launch(s)
        e1.record(s.h)
        e1.synchronize()
        print(f"config {a.config} T={T}: {e0.elapsed_ms(e1) / a.iters * 1e3:.1f} us per call (graph replay)",
              flush=True)
        g.destroy()
        s.destroy()
    if a.stages:
        ctx.set_profiling(True)
        acc = {}
        for i in range(32):
            M.check("forward", ctx.forward(layers[i % n].layer, xs[i % n], T, None, out))
            for k, v in ctx.stage_times():
                acc[k] = acc.get(k, 0.0) + v / 32
        ctx.set_profiling(False)
        print(f"config {a.config} T={T} stages (us): " + ", ".join(f"{k} {1e3 * v:.1f}" for k, v in acc.items()),
              flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
