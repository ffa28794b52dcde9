"""bench.py - MoE layer throughput on one MI355X (BASELINE.json metric).

Default workload: config 1, the moondream3-shape MoE layer on a 1024-token
prefill (gate/up Q4_K, down Q6_K, E=64, top-8), seeded synthetic data.  One
step = one full layer forward (router -> top-k -> dispatch -> gate/up GEMM +
GeGLU -> Q8_K -> down GEMM -> weighted combine) over the 1024 tokens, with
the inputs resident in HBM.  Steps rotate over --copies distinct layer copies
so the 256 MB Infinity Cache cannot hold the weights between steps.  Each
layer carries tiled copies of its tables (mi_moe_tile: Q4_K reordered, Q6_K
down with merged codes; made when the layer is built, outside the timed
region), which the grouped GEMMs read in place of the GGUF rows
(bit-identical output); --no-tiled runs on the GGUF rows alone.

Printed JSON line (rank 0):
  value          tokens/s of the whole layer (T * steps / time); the K forwards
                 are captured once into a HIP graph and replayed (every kernel
                 of every step runs; --no-graph times stream-issued forwards,
                 whose rate is also in the line)
  roofline       the dominant kernel (gate/up grouped GEMM): algorithmic flops
                 per launch / its average duration (HIP events on its stream)
                 vs the 2.5 PFLOP/s dense fp16/bf16 MFMA peak
  decode         config 0 (1 token) on the same box: tokens/s and the HBM
                 roofline of its dominant kernel (selected experts' bytes /
                 duration vs 8 TB/s)
  cpu_baseline   the CPU oracle (ggml-semantics restatement, C, OpenMP) on a
                 bounded sample of the same workload, physical cores
  config3        qwen3omni layer, batched decode at 1 / 8 / 32 / 64 tokens on
                 the GEMV and GEMM paths (and the fused single-token kernel):
                 times, HBM rates, the GEMV-to-GEMM crossover
  config4        24-layer stack h + MoE(RMSNorm(h)): 2048-token prefill and
                 256 decode steps, sustained tokens/s, TFLOP/s and GB/s
(--no-decode, --no-sweeps and --no-cpu skip the extra legs.)
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "skyvision.cpp_amd"))

import numpy as np  # noqa: E402

import mimoe as M  # noqa: E402
import workloads as W  # noqa: E402

PEAK_MFMA_TFLOPS = 2500.0      # MI355X dense fp16 / bf16 MFMA (published, 2.4 GHz)
CUS, FLOPS_PER_CU_CYCLE = 256, 4096
ACT_NAMES = {0: "silu(gate)*up", 1: "gelu_erf(h)*(g+1)", 2: "gelu_tanh(gate)*up", 3: "gelu_erf(gate)*up"}
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def time_layer(ctx, layers, xs, T, out, steps, warmup, profile=False):
    """Run `steps` forwards rotating over layer copies; returns (ms/step,
    {"wall_ms_per_step"}), or with profile=True (the shader clock in GHz under
    each grouped GEMM, per-stage mean ms)."""
    n = len(layers)
    for i in range(warmup):
        M.check("forward", ctx.forward(layers[i % n].layer, xs[i % n], T, None, out))
    M.synchronize()
    if profile:
        ctx.set_profiling(True)
        acc, clk = {}, {}
        for i in range(steps):
            M.check("forward", ctx.forward(layers[i % n].layer, xs[i % n], T, None, out))
            for name, ms in ctx.stage_times():
                acc.setdefault(name, []).append(ms)
            for name in ("gate_up", "down"):
                r = ctx.stage_clock(name)
                if r is not None:
                    clk.setdefault(name, []).append(r[0])
        ctx.set_profiling(False)
        M.synchronize()
        return ({k: float(np.mean(v)) for k, v in clk.items()},
                {k: float(np.mean(v)) for k, v in acc.items()})
    e0, e1 = M.Event(), M.Event()
    M.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for i in range(steps):
        M.check("forward", ctx.forward(layers[i % n].layer, xs[i % n], T, None, out))
    e1.record()
    e1.synchronize()
    M.synchronize()
    wall = (time.perf_counter() - t0) * 1e3
    dev = e0.elapsed_ms(e1)
    return max(dev, 0.0) / steps, {"wall_ms_per_step": wall / steps}


def time_layer_graph(ctx, layers, xs, T, out, steps):
    """The same `steps` forwards (same copy rotation) captured once into a HIP
    graph (mi_stream_begin_capture / mi_stream_end_capture) and replayed:
    every kernel of every step runs, the host launch gaps between them leave
    the timed region.  One untimed replay, then one timed replay between
    events on the replay stream and device synchronizations.  Returns (ms/step,
    wall ms/step)."""
    n = len(layers)
    M.synchronize()
    s = M.Stream()

    def record(st):
        for i in range(steps):
            M.check("forward (capture)", ctx.forward(layers[i % n].layer, xs[i % n], T, None, out, stream=st.h))

    g = M.Graph(s, record)
    g.launch(s)
    s.synchronize()
    e0, e1 = M.Event(), M.Event()
    M.synchronize()
    t0 = time.perf_counter()
    e0.record(s.h)
    g.launch(s)
    e1.record(s.h)
    e1.synchronize()
    M.synchronize()
    wall = (time.perf_counter() - t0) * 1e3
    ms = e0.elapsed_ms(e1) / steps
    g.destroy()
    s.destroy()
    return ms, wall / steps


def profile_key(kernel: str, config: int) -> str:
    """key of a kernel's entry in the committed counter summaries: the kernel
    name for config 1 (and the decode kernels), name@configN for another
    prefill config"""
    return kernel if config == 1 else f"{kernel}@config{config}"


def measured_traffic(kernel: str, config: int = 1):
    """HBM bytes per launch of `kernel` under `config` from the committed
    counter summary (profiles/traffic.json: FETCH_SIZE + WRITE_SIZE per
    dispatch, scaled by the same counters on a copy of known size); None when
    that config was not measured."""
    p = ROOT / "profiles" / "traffic.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get(profile_key(kernel, config), {}).get("bytes_per_launch")
    except (ValueError, AttributeError):
        return None


def touched_experts(ctx, layer, x, T):
    counts = M.DeviceBuffer(4 * layer.spec.E)
    r = M.Routing()
    r.counts = counts.addr
    out = M.DeviceBuffer(4 * T * layer.spec.D)
    M.check("forward", ctx.forward(layer.layer, x, T, None, out, r))
    M.synchronize()
    c = counts.download(np.int32, (layer.spec.E,))
    return int((c > 0).sum()), c


def gpu_reference(ctx, layer, x, T) -> dict:
    """One forward of `layer` on the device rows x with every routing output:
    the GPU side of the bench line's parity columns."""
    spec = layer.spec
    bufs = dict(sel=M.DeviceBuffer(4 * T * spec.K), counts=M.DeviceBuffer(4 * spec.E),
                offsets=M.DeviceBuffer(4 * (spec.E + 1)), perm=M.DeviceBuffer(4 * T * spec.K),
                logits=M.DeviceBuffer(4 * T * spec.E))
    r = M.Routing()
    for k, v in bufs.items():
        setattr(r, k, C.c_void_p(v.addr))
    out = M.DeviceBuffer(4 * T * spec.D)
    M.check("forward", ctx.forward(layer.layer, x, T, None, out, r))
    M.synchronize()
    shapes = dict(sel=(T, spec.K), counts=(spec.E,), offsets=(spec.E + 1,), perm=(T * spec.K,), logits=(T, spec.E))
    got = {k: bufs[k].download(np.float32 if k == "logits" else np.int32, shapes[k]) for k in bufs}
    got["out"] = out.download(np.float32, (T, spec.D))
    got["x"] = x.download(np.float32, (T, spec.D))
    return got


def parity_columns(gpu: dict, ref: np.ndarray, dbg: dict) -> dict:
    """The parity columns of the benchmark: routing bit-exactness and the
    output's rel-L2 / max-abs against the CPU oracle on the same tokens."""
    exact = {k: bool(np.array_equal(gpu[k], dbg[k])) for k in ("sel", "counts", "offsets", "perm")}
    exact["logits"] = bool(np.array_equal(gpu["logits"].view(np.uint32), dbg["logits"].view(np.uint32)))
    d = (gpu["out"].astype(np.float64) - ref.astype(np.float64)).ravel()
    return {"routing_bit_exact": all(exact.values()), "routing": exact,
            "rel_l2": float(np.linalg.norm(d) / np.linalg.norm(ref.astype(np.float64).ravel())),
            "max_abs": float(np.abs(d).max()), "tolerance_rel_l2": 1e-2,
            "tokens": int(ref.shape[0])}


def cpu_baseline(spec, layer0: W.GpuLayer, T_sample: int, gpu_ref: dict | None = None, budget_s: float = 20.0):
    """CPU oracle (ggml-semantics restatement) on T_sample tokens of the same
    layer; weights copied from the GPU tables (bit-identical to the oracle's
    own quantizer output).  Its output on the layer's 1024 bench tokens also
    gives the parity columns against the GPU forward of the same tokens."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import pyoracle as O
    cores = O.physical_cores()
    tables = layer0.download_tables()
    rw = layer0.download_router()
    L = dict(D=spec.D, E=spec.E, K=spec.K, I=spec.I, router_w=rw, router_b=layer0.bias_host,
             gate_type=spec.gate_type, down_type=spec.down_type, fused=spec.fused, act=spec.act,
             gate=tables["gate"], down=tables["down"])
    if "up" in tables:
        L["up"] = tables["up"]
    x = O.fill_normal(T_sample * spec.D, spec.seed, W.S_X, 0.0, 1.0, cores).reshape(T_sample, spec.D)
    parity = None
    if gpu_ref is not None:
        ref, dbg = O.moe_forward(L, gpu_ref["x"], nthreads=cores)        # also the warm-up
        parity = parity_columns(gpu_ref, ref, dbg)
        log(f"parity vs the CPU oracle on {ref.shape[0]} tokens: routing bit-exact {parity['routing_bit_exact']}, "
            f"rel-L2 {parity['rel_l2']:.3e}, max-abs {parity['max_abs']:.3e}")
    else:
        O.moe_forward(L, x, nthreads=cores, debug=False)          # warm

    def timed(simd: bool):
        O.set_simd(simd)
        out, _ = O.moe_forward(L, x, nthreads=cores, debug=False)   # warm this form
        times = []
        t_start = time.perf_counter()
        while len(times) < 10 and (time.perf_counter() - t_start) < budget_s / 2:
            t0 = time.perf_counter()
            O.moe_forward(L, x, nthreads=cores, debug=False)
            times.append(time.perf_counter() - t0)
        O.set_simd(False)
        return float(np.median(times)), len(times), out

    # the scalar generic dots (the checker's definition), and the AVX-512 VNNI
    # form of the same dots (bit for bit the same outputs) where the host has it
    med_s, n_s, out_s = timed(False)
    simd = O.host_has_avx512_vnni()
    med, n, how = med_s, n_s, "scalar generic-order Q4_K / Q6_K x Q8_K dots"
    extra = {}
    if simd:
        med_v, n_v, out_v = timed(True)
        same = bool(np.array_equal(out_s.view(np.uint32), out_v.view(np.uint32)))
        extra = {"scalar_value": T_sample / med_s, "simd_bit_identical_to_scalar": same}
        if same:
            med, n, how = med_v, n_v, "AVX-512 VNNI Q4_K / Q6_K x Q8_K dots (bit for bit the scalar order)"
    res = {"value": T_sample / med, "unit": "tokens/s", "cores": cores, "kind": "port",
           "sample": f"{spec.name}: {T_sample} tokens x {n} runs (median {med * 1e3:.1f} ms), "
                     f"ggml-semantics CPU restatement (Q8_K activations, {how}), "
                     f"{cores} threads on {host_cpu()}", **extra}
    return res, parity


def host_cpu() -> str:
    """The host CPU's model name and vector ISA (from /proc/cpuinfo)."""
    model, flags = "unknown CPU", set()
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            if k.strip() == "model name" and model == "unknown CPU":
                model = v.strip()
            elif k.strip() == "flags" and not flags:
                flags = set(v.split())
    except OSError:
        pass
    isa = [f for f in ("avx512_vnni", "avx512bw", "avx512f", "avx2") if f in flags]
    return f"{model} ({', '.join(isa) if isa else 'no AVX2'})"


def make_layers(ctx, spec, n: int, tiled: bool) -> list:
    """n seeded layer copies; tiled: with tiled copies of their tables
    (mi_moe_tile, made at load time, outside every timed region) for the
    grouped GEMMs to read."""
    layers = [W.GpuLayer(ctx, spec, copy=c) for c in range(n)]
    if tiled:
        for g in layers:
            g.add_tiled(ctx)
    return layers


TABLES_TILED = ("GGUF tables + tiled copies (mi_moe_tile: Q4_K gate/up/down, Q6_K down) read by the grouped "
                "GEMMs, made at load time")
TABLES_ROWS = "GGUF rows only"


def config3_sweep(copies: int, tiled: bool = True) -> dict:
    """Config 3: qwen3omni layer (E 128, I 768, SwiGLU, Q4_K), batched decode
    at T = 1, 8, 32, 64 on both product paths of the kernel chain (grouped
    GEMV, grouped MFMA GEMM) and, up to 16 tokens, the fused kernel (the
    single-token kernel at T = 1, the batched one above), rotating layer
    copies.  Bytes per call = the touched experts' tables + the router
    (measured touched count); the crossover is the smallest T at which the
    chain's GEMM path is faster than its GEMV path.  tiled: the GEMM path
    reads the tables' tiled copies (gemm_rows_ms: the same path on the GGUF
    rows, beside it)."""
    spec = W.CONFIGS[3]["spec"]
    Ts = W.CONFIGS[3]["tokens"]
    ctx = M.Context(0)
    ctx.reserve(max(Ts), spec.D, spec.I, spec.E, spec.K)
    layers = make_layers(ctx, spec, copies, tiled)
    rows = []
    for T in Ts:
        xs = [W.gen_x(ctx, spec, T, copy=c) for c in range(copies)]
        out = M.DeviceBuffer(4 * T * spec.D)
        touched, _ = touched_experts(ctx, layers[0], xs[0], T)
        nbytes = W.algorithmic_bytes(spec, touched)
        row = {"tokens": T, "touched_experts": touched, "layer_bytes": nbytes}
        paths = [("gemv", 1 << 30), ("gemm", 1)]
        ctx.set_fused_decode(M.DECODE_CHAIN)
        for name, thr in paths:
            ctx.set_gemm_threshold(thr)
            ms, _ = time_layer(ctx, layers, xs, T, out, 100, 10)
            row[f"{name}_ms"] = ms
        if tiled:
            for g in layers:
                g.use_tiled(False)
            row["gemm_rows_ms"] = time_layer(ctx, layers, xs, T, out, 100, 10)[0]
            for g in layers:
                g.use_tiled(True)
        ctx.set_fused_decode(M.DECODE_FUSED)
        ctx.set_gemm_threshold(0)
        if T <= 16:
            row["fused_ms"] = time_layer(ctx, layers, xs, T, out, 100, 10)[0]
        best = min(v for k, v in row.items() if k.endswith("_ms") and k != "gemm_rows_ms")
        row["best_ms"] = best
        row["tokens_per_s"] = T / (best * 1e-3)
        row["GBs"] = nbytes / (best * 1e-3) / 1e9
        row["frac_hbm"] = row["GBs"] / PEAK_HBM_GBS
        log(f"config 3 T={T}: " + ", ".join(f"{k} {v:.4f}" for k, v in row.items() if k.endswith("_ms")) +
            f" | touched {touched}, {row['GBs']:.0f} GB/s")
        rows.append(row)
        del xs, out
    ctx.set_gemm_threshold(0)
    cross = next((r["tokens"] for r in rows if r["gemm_ms"] < r["gemv_ms"]), None)
    del layers
    ctx.close()
    return {"workload": "config 3: qwen3omni MoE layer (E 128, top-8, I 768, SwiGLU, Q4_K), batched decode",
            "layer_copies": copies, "tables": TABLES_TILED if tiled else TABLES_ROWS, "points": rows,
            "gemm_faster_from_tokens": cross}


def config4_stack(n_layers: int = 24, T_prefill: int = 2048, n_decode: int = 256, eps: float = 1e-6,
                  tiled: bool = True) -> dict:
    """Config 4: 24 moondream-shape layers (Q4_K gate/up and down, per-layer
    seeds), h <- h + MoE_l(RMSNorm(h)) with attention as identity: a
    2048-token prefill through the stack, then 256 single-token steps, each
    fed the RMSNorm of the previous step's final hidden state.  Reports
    sustained tokens/s, the prefill's TFLOP/s and the decode's GB/s (touched
    experts' bytes of every layer, counted on the first step)."""
    spec = W.md_spec(4, M.TYPE_Q4_K)
    ctx = M.Context(0)
    ctx.reserve(T_prefill, spec.D, spec.I, spec.E, spec.K)
    ctx.set_fused_decode(M.DECODE_FUSED)
    t0 = time.perf_counter()
    layers = make_layers(ctx, spec, n_layers, tiled)
    resident = sum(l.expert_bytes() * spec.E + 4 * spec.E * spec.D for l in layers)
    log(f"config 4: built {n_layers} layers in {time.perf_counter() - t0:.1f}s ({resident / 1e9:.2f} GB)")
    h0 = W.gen_x(ctx, spec, T_prefill)
    h = M.DeviceBuffer(4 * T_prefill * spec.D)
    h2 = M.DeviceBuffer(4 * T_prefill * spec.D)

    nrm = M.make_norm(M.NORM_RMS, eps)

    def stack_on(T, cur, nxt, st=None):
        # ping-pong: out = cur + MoE(RMSNorm(cur)) into the other buffer, the
        # norm applied where the MoE block reads its input
        sh = st.h if st is not None else None
        for L in layers:
            M.check("forward_norm", ctx.forward_norm(L.layer, nrm, cur, T, cur, nxt, stream=sh))
            cur, nxt = nxt, cur
        return cur

    def stack(T, cur, nxt):
        return stack_on(T, cur, nxt)

    def prefill():
        M.check("copy", M.load().mi_memcpy_d2d(h.ptr, h0.ptr, 4 * T_prefill * spec.D))
        return stack(T_prefill, h, h2)

    prefill()
    M.synchronize()
    e0, e1 = M.Event(), M.Event()
    reps = 3
    e0.record()
    for _ in range(reps):
        last = prefill()
    e1.record()
    e1.synchronize()
    pre_ms_stream = e0.elapsed_ms(e1) / reps
    # the same prefill with the stack captured once (n_layers even: the result
    # lands in h, like the issued run) and replayed after the input copy
    gs = M.Stream()
    g = M.Graph(gs, lambda st: stack_on(T_prefill, h, h2, st))
    M.check("copy", M.load().mi_memcpy_d2d(h.ptr, h0.ptr, 4 * T_prefill * spec.D))
    g.launch(gs)
    gs.synchronize()
    M.synchronize()
    e0.record(gs.h)
    for _ in range(reps):
        M.check("copy", M.load().mi_memcpy_d2d(h.ptr, h0.ptr, 4 * T_prefill * spec.D))
        g.launch(gs)
    e1.record(gs.h)
    e1.synchronize()
    pre_ms = e0.elapsed_ms(e1) / reps
    g.destroy()
    M.synchronize()
    # decode: the next token's input is the RMSNorm of the previous final hidden
    tok = M.DeviceBuffer(4 * spec.D)
    M.check("copy", M.load().mi_memcpy_d2d(tok.ptr, C.c_void_p(last.addr + 4 * (T_prefill - 1) * spec.D),
                                           4 * spec.D))
    M.check("rmsnorm", ctx.rmsnorm(tok, 1, spec.D, eps, tok))
    touched = 0
    counts = M.DeviceBuffer(4 * spec.E)
    r = M.Routing()
    r.counts = counts.addr
    cur, nxt = tok, M.DeviceBuffer(4 * spec.D)
    for L in layers:   # first step, counting the touched experts of every layer
        M.check("forward_norm", ctx.forward_norm(L.layer, nrm, cur, 1, cur, nxt, r))
        touched += int((counts.download(np.int32, (spec.E,)) > 0).sum())
        cur, nxt = nxt, cur
    step_bytes = sum(W.algorithmic_bytes(spec, 0) for _ in layers) + touched * (W.algorithmic_bytes(spec, 1) - W.algorithmic_bytes(spec, 0))
    def step(st=None):
        nonlocal cur, nxt
        sh = st.h if st is not None else None
        for L in layers:
            M.check("forward_norm", ctx.forward_norm(L.layer, nrm, cur, 1, cur, nxt, stream=sh))
            cur, nxt = nxt, cur
        M.check("rmsnorm", ctx.rmsnorm(cur, 1, spec.D, eps, cur, stream=sh))

    M.synchronize()
    e0.record()
    for _ in range(n_decode):
        step()
    e1.record()
    e1.synchronize()
    dec_ms_stream = e0.elapsed_ms(e1) / n_decode
    # one decode step captured (n_layers even: it ends in the buffer it
    # started from) and replayed n_decode times
    g = M.Graph(gs, step)
    M.synchronize()
    e0.record(gs.h)
    for _ in range(n_decode):
        g.launch(gs)
    e1.record(gs.h)
    e1.synchronize()
    dec_ms = e0.elapsed_ms(e1) / n_decode
    g.destroy()
    gs.destroy()
    M.synchronize()
    fl = n_layers * W.flops(spec, T_prefill)
    res = {"workload": f"config 4: {n_layers}-layer moondream-shape MoE stack (Q4_K, 64 experts, top-8), "
                       f"h + MoE(RMSNorm(h)), attention as identity",
           "resident_bytes": resident,
           "schedule": "each prefill / decode step captured once into a HIP graph and replayed",
           "prefill": {"tokens": T_prefill, "ms": pre_ms, "tokens_per_s": T_prefill / (pre_ms * 1e-3),
                       "TFLOPs": fl / (pre_ms * 1e-3) / 1e12, "stream_ms": pre_ms_stream},
           "decode": {"steps": n_decode, "ms_per_token": dec_ms, "tokens_per_s": 1.0 / (dec_ms * 1e-3),
                      "bytes_per_step": step_bytes, "GBs": step_bytes / (dec_ms * 1e-3) / 1e9,
                      "frac_hbm": step_bytes / (dec_ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
                      "stream_ms_per_token": dec_ms_stream,
                      "schedule": "per layer: one fused single-token kernel (RMSNorm of the row inside it), plain launch"}}
    log(f"config 4: prefill {pre_ms:.2f} ms ({res['prefill']['tokens_per_s']:.0f} tok/s, "
        f"{res['prefill']['TFLOPs']:.0f} TFLOP/s), decode {dec_ms:.3f} ms/token "
        f"({res['decode']['GBs']:.0f} GB/s); issued kernel by kernel: prefill {pre_ms_stream:.2f} ms, "
        f"decode {dec_ms_stream:.3f} ms/token")
    del layers
    ctx.close()
    return res


def mfma_counters(kernel: str, config: int = 1):
    """MFMA utilisation of `kernel` under `config` from the committed counter
    summary (profiles/mfma_counters.json: rocprofv3 SQ_VALU_MFMA_BUSY_CYCLES
    and SQ_INSTS_VALU_MFMA_MOPS_F16 per dispatch, and the shader clock
    measured under the kernel); None when that config was not measured."""
    p = ROOT / "profiles" / "mfma_counters.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get(profile_key(kernel, config))
    except (ValueError, AttributeError):
        return None


def prefill_line(config: int, args, primary: bool) -> dict:
    """One prefill configuration (1 or 2): the K forwards replayed as a HIP
    graph (stream-issued timing beside it), the per-stage times, the roofline
    of the gate/up grouped GEMM and the routing's load balance."""
    cfg = W.CONFIGS[config]
    spec = cfg["spec"]
    T = cfg["tokens"][0]
    ctx = M.Context(0)
    ctx.reserve(T, spec.D, spec.I, spec.E, spec.K)
    t0 = time.perf_counter()
    layers = make_layers(ctx, spec, args.copies, not args.no_tiled)
    xs = [W.gen_x(ctx, spec, T, copy=c) for c in range(args.copies)]
    out = M.DeviceBuffer(4 * T * spec.D)
    M.synchronize()
    log(f"built {args.copies} layer copies of {spec.name} in {time.perf_counter() - t0:.1f}s "
        f"({sum(l.expert_bytes() * spec.E for l in layers) / 1e9:.2f} GB of expert tables)")
    if args.calib_copy and primary:
        nbytes = 512 << 20
        src, dst = M.DeviceBuffer(nbytes), M.DeviceBuffer(nbytes)
        M.check("memcpy", M.load().mi_memcpy_d2d(dst.ptr, src.ptr, nbytes))
        M.synchronize()
        log(f"calibration copy: {nbytes} bytes device to device")
        del src, dst
    ms, extra = time_layer(ctx, layers, xs, T, out, args.steps, args.warmup)
    log(f"config {config}: {ms:.4f} ms/step, wall {extra['wall_ms_per_step']:.4f} ms/step (stream)")
    schedule = "stream: one host launch per kernel"
    gr = None if args.no_graph else time_layer_graph(ctx, layers, xs, T, out, args.steps)
    if gr is not None:
        log(f"config {config}: {gr[0]:.4f} ms/step, wall {gr[1]:.4f} ms/step (HIP graph replay)")
        extra = {"stream_ms_per_step": ms, "stream_wall_ms_per_step": extra["wall_ms_per_step"],
                 "wall_ms_per_step": gr[1]}
        ms = gr[0]
        schedule = "HIP graph of the K forwards (captured once, replayed; every kernel runs each step)"
    clocks, stages = time_layer(ctx, layers, xs, T, out, min(args.steps, 20), 2, profile=True)
    log(f"config {config} stages (ms): {json.dumps({k: round(v, 4) for k, v in stages.items()})}; "
        f"shader clock under the GEMMs (GHz): {json.dumps({k: round(v, 3) for k, v in clocks.items()})}")
    gu_ms = stages.get("gate_up", float("nan"))
    gu_flops = 2.0 * T * spec.K * spec.D * (2 * spec.I)
    achieved = gu_flops / (gu_ms * 1e-3) / 1e12
    touched, counts = touched_experts(ctx, layers[0], xs[0], T)
    srt = np.sort(counts)[::-1]
    roof = {"bound": "mfma", "kernel": "k_g4_glu (gate/up grouped GEMM + GLU)",
            "achieved": achieved, "peak": PEAK_MFMA_TFLOPS, "unit": "TFLOP/s",
            "frac": achieved / PEAK_MFMA_TFLOPS, "traffic": measured_traffic("k_g4_glu", config),
            "kernel_ms": gu_ms, "flops_per_launch": gu_flops}
    clk = clocks.get("gate_up")
    if clk:
        # the dense fp16 peak at the shader clock measured under this kernel:
        # 256 CUs x 4 SIMDs x 1024 flops per SIMD-cycle (one 32x32x16 MFMA,
        # 32768 flops, per 32 cycles) x clock
        peak_clk = CUS * FLOPS_PER_CU_CYCLE * clk * 1e9 / 1e12
        roof["measured_clock_ghz"] = clk
        roof["peak_at_measured_clock"] = peak_clk
        roof["frac_of_peak_at_measured_clock"] = achieved / peak_clk
    mc = mfma_counters("k_g4_glu", config)
    if mc:
        # MFMA busy share of the SIMD cycles under the kernel (committed profile)
        roof["mfma_busy_frac_profiled"] = mc.get("mfma_busy_frac")
    line = {
        "workload": f"config {config}: moondream3 MoE layer prefill" +
                    (", Zipf(1.2) router bias (load-imbalanced)" if spec.router_bias == "zipf" else ""),
        "tokens_per_s": T / (ms * 1e-3),
        "ms_per_step": ms,
        "config": {"workload": f"config {config}: moondream3 MoE layer prefill", "schedule": schedule,
                   "tokens": T, "n_embd": spec.D, "n_expert": spec.E, "n_expert_used": spec.K,
                   "n_ff": spec.I, "gate_up": "Q4_K",
                   "tables": TABLES_ROWS if args.no_tiled else TABLES_TILED,
                   "down": "Q6_K" if spec.down_type == M.TYPE_Q6_K else "Q4_K",
                   "act": ACT_NAMES[spec.act], "layer_copies": args.copies,
                   "touched_experts": touched, "layer_flops": W.flops(spec, T)},
        "roofline": roof,
        "stages_ms": stages,
        "gemm_clock_ghz": clocks,
        "load_balance": {"empty_experts": int((counts == 0).sum()),
                         "top4_share": float(srt[:4].sum() / counts.sum()),
                         "hot_expert_rows": [int(v) for v in srt[:4]],
                         "tiles_per_hot_expert": [int((v + 191) // 192) for v in srt[:4]],
                         "rows_per_expert_min_max": [int(counts[counts > 0].min()), int(counts.max())]},
        "extra": extra,
        "layer0": layers[0],
        "gpu_ref": gpu_reference(ctx, layers[0], xs[0], T) if primary and not args.no_cpu else None,
    }
    del layers, xs, out
    ctx.close()
    return line


def dense_reference(reps: int = 100) -> dict:
    """Dense fp16 x fp16 -> fp16 GEMMs (fp32 accumulation) with the FLOP counts
    of config 1's grouped products, through torch.matmul (hipBLASLt): gate/up
    [T*K, D] x [D, 2I], down [T*K, I] x [I, D].  A reference point for what the
    vendor library reaches on this GPU at the same work without dequantization,
    routing or fused epilogues; not part of the layer."""
    import torch  # only here: the layer itself runs on the HIP library

    spec = W.CONFIGS[1]["spec"]
    rows = W.CONFIGS[1]["tokens"][0] * spec.K
    out = {"metric": "dense_fp16_gemm_reference", "unit": "TFLOP/s", "library": "torch.matmul (hipBLASLt)",
           "torch": torch.__version__}
    torch.manual_seed(0)
    for name, (m, k, n) in (("gate_up", (rows, spec.D, 2 * spec.I)), ("down", (rows, spec.I, spec.D))):
        a = torch.randn(m, k, device="cuda", dtype=torch.float16)
        b = torch.randn(k, n, device="cuda", dtype=torch.float16)
        for _ in range(10):
            c = a @ b
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            c = a @ b
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1000.0 / reps
        out[name] = {"shape": f"{m}x{k} @ {k}x{n}", "gflop": 2.0 * m * n * k / 1e9, "us": us,
                     "tflops": 2.0 * m * n * k / us / 1e6, "frac_of_2.5PF": 2.0 * m * n * k / us / 1e6 / 2500.0}
        del a, b, c
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--copies", type=int, default=16)
    ap.add_argument("--config", type=int, default=1, choices=[1, 2])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-tiled", action="store_true",
                    help="no tiled copies of the Q4_K tables: the grouped GEMMs read the GGUF rows")
    ap.add_argument("--no-graph", action="store_true",
                    help="time the stream-issued forwards only (no HIP graph replay)")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-sweeps", action="store_true",
                    help="skip the config-3 batched-decode sweep and the config-4 layer stack")
    ap.add_argument("--no-stack", action="store_true",
                    help="skip the config-4 layer stack (its HIP graph capture) but run the config-3 sweep")
    ap.add_argument("--cpu-tokens", type=int, default=1024,
                    help="tokens of the CPU baseline sample (default: the whole config-1 batch)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run one 512 MiB device-to-device copy (the known-size kernel "
                         "that scales FETCH_SIZE / WRITE_SIZE counters to bytes)")
    ap.add_argument("--dense-ref", action="store_true",
                    help="only time dense fp16 GEMMs of the two grouped products' FLOP counts "
                         "through torch (hipBLASLt) on this GPU and print them as one JSON line: "
                         "the vendor library's rate at the same work, for reference")
    args = ap.parse_args()
    if args.dense_ref:
        print(json.dumps(dense_reference()), flush=True)
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(across GPUs the layer would shard by experts: each GPU holds E/N experts' "
              "tables, tokens reach them by an all-to-all, and each GPU runs these same kernels "
              "on its share)",
              file=sys.stderr)
        return 2

    M.load()
    info = M.device_info(0)
    log(f"device: {info}")
    line = prefill_line(args.config, args, primary=True)
    result = {
        "metric": "MoE layer tokens/s + % HBM roofline (decode) / % MFMA peak (prefill), 1 GPU",
        "value": line["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": line["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": line["config"],
        "roofline": line["roofline"],
        "stages_ms": line["stages_ms"],
    }
    extra = line["extra"]
    layers0 = line["layer0"]
    if args.config == 1 and not args.no_sweeps:
        c2 = prefill_line(2, args, primary=False)
        result["config2"] = {k: v for k, v in c2.items() if k not in ("extra", "layer0", "gpu_ref")}

    if not args.no_decode:
        dspec = W.CONFIGS[0]["spec"]
        dctx = M.Context(0)
        dctx.reserve(64, dspec.D, dspec.I, dspec.E, dspec.K)
        dl = [W.GpuLayer(dctx, dspec, copy=c) for c in range(args.copies)]
        dx = [W.gen_x(dctx, dspec, 1, copy=c) for c in range(args.copies)]
        dout = M.DeviceBuffer(4 * dspec.D)
        # fused single-token kernel, plain launch; the kernel chain is timed
        # beside it
        dctx.set_fused_decode(M.DECODE_FUSED)
        dms, _ = time_layer(dctx, dl, dx, 1, dout, 200, 20)
        _, dst = time_layer(dctx, dl, dx, 1, dout, 50, 5, profile=True)
        modes = {}
        for mname, mode in [("chain", M.DECODE_CHAIN)]:
            dctx.set_fused_decode(mode)
            modes[mname] = time_layer(dctx, dl, dx, 1, dout, 200, 20)[0]
        dctx.set_fused_decode(M.DECODE_FUSED)
        dtouched, _ = touched_experts(dctx, dl[0], dx[0], 1)
        layer_bytes = W.algorithmic_bytes(dspec, dtouched)
        if "decode1" in dst:
            # the whole block is one kernel launched back to back: its duration
            # is the timed loop's per-step time (HIP events around the loop on
            # the launch stream; rocprofv3 reports the same kernel average), and
            # its bytes are the layer's bytes
            kname, kbytes, kms = "k_decode1 (fused single-token MoE block)", layer_bytes, dms
        else:
            kname = "gate_up grouped GEMV (k_gemv GLU)"
            kbytes = dtouched * 2 * dspec.I * M.row_size(dspec.gate_type, dspec.D)
            kms = dst.get("gate_up", float("nan"))
        result["decode"] = {
            "workload": "config 0: moondream3 MoE layer, 1-token decode, Q4_K",
            "schedule": "fused kernel, plain launch (MI_DECODE_FUSED, the default)",
            "tokens_per_s": 1.0 / (dms * 1e-3), "ms_per_token": dms,
            "ms_per_token_other_schedules": modes,
            "layer_bytes": layer_bytes, "layer_GBs": layer_bytes / (dms * 1e-3) / 1e9,
            "layer_frac_hbm": layer_bytes / (dms * 1e-3) / 1e9 / PEAK_HBM_GBS,
            "roofline": {"bound": "hbm", "kernel": kname,
                         "achieved": kbytes / (kms * 1e-3) / 1e9, "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": kbytes / (kms * 1e-3) / 1e9 / PEAK_HBM_GBS,
                         "kernel_ms": kms, "bytes_per_launch": kbytes,
                         "traffic": measured_traffic("k_decode1")},
            "stages_ms": dst,
        }
        del dl, dx
        dctx.close()

    if not args.no_cpu:
        cb, parity = cpu_baseline(layers0.spec, layers0, args.cpu_tokens, line["gpu_ref"])
        result["cpu_baseline"] = cb
        if parity is not None:
            result["parity"] = parity
    del layers0, line

    if not args.no_sweeps:
        result["config3"] = config3_sweep(args.copies, not args.no_tiled)
        if not args.no_stack:
            result["config4"] = config4_stack(tiled=not args.no_tiled)
    result.update({k: v for k, v in extra.items() if k.startswith("stream")})
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
