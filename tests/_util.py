"""Shared test helpers: metrics, small layer specs, CPU-side layer generation."""
from __future__ import annotations

import dataclasses

import numpy as np

import pyoracle as O
import workloads as W


def rel_l2(got, ref) -> float:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm((got - ref).ravel()) / (np.linalg.norm(ref.ravel()) + 1e-30))


def max_abs(got, ref) -> float:
    d = np.abs(np.asarray(got, dtype=np.float64) - np.asarray(ref, dtype=np.float64))
    return float(d.max()) if d.size else 0.0


def small_spec(name="small", D=512, E=8, K=2, I=256, fused=True, gate_type=O.TYPE_Q4_K,
               down_type=O.TYPE_Q4_K, act=O.ACT_GELU_ERF_GP1, bias="none", seed=0x5EED1000,
               w_std=0.02):
    return W.LayerSpec(name, D, E, K, I, fused, gate_type, down_type, act, bias, seed, w_std)


def cpu_layer(spec: W.LayerSpec, copy: int = 0, nthreads: int = 0) -> dict:
    """The layer W.GpuLayer builds, regenerated on the CPU with the oracle's
    generator and quantizers (same seeds and streams -> same bytes)."""
    base = W.STREAMS_PER_COPY * copy
    D, E, I = spec.D, spec.E, spec.I
    rw = O.fill_normal(E * D, spec.seed, base + W.S_ROUTER_W, 0.0, spec.router_std,
                       nthreads).reshape(E, D)
    rb = W.zipf_bias(E, spec.seed + copy) if spec.router_bias == "zipf" else None
    out = dict(D=D, E=E, K=spec.K, I=I, router_w=rw, router_b=rb, gate_type=spec.gate_type,
               down_type=spec.down_type, fused=spec.fused, act=spec.act)
    names = ["gate", "down"] if spec.fused else ["gate", "up", "down"]
    stream_of = {"gate": W.S_GATE, "up": W.S_UP, "down": W.S_DOWN}
    for nm in names:
        Kin, N = W.table_shape(spec, nm)
        ttype = spec.down_type if nm == "down" else spec.gate_type
        f = O.fill_normal(E * N * Kin, spec.seed, base + stream_of[nm], 0.0, spec.w_std,
                          nthreads).reshape(E * N, Kin)
        out[nm] = O.quantize(ttype, f, nthreads).reshape(E, N, -1)
    return out


def cpu_x(spec: W.LayerSpec, T: int, copy: int = 0, stream: int = W.S_X) -> np.ndarray:
    return O.fill_normal(T * spec.D, spec.seed, W.STREAMS_PER_COPY * copy + stream, 0.0,
                         1.0).reshape(T, spec.D)


def oracle_layer_dict(tables: dict, spec: W.LayerSpec, router_w, router_b) -> dict:
    d = dict(D=spec.D, E=spec.E, K=spec.K, I=spec.I, router_w=router_w, router_b=router_b,
             gate_type=spec.gate_type, down_type=spec.down_type, fused=spec.fused, act=spec.act,
             gate=tables["gate"], down=tables["down"])
    if "up" in tables:
        d["up"] = tables["up"]
    return d
