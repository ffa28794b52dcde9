"""Synthetic MoE-layer workloads built on the GPU.

Every tensor is a seeded N(mean, std^2) stream produced by mi_fill_normal and,
for expert tables, quantized on the GPU by mi_quantize (ggml's reference
quantizers).  Value i of (seed, stream) is a pure function, so a CPU checker
can regenerate the same bytes.

Stream ids inside a layer (add 64 * copy for rotated layer copies):
  1 router weight   2 router bias   3 gate (or fused up_exps)   4 up
  5 down            6 x             7 residual
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np

import mimoe as M

S_ROUTER_W, S_ROUTER_B, S_GATE, S_UP, S_DOWN, S_X, S_RES = 1, 2, 3, 4, 5, 6, 7
STREAMS_PER_COPY = 64


@dataclasses.dataclass(frozen=True)
class LayerSpec:
    name: str
    D: int
    E: int
    K: int
    I: int
    fused: bool          # moondream ffn_up_exps = [h | g]
    gate_type: int
    down_type: int
    act: int
    router_bias: str     # "none" | "zipf"
    seed: int
    w_std: float = 0.02
    router_std: float = 0.02


def md_spec(cfg: int, down_type: int, bias: str = "none", act: int = M.ACT_GELU_TANH) -> LayerSpec:
    """moondream3-shape MoE layer: D 2048, 64 experts, top-8, I 1024, fused
    gate/up (moondream.cpp:93-96, 509-544).  The BASELINE configs 0-2 state
    the GeGLU as tanh-GELU on gate x up (the default here); moondream3's own
    graph uses gelu_erf(h) * (g + 1) (moondream.cpp:534, ACT_GELU_ERF_GP1),
    which the parity tests cover as well."""
    return LayerSpec(f"md_cfg{cfg}", 2048, 64, 8, 1024, True, M.TYPE_Q4_K, down_type, act, bias,
                     0x5EED0000 + cfg)


def qo_spec(cfg: int = 3) -> LayerSpec:
    """qwen3omni MoE layer: D 2048, 128 experts, top-8, I 768, SwiGLU
    (qwen3omni_model.cpp:755-780)."""
    return LayerSpec(f"qo_cfg{cfg}", 2048, 128, 8, 768, False, M.TYPE_Q4_K, M.TYPE_Q4_K,
                     M.ACT_SILU, "none", 0x5EED0000 + cfg)


# BASELINE.json configs
CONFIGS = {
    0: dict(spec=md_spec(0, M.TYPE_Q4_K), tokens=[1]),
    1: dict(spec=md_spec(1, M.TYPE_Q6_K), tokens=[1024]),
    2: dict(spec=md_spec(2, M.TYPE_Q6_K, bias="zipf"), tokens=[1024]),
    3: dict(spec=qo_spec(3), tokens=[1, 8, 32, 64]),
}

# config 2 skew: bias_e = BETA * log(p_e), p_e ~ rank^-1.2 (Zipf s = 1.2) over a
# seeded permutation of the experts; the last 16 experts of the permutation get
# DEAD_BIAS (finite, guarantees zero tokens).  BETA is fixed so the 4 hottest
# experts take about 40 % of the 8192 assignments of the config-2 inputs
# (40.4 % with 16 idle experts for layer copy 0; tests/test_workloads.py).
ZIPF_S = 1.2
N_DEAD = 16
DEAD_BIAS = -1.0e4
ZIPF_BETA = 0.8


def zipf_bias(E: int, seed: int, beta: float = ZIPF_BETA) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64(seed))
    order = rng.permutation(E)                  # order[r] = expert with rank r
    live = E - N_DEAD
    ranks = np.arange(1, live + 1, dtype=np.float64)
    p = ranks ** (-ZIPF_S)
    p /= p.sum()
    b = np.full(E, DEAD_BIAS, dtype=np.float32)
    b[order[:live]] = (beta * np.log(p)).astype(np.float32)
    return b


def table_shape(spec: LayerSpec, which: str):
    """(Kin, N) of an expert table (ggml ne[0], ne[1])."""
    if which == "gate":
        return spec.D, (2 * spec.I if spec.fused else spec.I)
    if which == "up":
        return spec.D, spec.I
    return spec.I, spec.D


class GpuLayer:
    """Device-resident layer: router, quantized expert tables, descriptor."""

    def __init__(self, ctx: M.Context, spec: LayerSpec, copy: int = 0, keep_f32: bool = False):
        self.spec = spec
        self.copy = copy
        base = STREAMS_PER_COPY * copy
        D, E, I = spec.D, spec.E, spec.I
        self.router_w = M.DeviceBuffer(4 * E * D)
        M.check("mi_fill_normal", ctx.fill_normal(self.router_w, E * D, spec.seed, base + S_ROUTER_W,
                                                  0.0, spec.router_std))
        self.router_b = None
        if spec.router_bias == "zipf":
            self.bias_host = zipf_bias(E, spec.seed + copy)
            self.router_b = M.to_device(self.bias_host)
        else:
            self.bias_host = None
        self.tables = {}
        self.f32 = {}
        names = ["gate", "down"] if spec.fused else ["gate", "up", "down"]
        stream_of = {"gate": S_GATE, "up": S_UP, "down": S_DOWN}
        for nm in names:
            Kin, N = table_shape(spec, nm)
            ttype = spec.down_type if nm == "down" else spec.gate_type
            n = E * N * Kin
            tmp = M.DeviceBuffer(4 * n)
            M.check("mi_fill_normal", ctx.fill_normal(tmp, n, spec.seed, base + stream_of[nm], 0.0,
                                                      spec.w_std))
            q = M.DeviceBuffer(M.row_size(ttype, Kin) * E * N)
            M.check("mi_quantize", ctx.quantize(ttype, tmp, q, E * N, Kin))
            if keep_f32:
                self.f32[nm] = tmp
            else:
                tmp.free()
            self.tables[nm] = (q, ttype, Kin, N)
        M.synchronize()
        self.layer = M.make_layer(
            D, E, spec.K, I, self.router_w, self.router_b,
            self.tensor("gate"), self.tensor("up") if "up" in self.tables else None,
            self.tensor("down"), spec.fused, spec.act)

    def add_tiled(self, ctx: M.Context, q6k: bool = True) -> None:
        """Tiled copies (mi_moe_tile) of the Q4_K tables and, with q6k, of a
        Q6_K down table, attached to the layer descriptor for the grouped
        GEMMs to read."""
        self.tiled = {}
        for nm, (q, ttype, Kin, N) in self.tables.items():
            if ttype != M.TYPE_Q4_K and not (q6k and nm == "down" and ttype == M.TYPE_Q6_K):
                continue
            src = self.tensor(nm)
            dst = M.DeviceBuffer(M.tiled_bytes(src))
            desc = M.Tensor()
            M.check("mi_moe_tile", ctx.tile(src, dst, desc))
            desc._buf = dst
            self.tiled[nm] = desc
        M.synchronize()
        self.use_tiled(True)

    def use_tiled(self, on: bool) -> None:
        """Point the descriptor's tiled fields at the copies (on) or at none."""
        for nm, desc in getattr(self, "tiled", {}).items():
            setattr(self.layer, nm + "_tiled", desc if on else M.Tensor())

    def tensor(self, nm: str) -> M.Tensor:
        q, ttype, Kin, N = self.tables[nm]
        return M.tensor(q, ttype, [Kin, N, self.spec.E])

    def weight_bytes(self, nm: str) -> int:
        q, ttype, Kin, N = self.tables[nm]
        return q.nbytes

    def expert_bytes(self) -> int:
        """bytes of one expert across all its tables"""
        return sum(self.weight_bytes(nm) for nm in self.tables) // self.spec.E

    def download_tables(self) -> dict:
        out = {}
        for nm, (q, ttype, Kin, N) in self.tables.items():
            rs = M.row_size(ttype, Kin)
            out[nm] = q.download(np.uint8, (self.spec.E, N, rs))
        return out

    def download_router(self) -> np.ndarray:
        return self.router_w.download(np.float32, (self.spec.E, self.spec.D))


def gen_x(ctx: M.Context, spec: LayerSpec, T: int, copy: int = 0, stream: int = S_X) -> M.DeviceBuffer:
    buf = M.DeviceBuffer(4 * max(1, T) * spec.D)
    if T > 0:
        M.check("mi_fill_normal", ctx.fill_normal(buf, T * spec.D, spec.seed,
                                                  STREAMS_PER_COPY * copy + stream, 0.0, 1.0))
    return buf


def algorithmic_bytes(spec: LayerSpec, touched_experts: int) -> int:
    """bytes a layer call must read: the touched experts' tables + the router"""
    rs_g = M.row_size(spec.gate_type, spec.D)
    rs_d = M.row_size(spec.down_type, spec.I)
    n_gate_rows = (2 if spec.fused else 1) * spec.I
    per_expert = n_gate_rows * rs_g + (0 if spec.fused else spec.I * rs_g) + spec.D * rs_d
    return touched_experts * per_expert + 4 * spec.E * spec.D


def flops(spec: LayerSpec, T: int) -> float:
    """2 * MACs of the router and the K selected experts per token"""
    per_tok = 2.0 * spec.K * 3 * spec.D * spec.I + 2.0 * spec.D * spec.E
    return per_tok * T
