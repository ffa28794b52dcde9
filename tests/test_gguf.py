"""GGUF expert-tensor loader (mi_gguf_*; csrc/gguf.cpp).

The files are written here by a small GGUF v3 writer (magic, version, counts,
metadata, tensor infos, aligned data), in the two layouts the reference's
converters produce: moondream3 (blk.N.ffn_gate_inp.{weight F16, bias},
fused [h | g] ffn_up_exps Q4_K, ffn_down_exps Q6_K; convert_hf_to_gguf.py:
173-183, moondream.cpp:149-172, 241-251) and qwen3omni (blk.N.ffn_router F32,
ffn_gate_exps / ffn_up_exps / ffn_down_exps; convert_qwen3omni.py:188-219).
CPU: parsing, metadata, tensor infos and every malformed-file error (no
device).  GPU: a loaded layer's forward matches the CPU oracle run on the
tables the test wrote (the F16 router promoted to F32 by numpy): routing
bit-exact, output rel-L2 <= 1e-2; and it is bit-identical to the forward of
the same tables uploaded directly.
"""
import pathlib
import struct

import numpy as np
import pytest

import mimoe as M
import pyoracle as O
from _util import max_abs, rel_l2

GV_U32, GV_F32, GV_STR, GV_ARR = 4, 6, 8, 9


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def write_gguf(path, kv, tensors, alignment=32, version=3, magic=b"GGUF"):
    """kv: [(key, gguf type, value)]; tensors: [(name, ggml type, ne, bytes)]."""
    out = bytearray(magic + struct.pack("<I", version) + struct.pack("<QQ", len(tensors), len(kv)))
    for key, t, v in kv:
        out += _s(key) + struct.pack("<I", t)
        if t == GV_STR:
            out += _s(v)
        elif t == GV_U32:
            out += struct.pack("<I", v)
        elif t == GV_F32:
            out += struct.pack("<f", v)
        elif t == GV_ARR:   # (element type, values) - u32 elements here
            out += struct.pack("<IQ", GV_U32, len(v)) + b"".join(struct.pack("<I", e) for e in v)
    off = 0
    offs = []
    for name, typ, ne, data in tensors:
        offs.append(off)
        out += _s(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        out += struct.pack("<IQ", typ, off)
        off += (len(data) + alignment - 1) // alignment * alignment
    out += b"\0" * ((-len(out)) % alignment)
    for (name, typ, ne, data), o in zip(tensors, offs):
        out += data + b"\0" * ((-len(data)) % alignment)
    pathlib.Path(path).write_bytes(bytes(out))


D, E, K, I = 512, 8, 2, 256


def _q(type_, a):
    return a.astype(np.float16).tobytes() if type_ == O.TYPE_F16 else O.quantize(type_, a).tobytes()


def table_types(fused, qtype):
    """(gate/up type, down type) of a test file: k-quant files as moondream3
    --q4 mixes them (Q4_K gate/up, Q6_K down) or qwen3omni Q4_K; the other
    types throughout, as the converters' --outtype writes them"""
    if qtype == O.TYPE_Q4_K:
        return O.TYPE_Q4_K, (O.TYPE_Q6_K if fused else O.TYPE_Q4_K)
    return qtype, qtype


def _tables(seed, fused, qtype=O.TYPE_Q4_K):
    rng = np.random.default_rng(seed)
    w = lambda *s: (rng.standard_normal(s) * 0.02).astype(np.float32)
    router = w(E, D)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    gt, dt = table_types(fused, qtype)
    t = {}
    if fused:
        t["up"] = _q(gt, w(E * 2 * I, D))
    else:
        t["gate"] = _q(gt, w(E * I, D))
        t["up"] = _q(gt, w(E * I, D))
    t["down"] = _q(dt, w(E * D, I))
    return router, bias, t


def moondream_file(path, seed=1, alignment=32, qtype=O.TYPE_Q4_K):
    router, bias, t = _tables(seed, True, qtype)
    gt, dt = table_types(True, qtype)
    r16 = router.astype(np.float16)
    kv = [("general.architecture", GV_STR, "moondream"), ("moondream.expert_used_count", GV_U32, K),
          ("general.alignment", GV_U32, alignment), ("moondream.some_list", GV_ARR, [1, 2, 3]),
          ("moondream.norm_eps", GV_F32, 1e-5)]
    tensors = [("blk.3.ffn_gate_inp.weight", M.TYPE_F16, [D, E], r16.tobytes()),
               ("blk.3.ffn_gate_inp.bias", M.TYPE_F32, [E], bias.tobytes()),
               ("blk.3.ffn_up_exps.weight", gt, [D, 2 * I, E], t["up"]),
               ("blk.3.ffn_down_exps.weight", dt, [I, D, E], t["down"])]
    write_gguf(path, kv, tensors, alignment=alignment)
    return r16.astype(np.float32), bias, t


def qwen_file(path, seed=2, qtype=O.TYPE_Q4_K):
    router, _, t = _tables(seed, False, qtype)
    gt, dt = table_types(False, qtype)
    kv = [("general.architecture", GV_STR, "qwen3omni"), ("qwen3omni.expert_used_count", GV_U32, K)]
    tensors = [("blk.0.ffn_router.weight", M.TYPE_F32, [D, E], router.tobytes()),
               ("blk.0.ffn_gate_exps.weight", gt, [D, I, E], t["gate"]),
               ("blk.0.ffn_up_exps.weight", gt, [D, I, E], t["up"]),
               ("blk.0.ffn_down_exps.weight", dt, [I, D, E], t["down"])]
    write_gguf(path, kv, tensors)
    return router, t


def test_gguf_parse(tmp_path):
    p = tmp_path / "md.gguf"
    moondream_file(p, alignment=64)
    g = M.Gguf(p)
    assert g.get_int("moondream.expert_used_count") == K
    assert g.get_int("general.alignment") == 64
    assert g.get_int("moondream.norm_eps") is None       # a float: not an integer key
    assert g.get_int("absent") is None
    t, ne, nb = g.tensor_info("blk.3.ffn_up_exps.weight")
    assert (t, ne, nb) == (M.TYPE_Q4_K, [D, 2 * I, E, 1], E * 2 * I * (D // 256) * 144)
    t, ne, nb = g.tensor_info("blk.3.ffn_gate_inp.weight")
    assert (t, ne, nb) == (M.TYPE_F16, [D, E, 1, 1], D * E * 2)
    assert g.tensor_info("blk.3.ffn_gate_exps.weight") is None
    g.close()
    # the converters' default expert type
    p8 = tmp_path / "md8.gguf"
    moondream_file(p8, qtype=O.TYPE_Q8_0)
    g = M.Gguf(p8)
    t, ne, nb = g.tensor_info("blk.3.ffn_up_exps.weight")
    assert (t, ne, nb) == (M.TYPE_Q8_0, [D, 2 * I, E, 1], E * 2 * I * (D // 32) * 34)
    g.close()


def test_gguf_bad_files(tmp_path):
    lib = M.load()
    h = M.P()
    assert lib.mi_gguf_open(M.C.byref(h), str(tmp_path / "missing.gguf").encode()) == -9
    good = tmp_path / "md.gguf"
    moondream_file(good)
    raw = good.read_bytes()
    cases = {
        "magic": b"GGUX" + raw[4:],
        "version": raw[:4] + struct.pack("<I", 1) + raw[8:],
        "truncated infos": raw[:200],
        "data past end": raw[:-4096],
    }
    for name, data in cases.items():
        p = tmp_path / f"bad_{name.replace(' ', '_')}.gguf"
        p.write_bytes(data)
        assert lib.mi_gguf_open(M.C.byref(h), str(p).encode()) == -9, name
    assert lib.mi_gguf_open(M.C.byref(h), None) == -1


@pytest.mark.gpu
@pytest.mark.parametrize("style,qtype", [("moondream", O.TYPE_Q4_K), ("qwen3omni", O.TYPE_Q4_K),
                                         ("moondream", O.TYPE_Q8_0), ("qwen3omni", O.TYPE_Q8_0),
                                         ("qwen3omni", O.TYPE_F16), ("moondream", O.TYPE_Q5_0)])
def test_gguf_layer_forward(tmp_path, style, qtype):
    ctx = M.Context(0)
    T = 300
    ctx.reserve(T, D, I, E, K)
    p = tmp_path / f"{style}.gguf"
    if style == "moondream":
        router, bias, t = moondream_file(p, qtype=qtype)
        blk, act, fused = 3, M.ACT_GELU_ERF_GP1, True
    else:
        router, t = qwen_file(p, qtype=qtype)
        bias, blk, act, fused = None, 0, M.ACT_SILU, False
    gt, dt = table_types(fused, qtype)
    g = M.Gguf(p)
    L, buf = g.load_moe_layer(blk, act)
    assert (L.n_embd, L.n_expert, L.n_expert_used, L.n_ff, L.fused_gate_up) == (D, E, K, I, int(fused))
    # the same tables uploaded directly
    rd = M.to_device(router)
    bd = M.to_device(bias) if bias is not None else None
    keep = {k: M.to_device(np.frombuffer(v, np.uint8)) for k, v in t.items()}   # alive through the forwards
    down = M.tensor(keep["down"], dt, [I, D, E])
    if fused:
        gate = M.tensor(keep["up"], gt, [D, 2 * I, E])
        up = None
    else:
        gate = M.tensor(keep["gate"], gt, [D, I, E])
        up = M.tensor(keep["up"], gt, [D, I, E])
    Ld = M.make_layer(D, E, K, I, rd, bd, gate, up, down, fused, act)
    x = np.random.default_rng(5).standard_normal((T, D)).astype(np.float32)
    xd = M.to_device(x)
    o1, o2 = M.DeviceBuffer(4 * T * D), M.DeviceBuffer(4 * T * D)
    sel = M.DeviceBuffer(4 * T * K)
    r = M.Routing()
    r.sel = sel.addr
    M.check("forward gguf", ctx.forward(L, xd, T, xd, o1, r))
    M.check("forward direct", ctx.forward(Ld, xd, T, xd, o2))
    a, b = o1.download(np.float32, (T, D)), o2.download(np.float32, (T, D))
    assert np.isfinite(a).all() and np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # the oracle on the written tables; router = the file's F16 values promoted by numpy
    OL = dict(D=D, E=E, K=K, I=I, router_w=router, router_b=bias, gate_type=gt,
              gate=np.frombuffer(t["up"] if fused else t["gate"], np.uint8),
              up=None if fused else np.frombuffer(t["up"], np.uint8), fused=fused,
              down_type=dt, down=np.frombuffer(t["down"], np.uint8), act=act)
    ref, dbg = O.moe_forward(OL, x, x)
    assert np.array_equal(sel.download(np.int32, (T, K)), dbg["sel"]), "routing of the loaded layer"
    e = rel_l2(a - x, ref - x)
    print(f"gguf {style} type {qtype}: loaded layer vs oracle rel-L2 {e:.3e} max-abs {max_abs(a, ref):.3e}", flush=True)
    assert e <= 1e-2
    M.check("free", M.load().mi_dev_free(buf))
    g.close()
    ctx.close()
