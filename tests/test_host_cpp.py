"""The C++ host mirror of the reference's vqa::moe segment
(skyvision.cpp_amd/host/vqa_moe.{hpp,cpp}; reference
src/core/engine/moe_compute.hpp:25-86).

CPU: the header declares the reference's four builders with their argument
lists, and the self-test binary is built and linked to libmimoe.so.
GPU: the self-test runs - the reference's own known answer (D = 2, I = 3,
K = 2, F32 SiLU -> [3.6423913, 4.1931758], moe_compute.cpp:154-230) through
the per-slot and slot-table forms, the residual split, and the nullptr
returns of the argument checks; and vqa::moe::GraphB, the decode driver's
graph B (Hooks::build_b / feed_b, moe_decode_driver.hpp:125-144): the same
known answer with the driver's routing, and a Q4_K layer routing its own
rows bit-identical to mi_moe_forward, also with tiled copies of its tables
(GraphB's tiled option, 40 rows: the grouped GEMMs read the copies)."""
import pathlib
import re
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
HOST = ROOT / "skyvision.cpp_amd" / "host"
BIN = HOST / "vqa_moe_selftest"


def test_header_mirrors_reference_builders():
    h = (HOST / "vqa_moe.hpp").read_text()
    assert "namespace vqa" in h and "namespace moe" in h
    sigs = {
        "build_expert_ffn": ["x", "gate", "up", "down", "w", "act"],
        "build_expert_ffn_res": ["x", "res", "gate", "up", "down", "w", "act"],
        "build_expert_ffn_table": ["x", "gate_table", "up_table", "down_table", "gate_up_ids", "down_ids", "w",
                                   "act"],
        "build_expert_ffn_table_res": ["x", "res", "gate_table", "up_table", "down_table", "gate_up_ids",
                                       "down_ids", "w", "act"],
    }
    for name, args in sigs.items():
        m = re.search(r"Tensor \*" + name + r"\(([^;]*)\);", h)
        assert m, name
        got = [re.findall(r"([A-Za-z_]+)\s*(?:=[^,]*)?$", a.strip())[0] for a in m.group(1).split(",")]
        assert got[0] == "s" and got[1:] == args, (name, got)


def test_selftest_built_and_linked():
    if not BIN.exists():
        pytest.fail(f"{BIN} is not built: run __graft_entry__.build()")
    out = subprocess.run(["ldd", str(BIN)], capture_output=True, text=True).stdout
    assert "libmimoe.so" in out and "not found" not in out, out


@pytest.mark.gpu
def test_selftest_runs_on_gpu():
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=120)
    print(r.stderr, flush=True)
    assert r.returncode == 0, r.stderr
    assert "PASS (0 failures)" in r.stderr
    m = re.search(r"moe out = \[([-0-9.]+), ([-0-9.]+)\]", r.stderr)
    assert m, r.stderr
    # the reference's hand-computed answer, to its 1e-5
    assert abs(float(m.group(1)) - 3.6423913) < 1e-5 and abs(float(m.group(2)) - 4.1931758) < 1e-5
    m = re.search(r"graphb out = \[([-0-9.]+), ([-0-9.]+)\]", r.stderr)
    assert m, r.stderr
    assert abs(float(m.group(1)) - 3.6423913) < 1e-5 and abs(float(m.group(2)) - 4.1931758) < 1e-5
    assert "graphb q4_k layer: bit-identical to mi_moe_forward" in r.stderr
    assert "graphb q4_k layer with tiled copies, 40 rows: bit-identical to mi_moe_forward" in r.stderr
