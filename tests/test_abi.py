"""The C-ABI library loads on a host without a GPU and exports every entry
point its headers declare; the pure host functions (version, row sizes,
status strings) answer without touching a device."""
import ctypes as C
import pathlib
import re

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
LIB = ROOT / "skyvision.cpp_amd" / "libmimoe.so"
HEADERS = sorted((ROOT / "include").glob("*.h"))

DECL = re.compile(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**\s*(mi_[a-z0-9_]+)\s*\(", re.M)


def declared():
    names = []
    for h in HEADERS:
        names += DECL.findall(h.read_text())
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    if not LIB.exists():
        pytest.fail(f"{LIB} is not built: run __graft_entry__.build()")
    return C.CDLL(str(LIB))


def test_headers_declare_entry_points():
    names = declared()
    for must in ["mi_moe_ctx_create", "mi_moe_forward", "mi_moe_expert_ffn", "mi_top_k", "mi_mul_mat_id",
                 "mi_quantize", "mi_fill_normal", "mi_row_size", "mi_moe_abi_version"]:
        assert must in names


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_abi_version(lib):
    hdr = (ROOT / "include" / "mi_moe.h").read_text()
    ver = int(re.search(r"#define MI_MOE_ABI_VERSION (\d+)", hdr).group(1))
    lib.mi_moe_abi_version.restype = C.c_int
    assert lib.mi_moe_abi_version() == ver


def test_row_size(lib):
    lib.mi_row_size.restype = C.c_size_t
    lib.mi_row_size.argtypes = [C.c_int32, C.c_int64]
    assert lib.mi_row_size(12, 2048) == 8 * 144      # Q4_K
    assert lib.mi_row_size(14, 1024) == 4 * 210      # Q6_K
    assert lib.mi_row_size(0, 7) == 28               # F32
    assert lib.mi_row_size(12, 100) == 0             # not a multiple of 256


def test_status_strings(lib):
    lib.mi_moe_status_string.restype = C.c_char_p
    lib.mi_moe_status_string.argtypes = [C.c_int]
    seen = {lib.mi_moe_status_string(s) for s in range(0, -9, -1)}
    assert len(seen) == 9 and all(seen)


def test_null_arguments_rejected_without_device(lib):
    # argument checks come before any HIP call
    lib.mi_moe_forward.restype = C.c_int
    assert lib.mi_moe_forward(None, None, None, C.c_int64(1), None, None, None, None) == -1


def test_status_codes_match_header():
    """The binding's status constants are the header's mi_moe_status values."""
    import mimoe as M
    text = (ROOT / "include" / "mi_moe.h").read_text()
    codes = dict(re.findall(r"MI_MOE_(OK|ERR_[A-Z]+)\s*=\s*(-?\d+)", text))
    assert len(codes) == 10, codes
    for name, v in codes.items():
        assert getattr(M, name) == int(v), name


def test_layer_struct_layout_matches_header(tmp_path):
    """The binding's mi_moe_layer / mi_tensor mirrors have the C layout: a
    program compiled against include/mi_moe.h prints sizeof and every field's
    offset (gcc, host only)."""
    import ctypes as Cty
    import subprocess

    import mimoe as M
    fields = [f for f, _ in M.Layer._fields_]
    src = tmp_path / "layout.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "mi_moe.h"\nint main(void) {\n'
                   '  printf("%zu %zu\\n", sizeof(mi_moe_layer), sizeof(mi_tensor));\n' +
                   "".join(f'  printf("%zu\\n", offsetof(mi_moe_layer, {f}));\n' for f in fields) +
                   "  return 0;\n}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()
    assert int(out[0]) == Cty.sizeof(M.Layer) and int(out[1]) == Cty.sizeof(M.Tensor)
    for f, off in zip(fields, out[2:]):
        assert getattr(M.Layer, f).offset == int(off), f
