"""pytest setup: the `gpu` marker, import paths, and device detection.

`-m "not gpu"` runs the oracle, host-logic and ABI-export tests (no GPU);
`-m gpu` runs the parity tests through the C ABI on an MI355X.
"""
import os
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
for p in (ROOT / "skyvision.cpp_amd", ROOT / "oracle", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")


def _have_gpu() -> bool:
    """A GPU node exposes /dev/kfd.  Where it exists the GPU tests run and a
    missing or broken HIP library fails them loudly (no silent skip)."""
    return os.path.exists("/dev/kfd")


def pytest_collection_modifyitems(config, items):
    gpu_items = [it for it in items if "gpu" in it.keywords]
    if not gpu_items:
        return
    if os.environ.get("MIMOE_REQUIRE_GPU") == "1":
        return
    if not _have_gpu():
        skip = pytest.mark.skip(reason="no GPU visible")
        for it in gpu_items:
            it.add_marker(skip)
