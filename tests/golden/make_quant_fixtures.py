"""Writes the golden Q4_K / Q6_K block fixtures from the reference's own
Python ports of ggml's quantizers (convert/q4k.py quantize_q4_k,
convert/q6k.py _quantize_q6_k_numpy), which nothing else available here can
pin byte for byte.  Run once, in the build container, where the reference
tree is mounted (REF_ROOT, default /root/reference); only the resulting data
(inputs + packed blocks) is committed, never the reference code.

  python tests/golden/make_quant_fixtures.py
"""
import os
import pathlib
import sys

import numpy as np

REF_ROOT = pathlib.Path(os.environ.get("REF_ROOT", "/root/reference"))
HERE = pathlib.Path(__file__).resolve().parent


def rows():
    rng = np.random.default_rng(0x51D0)
    r = [np.zeros(256, np.float32),                                  # zero block
         np.full(256, 1e-20, np.float32),                            # below GROUP_MAX_EPS
         np.full(256, 0.75, np.float32),                             # constant
         np.full(256, -1.0, np.float32),
         (rng.standard_normal(256) * 1e4).astype(np.float32),        # large magnitude
         np.concatenate([rng.standard_normal(128) * 1e-3, rng.standard_normal(128) * 10]).astype(np.float32)]
    r += list((rng.standard_normal((40, 256)) * 0.02).astype(np.float32))   # weight-like
    r += list(rng.standard_normal((18, 256)).astype(np.float32))
    return np.stack(r)


def main():
    sys.path.insert(0, str(REF_ROOT / "convert"))
    import q4k  # noqa: E402  (reference port, read-only)
    import q6k  # noqa: E402
    x = rows()
    b4 = np.asarray(q4k.quantize_q4_k(x), dtype=np.uint8)
    b6 = np.asarray(q6k._quantize_q6_k_numpy(x.reshape(-1, 256)), dtype=np.uint8)
    np.savez_compressed(HERE / "quant_blocks.npz", x=x, q4k=b4, q6k=b6)
    print("wrote", HERE / "quant_blocks.npz", x.shape, b4.shape, b6.shape)


if __name__ == "__main__":
    main()
