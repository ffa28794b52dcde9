"""The numpy model of the Q6_K tiled copy (tests/_tiled_model.py) against the
oracle's Q6_K dequantization (oracle/moe_oracle.c, ggml's
dequantize_row_q6_K): with d = 1 and nonzero integer scales every value is
scale * (code - 32) exactly, so each code the model places (lane, chunk,
byte) and each fp16 scale must be the one the oracle decodes.  The GPU tests
then hold the copy kernel to this model byte for byte."""
import numpy as np

import pyoracle as O
from _tiled_model import np_tiled, np_tiled_q6k


def test_q6k_model_codes_and_scales():
    rng = np.random.default_rng(11)
    E, N, nb = 1, 32, 2
    blk = rng.integers(0, 256, size=(E, N, nb, 210), dtype=np.uint8)
    sc = rng.integers(1, 120, size=(E, N, nb, 16)) * rng.choice([-1, 1], size=(E, N, nb, 16))
    blk[..., 192:208] = sc.astype(np.int8).view(np.uint8)
    blk[..., 208:210] = np.full(blk.shape[:-1] + (1,), 1.0, np.float16).view(np.uint8)
    src = blk.reshape(E, N, nb * 210)
    vals = O.dequantize(O.TYPE_Q6_K, src.reshape(E * N, nb * 210), nb * 256).reshape(E, N, nb, 256)
    # scale of value v: ggml's sub-block 8 (v // 128) + (v % 32) // 16 + 2 ((v % 128) // 32)
    v = np.arange(256)
    sub = 8 * (v // 128) + (v % 32) // 16 + 2 * ((v % 128) // 32)
    codes = np.rint(vals / sc[..., sub]).astype(np.int64) + 32
    assert codes.min() >= 0 and codes.max() <= 63
    assert np.array_equal(vals, (sc[..., sub] * (codes - 32)).astype(np.float32))
    img = np_tiled_q6k(src)   # [E, N / 32, nb, 9216]
    for L in range(64):
        r, g = L % 32, L // 32
        for h in range(2):
            for m in range(4):
                for dw in range(4):
                    for i in range(4):
                        l = 16 * g + 4 * m + i
                        pos = 128 * h + l + (32 if dw >= 2 else 0) + (64 if dw % 2 else 0)
                        got = img[0, 0, :, 1024 * (4 * h + m) + 16 * L + 4 * dw + i]
                        assert np.array_equal(got, codes[0, r, :, pos]), (L, h, m, dw, i)
        for k in range(8):
            hh, j = k // 4, k % 4
            half = img[0, 0, :, 8192 + 16 * L + 2 * k:8192 + 16 * L + 2 * k + 2].copy().view(np.float16)[:, 0]
            assert np.array_equal(half.astype(np.float32), sc[0, r, :, 8 * hh + 2 * j + g].astype(np.float32))


def test_q4k_model_is_a_permutation():
    rng = np.random.default_rng(12)
    src = rng.integers(0, 256, size=(2, 64, 4 * 144), dtype=np.uint8)
    t = np_tiled(src)
    # the group's bytes stay in the group's range; block b of row r at 4608 b + 144 r
    for e in range(2):
        for grp in range(2):
            flat = t[e, 32 * grp:32 * grp + 32].reshape(-1)
            for b in range(4):
                for r in range(32):
                    assert np.array_equal(flat[4608 * b + 144 * r:4608 * b + 144 * r + 144],
                                          src[e, 32 * grp + r, 144 * b:144 * b + 144])
