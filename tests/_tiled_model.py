"""numpy models of the tiled table copies (mi_moe_tile), for the tests:
the Q4_K byte order and the Q6_K merged-code / fp16-scale image."""
import numpy as np


def np_tiled(src: np.ndarray) -> np.ndarray:
    """src: [E, N, row bytes] of Q4_K rows -> the tiled byte order"""
    E, N, rb = src.shape
    nb = rb // 144
    return src.reshape(E, N // 32, 32, nb, 144).transpose(0, 1, 3, 2, 4).reshape(E, N, rb)


def np_tiled_q6k(src: np.ndarray) -> np.ndarray:
    """src: [E, N, row bytes] of Q6_K rows -> [E, N / 32, blocks, 9216] bytes:
    code chunk 4 h + m, lane L (row L % 32, half g = L // 32): the 4 bytes of
    each of the codes q[k] (0..63) the GEMM takes for stage h, dword m, and
    the scale chunk's fp16 d * scale[8 h + 2 j + g] (+ 0)."""
    E, N, rb = src.shape
    nb = rb // 210
    blk = src.reshape(E, N // 32, 32, nb, 210)
    ql, qh, sc = blk[..., :128], blk[..., 128:192], blk[..., 192:208].view(np.int8)
    d = blk[..., 208:210].copy().view(np.float16)[..., 0].astype(np.float32)
    # the 256 codes of each block from its fields (ggml's dequantize_row_q6_K
    # order: value 128 n + 32 j' + l, l < 32, from ql[64 n + l (+32)] nibbles and
    # qh[32 n + l] bit pairs)
    codes = np.zeros(blk.shape[:-1] + (256,), np.uint8)
    for n in range(2):
        for l in range(32):
            a, b, h = ql[..., 64 * n + l], ql[..., 64 * n + 32 + l], qh[..., 32 * n + l]
            codes[..., 128 * n + l] = (a & 15) | (((h >> 0) & 3) << 4)
            codes[..., 128 * n + 32 + l] = (b & 15) | (((h >> 2) & 3) << 4)
            codes[..., 128 * n + 64 + l] = (a >> 4) | (((h >> 4) & 3) << 4)
            codes[..., 128 * n + 96 + l] = (b >> 4) | (((h >> 6) & 3) << 4)
    out = np.zeros((E, N // 32, nb, 9216), np.uint8)
    for L in range(64):
        r, g = L % 32, L // 32
        for h in range(2):
            for m in range(4):
                c = 4 * h + m
                for dw, (src_off, base) in enumerate([(64 * h + 16 * g + 4 * m, 0), (64 * h + 16 * g + 4 * m, 64),
                                                      (64 * h + 32 + 16 * g + 4 * m, 0),
                                                      (64 * h + 32 + 16 * g + 4 * m, 64)]):
                    # ql byte at src_off + i holds values (src_off + i) % 64 + 128 h (+ 64 for the
                    # high nibble) of the half h: positions 128 h + (src_off + i - 64 h) + base
                    for i in range(4):
                        pos = 128 * h + (src_off + i - 64 * h) + base
                        out[:, :, :, 1024 * c + 16 * L + 4 * dw + i] = codes[:, :, r, :, pos]
        for i in range(8):
            hh, j = i // 4, i % 4
            # (+ 0: a zero scale gives +0 for either sign of d, as on the GPU)
            v = (d[:, :, r, :] * sc[:, :, r, :, 8 * hh + 2 * j + g].astype(np.float32) + np.float32(0)).astype(np.float16)
            out[:, :, :, 8192 + 16 * L + 2 * i:8192 + 16 * L + 2 * i + 2] = v[..., None].view(np.uint8)
    return out
