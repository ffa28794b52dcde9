"""The oracle's 32-value block formats (Q4_0, Q5_0, Q8_0) and F16 products,
pinned without the oracle's own formulas.

The reference's converters write these expert tables by default (Q8_0:
convert/convert_hf_to_gguf.py:55-57, convert/convert_qwen3omni.py:60-61,135;
Q5_0: convert/convert_nemotronomni.py:113-114; F16 and Q4_0:
convert/convert_diffusiongemma.py:62), through gguf-py (`gguf>=0.10`,
convert/requirements.txt:9; not installed here) whose block layouts are
ggml's.  What pins each part:
  * layouts: blocks with known codes (every code position distinct) decode
    to the values the format defines, read by numpy structured dtypes: a
    swapped nibble half, a wrong 5th-bit order or offset fails;
  * quantizers: the invariants the format fixes (the largest-magnitude value
    of a block decodes to itself up to the fp16 rounding of d; every value
    within half a step plus d's rounding; an all-zero block is all zero;
    codes stay in range) and a brute-force search on tiny blocks (no code
    of the block's scale is closer);
  * dots: fp64 sums of the decoded integer codes times the fp16 scales (the
    integer part exact), against the oracle's fp32 block accumulation;
  * mul_mat_id: each (row, token) entry against quantize + dot of that row,
    and the exact mode against numpy fp64 on the dequantized weights.
"""
import math

import numpy as np
import pytest

import pyoracle as O

Q8_0 = np.dtype([("d", "<f2"), ("qs", "i1", 32)])
Q4_0 = np.dtype([("d", "<f2"), ("qs", "u1", 16)])
Q5_0 = np.dtype([("d", "<f2"), ("qh", "<u4"), ("qs", "u1", 16)])
assert Q8_0.itemsize == 34 and Q4_0.itemsize == 18 and Q5_0.itemsize == 22


def codes(type_, raw):
    """(d [nb], signed codes [nb, 32]) of the blocks in raw (uint8 bytes)"""
    if type_ == O.TYPE_Q8_0:
        b = np.frombuffer(raw.tobytes(), Q8_0)
        return b["d"].astype(np.float64), b["qs"].astype(np.int64)
    if type_ == O.TYPE_Q4_0:
        b = np.frombuffer(raw.tobytes(), Q4_0)
        q = np.concatenate([b["qs"] & 15, b["qs"] >> 4], axis=1).astype(np.int64)
        return b["d"].astype(np.float64), q - 8
    b = np.frombuffer(raw.tobytes(), Q5_0)
    lo = np.concatenate([b["qs"] & 15, b["qs"] >> 4], axis=1).astype(np.int64)
    hi = (b["qh"][:, None] >> np.arange(32, dtype=np.uint32)[None, :]) & 1
    return b["d"].astype(np.float64), lo + 16 * hi.astype(np.int64) - 16


def test_block_sizes():
    for t, size in ((O.TYPE_Q4_0, 18), (O.TYPE_Q5_0, 22), (O.TYPE_Q8_0, 34)):
        assert O.BLOCK_BYTES[t] == size
        assert O.row_size(t, 64) == 2 * size
    assert O.row_size(O.TYPE_F16, 704) == 1408


@pytest.mark.parametrize("type_", O.B32_TYPES)
def test_layout_known_codes(type_):
    """value j of a block carries a code that names j"""
    d = np.float16(0.375)
    if type_ == O.TYPE_Q8_0:
        blk = np.zeros(1, Q8_0)
        blk["d"], blk["qs"][0] = d, np.arange(32) * 4 - 64          # value j -> 4j - 64
        want = (np.arange(32) * 4 - 64) * 0.375
    elif type_ == O.TYPE_Q4_0:
        blk = np.zeros(1, Q4_0)
        lo, hi = np.arange(16), 15 - np.arange(16)                  # value j: j, value 16+j: 15-j
        blk["d"], blk["qs"][0] = d, lo | (hi << 4)
        want = np.concatenate([lo - 8, hi - 8]) * 0.375
    else:
        blk = np.zeros(1, Q5_0)
        q = (np.arange(32) * 7) % 32                                # 32 distinct 5-bit codes
        blk["d"], blk["qs"][0] = d, (q[:16] & 15) | ((q[16:] & 15) << 4)
        blk["qh"] = int(sum(int(q[j] >> 4) << j for j in range(32)))
        want = (q - 16) * 0.375
    raw = np.frombuffer(blk.tobytes(), np.uint8)
    got = O.dequantize(type_, raw, 32)
    assert np.array_equal(got, want.astype(np.float32))


@pytest.mark.parametrize("type_", O.B32_TYPES)
def test_quantizer_invariants(type_):
    rng = np.random.default_rng(type_)
    x = (rng.standard_normal((300, 64)) * rng.uniform(0.01, 10, (300, 1))).astype(np.float32)
    x[0] = 0.0                                                      # all-zero blocks
    x[1, :32] = 1.0                                                 # a constant block
    raw = O.quantize(type_, x)
    assert raw.shape == (300, O.row_size(type_, 64))
    d, q = codes(type_, raw.reshape(-1))
    xb = x.reshape(-1, 32).astype(np.float64)
    rng_q = {O.TYPE_Q8_0: (-127, 127), O.TYPE_Q4_0: (-8, 7), O.TYPE_Q5_0: (-16, 15)}[type_]
    assert q.min() >= rng_q[0] and q.max() <= rng_q[1]
    dq = O.dequantize(type_, raw.reshape(-1), 300 * 64).reshape(-1, 32).astype(np.float64)
    assert np.array_equal(dq, d[:, None] * q)                       # decode = the codes times d
    assert not dq[0].any() and not dq[1].any()                      # zero blocks -> zero
    assert np.allclose(dq[2], 1.0, rtol=1e-3)                       # constant block: every value is the max
    # largest-magnitude value: decodes to itself up to d's fp16 rounding
    j = np.abs(xb).argmax(axis=1)
    big = xb[np.arange(len(xb)), j]
    live = np.abs(big) > 0
    assert np.all(np.abs(dq[np.arange(len(xb)), j] - big)[live] <= 1e-3 * np.abs(big[live]))
    # every value within half a step plus the step's fp16 rounding times the
    # code; Q4_0 / Q5_0 (d = max / -8, -16) clamp the far end of the other
    # sign at the top code: there within a whole step
    step = np.abs(d)[:, None]
    half = np.where(q == rng_q[1], 1.0, 0.5) if type_ != O.TYPE_Q8_0 else 0.5
    assert np.all(np.abs(dq - xb) <= half * step * (1 + 1e-6) + np.abs(q) * step * 2.0 ** -11 + 1e-30)


@pytest.mark.parametrize("type_", O.B32_TYPES)
def test_quantizer_brute_force_codes(type_):
    """Given the block's scale, no other code in range is nearer any value by
    more than the stored scale's fp16 rounding times the code (the codes are
    chosen against the fp32 scale, ggml stores it as fp16): the codes are the
    rounding of x / d, not a shifted or mirrored one."""
    rng = np.random.default_rng(100 + type_)
    x = rng.standard_normal((50, 32)).astype(np.float32)
    raw = O.quantize(type_, x)
    d, q = codes(type_, raw.reshape(-1))
    lo, hi = {O.TYPE_Q8_0: (-127, 127), O.TYPE_Q4_0: (-8, 7), O.TYPE_Q5_0: (-16, 15)}[type_]
    cand = np.arange(lo, hi + 1)[None, None, :] * d[:, None, None]
    best = np.abs(cand - x[:, :, None]).min(axis=2)
    mine = np.abs(q * d[:, None] - x)
    assert np.all(mine <= best + np.abs(q * d[:, None]) * 2.0 ** -10 + 1e-30)


@pytest.mark.parametrize("type_", O.B32_TYPES)
def test_vec_dot_closed_form(type_):
    rng = np.random.default_rng(200 + type_)
    k = 704                                                         # 22 blocks (diffusiongemma's expert width)
    w = O.quantize(type_, rng.standard_normal(k).astype(np.float32))
    a = O.quantize(O.TYPE_Q8_0, (rng.standard_normal(k) * 3).astype(np.float32))
    dw, qw = codes(type_, w)
    da, qa = codes(O.TYPE_Q8_0, a)
    exact = float(np.sum(dw * da * (qw * qa).sum(axis=1)))
    got = O.vec_dot(type_, w, a, k)
    assert abs(got - exact) <= 4e-6 * np.sum(np.abs(dw * da * (qw * qa).sum(axis=1))) + 1e-30


def test_vec_dot_f16():
    rng = np.random.default_rng(7)
    k = 2816
    a = rng.standard_normal(k).astype(np.float16)
    b = rng.standard_normal(k).astype(np.float16)
    exact = math.fsum((a.astype(np.float64) * b.astype(np.float64)).tolist())
    got = O.vec_dot(O.TYPE_F16, a.view(np.uint16), b.view(np.uint16), k)
    assert got == np.float32(exact)                                 # exact products, one rounding


@pytest.mark.parametrize("type_", list(O.B32_TYPES) + [O.TYPE_F16])
@pytest.mark.parametrize("ne11", [1, 3])
def test_mul_mat_id_new_types(type_, ne11):
    rng = np.random.default_rng(300 + type_ + ne11)
    E, N, Kin, T, K = 5, 12, 96, 7, 3
    wf = (rng.standard_normal((E, N, Kin)) * 0.1).astype(np.float32)
    wq = O.quantize(type_, wf.reshape(-1, Kin)) if type_ != O.TYPE_F16 else \
        wf.astype(np.float16).view(np.uint8).reshape(E * N, -1)
    b = rng.standard_normal((T, ne11, Kin)).astype(np.float32)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    got = O.mul_mat_id(type_, wq, Kin, N, E, b, ids)
    rows = wq.reshape(E, N, -1)
    for t in range(T):
        for k in range(K):
            brow = b[t, k % ne11]
            if type_ == O.TYPE_F16:
                act = brow.astype(np.float16).view(np.uint16)
            else:
                act = O.quantize(O.TYPE_Q8_0, brow)
            for n in range(N):
                assert got[t, k, n] == np.float32(O.vec_dot(type_, rows[ids[t, k], n], act, Kin))
    ex = O.mul_mat_id(type_, wq, Kin, N, E, b, ids, exact=True)
    deq = O.dequantize(type_, wq.reshape(-1), E * N * Kin).reshape(E, N, Kin).astype(np.float64)
    for t in range(T):
        for k in range(K):
            ref = deq[ids[t, k]] @ b[t, k % ne11].astype(np.float64)
            assert np.allclose(ex[t, k], ref, rtol=1e-6, atol=1e-7)
    # ggml semantics stay near the exact product: activation rounding only
    rel = np.linalg.norm(got - ex) / np.linalg.norm(ex)
    assert rel < (1e-2 if type_ != O.TYPE_F16 else 1e-3), rel
