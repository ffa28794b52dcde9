"""Pins the oracle's format layer: fp16, nearest_int, Q4_K / Q6_K / Q8_K
(de)quantization and the k-quant x Q8_K dot products.

Independent checks (not restatements of the oracle's code):
  - fp16 <-> fp32 against numpy's IEEE conversions, exhaustively;
  - nearest_int against numpy's round-half-to-even;
  - dequantizers against vectorized numpy unpacking written from the block
    layouts (convert/q4k.py:9-10,93-126; scripts/test_q6k.py:41-62) on random
    bytes, i.e. every code / scale combination;
  - quantizer outputs against the mathematical definition of their last step
    (every stored code is the nearest code for the stored scales) and the
    round-trip bound of scripts/test_q6k.py:77-86 on its edge-case blocks
    (scripts/test_q6k.py:27-38);
  - dot products against fp64 sums of the dequantized operands.
"""
import numpy as np
import pytest

import pyoracle as O


# ------------------------------------------------------------------ scalars
def test_fp16_to_fp32_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([O.fp16_to_fp32(int(v)) for v in h], dtype=np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))
    assert np.array_equal(got[np.isinf(ref)], ref[np.isinf(ref)])


def test_fp32_to_fp16_round_to_nearest_even():
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 5, 20000),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e6, -1e6, 2 ** -24, 2 ** -25, 2 ** -26,
                  3 * 2 ** -26, 5.960464477539063e-08, 6.097555160522461e-05, 1.0 + 2 ** -11,
                  1.0 + 3 * 2 ** -11, 2049.0, 2051.0], dtype=np.float32),
        # exact halfway points between fp16 neighbours
        (np.arange(1, 2048, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10),
    ]).astype(np.float32)
    ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([O.fp32_to_fp16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, ref)


def test_nearest_int_is_round_half_even():
    vals = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 0.49999997, 3.4999998, 1e6 + 0.5,
                     -4194303.0, 4194303.0, 7.5, 8.5, -7.5, 126.5, 127.5], dtype=np.float32)
    rng = np.random.default_rng(2)
    vals = np.concatenate([vals, (rng.standard_normal(5000) * 300).astype(np.float32)])
    got = np.array([O.nearest_int(float(v)) for v in vals])
    assert np.array_equal(got, np.rint(vals).astype(np.int64))


# ------------------------------------------------------------------ layouts
def np_dequant_q4k(blocks: np.ndarray) -> np.ndarray:
    """Q4_K from its byte layout: d f16 | dmin f16 | scales[12] | qs[128]."""
    nb = blocks.shape[0]
    d = np.ascontiguousarray(blocks[:, 0:2]).view(np.float16).astype(np.float32)[:, 0]
    dmin = np.ascontiguousarray(blocks[:, 2:4]).view(np.float16).astype(np.float32)[:, 0]
    s = blocks[:, 4:16].astype(np.int32)
    sc = np.zeros((nb, 8), np.int32)
    mn = np.zeros((nb, 8), np.int32)
    sc[:, :4] = s[:, 0:4] & 63
    mn[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    qs = blocks[:, 16:144].reshape(nb, 4, 32).astype(np.int32)
    q = np.zeros((nb, 256), np.int32)
    for c in range(4):
        q[:, 64 * c:64 * c + 32] = qs[:, c] & 0xF
        q[:, 64 * c + 32:64 * c + 64] = qs[:, c] >> 4
    sub = np.arange(256) // 32
    d1 = (d[:, None] * sc.astype(np.float32))[:, sub]
    m1 = (dmin[:, None] * mn.astype(np.float32))[:, sub]
    return (d1 * q.astype(np.float32) - m1).astype(np.float32)


def np_dequant_q6k(blocks: np.ndarray) -> np.ndarray:
    """Q6_K from its byte layout: ql[128] | qh[64] | scales[16] i8 | d f16."""
    nb = blocks.shape[0]
    ql = blocks[:, 0:128].astype(np.int32)
    qh = blocks[:, 128:192].astype(np.int32)
    sc = blocks[:, 192:208].view(np.int8).astype(np.int32)
    d = np.ascontiguousarray(blocks[:, 208:210]).view(np.float16).astype(np.float32)[:, 0]
    q = np.zeros((nb, 256), np.int32)
    for h in range(2):
        l = np.arange(32)
        lo_a, lo_b = ql[:, 64 * h + l], ql[:, 64 * h + 32 + l]
        hh = qh[:, 32 * h + l]
        q[:, 128 * h + l] = (lo_a & 0xF) | ((hh & 3) << 4)
        q[:, 128 * h + 32 + l] = (lo_b & 0xF) | (((hh >> 2) & 3) << 4)
        q[:, 128 * h + 64 + l] = (lo_a >> 4) | (((hh >> 4) & 3) << 4)
        q[:, 128 * h + 96 + l] = (lo_b >> 4) | (((hh >> 6) & 3) << 4)
    sidx = np.arange(256) // 16
    return ((d[:, None] * sc[:, sidx].astype(np.float32)) * (q - 32).astype(np.float32)).astype(np.float32)


def random_blocks(type_, n, seed):
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, size=(n, O.BLOCK_BYTES[type_]), dtype=np.uint8)
    # keep fp16 scales finite and moderate
    if type_ == O.TYPE_Q4_K:
        b[:, 0:2] = np.float16(rng.uniform(1e-4, 1e-2, n)).view(np.uint8).reshape(n, 2) if False else \
            rng.uniform(1e-4, 1e-2, n).astype(np.float16).view(np.uint8).reshape(n, 2)
        b[:, 2:4] = rng.uniform(1e-4, 1e-2, n).astype(np.float16).view(np.uint8).reshape(n, 2)
    else:
        b[:, 208:210] = rng.uniform(1e-4, 1e-2, n).astype(np.float16).view(np.uint8).reshape(n, 2)
    return b


@pytest.mark.parametrize("type_,ref", [(O.TYPE_Q4_K, np_dequant_q4k), (O.TYPE_Q6_K, np_dequant_q6k)])
def test_dequant_matches_layout(type_, ref):
    blocks = random_blocks(type_, 512, 3)
    got = O.dequantize(type_, blocks, 256)
    assert np.array_equal(got.view(np.uint32), ref(blocks).view(np.uint32))


# ------------------------------------------------------------------ quantizers
def edge_rows(n_rand, seed=0):
    """scripts/test_q6k.py:27-38 edge cases (zeros, below GROUP_MAX_EPS, x1e4,
    constant, mixed magnitudes) plus random rows."""
    rng = np.random.RandomState(seed)
    return np.concatenate([
        rng.randn(n_rand, 256).astype(np.float32),
        np.zeros((1, 256), np.float32),
        rng.choice([-1e-18, 1e-18], 256).astype(np.float32)[None],
        (rng.randn(1, 256) * 1e4).astype(np.float32),
        np.full((1, 256), 3.25, np.float32),
        (rng.randn(4, 256) * rng.choice([0.01, 1.0, 100.0], (4, 1))).astype(np.float32),
        (rng.randn(8, 256) * 0.02).astype(np.float32),
        np.abs(rng.randn(2, 256)).astype(np.float32),          # all positive (min > 0 path)
        -np.abs(rng.randn(2, 256)).astype(np.float32),
    ])


def test_q6k_round_trip_bound_and_layout():
    rows = edge_rows(64)
    pack = O.quantize(O.TYPE_Q6_K, rows)
    assert pack.shape == (rows.shape[0], 210)
    deq = O.dequantize(O.TYPE_Q6_K, pack, 256)
    scale = np.abs(rows).max(axis=1)
    nz = scale > 1e-12
    rel = np.abs(deq[nz] - rows[nz]).max(axis=1) / scale[nz]
    assert rel.max() <= 0.02        # scripts/test_q6k.py:80
    # sub-GROUP_MAX_EPS and zero blocks quantize to all-zero bytes
    assert not pack[64:66].any()


def test_q6k_codes_are_nearest_for_stored_scales():
    rows = edge_rows(64, seed=5)
    pack = O.quantize(O.TYPE_Q6_K, rows)
    d = np.ascontiguousarray(pack[:, 208:210]).view(np.float16).astype(np.float32)[:, 0]
    sc = pack[:, 192:208].view(np.int8).astype(np.float32)
    q = np.rint(np_dequant_q6k(pack) / np.where(
        (d[:, None] * sc)[:, np.arange(256) // 16] == 0, 1, (d[:, None] * sc)[:, np.arange(256) // 16]))
    ds = (d[:, None] * sc).astype(np.float32)[:, np.arange(256) // 16]
    ok = ds != 0
    want = np.clip(np.rint(rows / np.where(ok, ds, 1)).astype(np.int64), -32, 31)
    assert np.array_equal(q[ok].astype(np.int64), want[ok])


def test_q4k_round_trip_and_codes():
    rows = np.concatenate([edge_rows(64, seed=7)[:-2]])   # Q4_K is not sign-symmetric: skip the all-negative rows
    pack = O.quantize(O.TYPE_Q4_K, rows)
    assert pack.shape == (rows.shape[0], 144)
    deq = O.dequantize(O.TYPE_Q4_K, pack, 256)
    rng_ = rows.max(axis=1) - np.minimum(rows.min(axis=1), 0)
    nz = rng_ > 1e-12
    rel = np.abs(deq[nz] - rows[nz]).max(axis=1) / rng_[nz]
    # 4-bit codes over the sub-block range with 6-bit scales: half a step of
    # range/15 plus scale rounding stays under 1/15
    assert rel.max() < 1.0 / 15
    # every code is the nearest one for the stored (d*sc, dmin*m)
    d = np.ascontiguousarray(pack[:, 0:2]).view(np.float16).astype(np.float32)[:, 0]
    dmin = np.ascontiguousarray(pack[:, 2:4]).view(np.float16).astype(np.float32)[:, 0]
    s = pack[:, 4:16].astype(np.int32)
    sc = np.concatenate([s[:, 0:4] & 63, (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)], axis=1)
    mn = np.concatenate([s[:, 4:8] & 63, (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)], axis=1)
    sub = np.arange(256) // 32
    dd = (d[:, None] * sc.astype(np.float32))[:, sub]
    dm = (dmin[:, None] * mn.astype(np.float32))[:, sub]
    ok = dd != 0
    want = np.clip(np.rint((rows + dm) / np.where(ok, dd, 1)), 0, 15)
    got = np.rint((deq + dm) / np.where(ok, dd, 1))
    assert np.array_equal(got[ok], want[ok])


def test_q8k_definition():
    rng = np.random.default_rng(9)
    rows = np.concatenate([rng.standard_normal((16, 256)).astype(np.float32),
                           np.zeros((1, 256), np.float32),
                           np.full((1, 256), -2.0, np.float32)])
    rows[3, 17] = 5.0
    rows[3, 200] = -5.0          # tie in |x|: the first one sets the sign
    pack = O.quantize(O.TYPE_Q8_K, rows)
    assert pack.shape == (rows.shape[0], 292)
    d = pack[:, 0:4].copy().view(np.float32)[:, 0]
    qs = pack[:, 4:260].view(np.int8).astype(np.int32)
    bs = pack[:, 260:292].copy().view(np.int16).astype(np.int32)
    for r in range(rows.shape[0]):
        x = rows[r]
        amax_i = int(np.argmax(np.abs(x)))           # first index of the max |x|
        if np.abs(x).max() == 0:
            assert d[r] == 0 and not qs[r].any()
            continue
        iscale = np.float32(-127.0) / x[amax_i]
        want = np.minimum(127, np.rint((iscale * x).astype(np.float32))).astype(np.int32)
        assert np.array_equal(qs[r], want)
        assert d[r] == np.float32(1.0) / iscale
        assert np.array_equal(bs[r], qs[r].reshape(16, 16).sum(axis=1))
    assert qs[3, 17] == -127 and qs[3, 200] == 127


@pytest.mark.parametrize("type_", [O.TYPE_Q4_K, O.TYPE_Q6_K])
def test_vec_dot_equals_dequantized_dot(type_):
    rng = np.random.default_rng(11)
    k = 2048
    w = (rng.standard_normal((32, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((32, k)).astype(np.float32)
    wq = O.quantize(type_, w)
    xq = O.quantize(O.TYPE_Q8_K, x)
    wd = O.dequantize(type_, wq, k).astype(np.float64)
    xd = O.dequantize(O.TYPE_Q8_K, xq, k).astype(np.float64)
    for r in range(32):
        got = O.vec_dot(type_, wq[r], xq[r], k)
        ref = float(wd[r] @ xd[r])
        assert abs(got - ref) <= 2e-6 * (np.abs(wd[r] * xd[r]).sum() + 1e-30), (r, got, ref)


# ------------------------------------------------------------------ RNG
def test_rng_is_counter_based_and_normal():
    a = O.fill_normal(10001, 123, 4)
    b = O.fill_normal(4000, 123, 4)
    assert np.array_equal(a[:4000].view(np.uint32), b.view(np.uint32))
    c = O.fill_normal(10001, 123, 5)
    assert not np.array_equal(a, c)
    z = O.fill_normal(1 << 21, 7, 1)
    assert abs(z.mean()) < 3e-3 and abs(z.std() - 1.0) < 3e-3
    # tails of N(0,1): P(|z| > 3) = 0.0027
    assert abs((np.abs(z) > 3).mean() - 0.0027) < 4e-4
    s = O.fill_normal(1 << 16, 7, 2, mean=1.5, std=0.02)
    assert abs(s.mean() - 1.5) < 1e-3 and abs(s.std() - 0.02) < 1e-3


def test_poly_log_sincos_accuracy():
    import math
    xs = np.concatenate([np.geomspace(1e-300, 1.0, 2000), np.linspace(0.5, 1.0, 2000)])
    for v in xs:
        assert abs(O.poly_log(float(v)) - math.log(v)) <= 4e-16 * max(1.0, abs(math.log(v)))
    for u in np.linspace(0.0, 1.0, 4001, endpoint=False):
        s, c = O.poly_sincos_2pi(float(u))
        assert abs(s - math.sin(2 * math.pi * u)) < 2e-15
        assert abs(c - math.cos(2 * math.pi * u)) < 2e-15
