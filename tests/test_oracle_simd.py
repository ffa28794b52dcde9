"""The AVX-512 VNNI forms of the oracle's Q4_K / Q6_K x Q8_K dots (the CPU
baseline's timed path) against the scalar generic forms, bit for bit: single
dots on random and extreme blocks, and whole layers through mul_mat_id.
Skipped where the host has no AVX-512 VNNI (then the baseline runs the scalar
form)."""
import numpy as np
import pytest

import pyoracle as O

pytestmark = pytest.mark.skipif(not O.host_has_avx512_vnni(), reason="host without AVX-512 VNNI")


def _rows(rng, n, k):
    x = rng.standard_normal((n, k)).astype(np.float32)
    x[0] = 0.0
    x[1] = 1e4 * np.sign(rng.standard_normal(k)).astype(np.float32)     # saturating codes
    x[2, ::7] = 50.0                                                     # outliers
    return x


@pytest.mark.parametrize("type_", [O.TYPE_Q4_K, O.TYPE_Q6_K])
def test_dot_bit_identical(type_):
    rng = np.random.default_rng(type_)
    k = 2048
    w = O.quantize(type_, _rows(rng, 64, k))
    a = O.quantize(O.TYPE_Q8_K, _rows(rng, 64, k) * 3)
    for i in range(64):
        for j in (i, (i * 7 + 3) % 64):
            s = O.vec_dot(type_, w[i], a[j], k)
            v = O.vec_dot_simd(type_, w[i], a[j], k)
            assert np.float32(s).view(np.uint32) == np.float32(v).view(np.uint32), (i, j, s, v)


@pytest.mark.parametrize("type_", [O.TYPE_Q4_K, O.TYPE_Q6_K])
def test_layer_products_bit_identical(type_):
    rng = np.random.default_rng(10 + type_)
    E, N, Kin, T, K = 6, 40, 512, 9, 2
    wq = O.quantize(type_, (rng.standard_normal((E * N, Kin)) * 0.02).astype(np.float32))
    b = rng.standard_normal((T, 1, Kin)).astype(np.float32)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    ref = O.mul_mat_id(type_, wq, Kin, N, E, b, ids)
    assert O.set_simd(True)
    try:
        got = O.mul_mat_id(type_, wq, Kin, N, E, b, ids)
    finally:
        O.set_simd(False)
    assert np.array_equal(ref.view(np.uint32), got.view(np.uint32))
