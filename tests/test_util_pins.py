"""Pins of the test helpers that stand in for the oracle at large sizes: the float32 matrix-product
partials equal the int64 brute force exactly, including the extreme magnitudes."""

from __future__ import annotations

import numpy as np

import ternary_oracle as T
from _util import exact_partials


def test_exact_partials_equal_the_int64_brute_force():
    rng = np.random.default_rng(11)
    for rows, k, m in [(5, 8, 1), (33, 300, 4), (64, 1024, 7)]:
        codes = rng.integers(0, 3, size=(rows, k), dtype=np.uint8)
        q = rng.integers(-127, 128, size=(m, k))
        got = exact_partials(codes, q)
        for t in range(m):
            assert np.array_equal(got[t].astype(np.int64), T.group_partials_int64(codes, q[t]))


def test_exact_partials_at_the_largest_group_sums():
    k = 384
    codes = np.zeros((3, k), dtype=np.uint8)
    codes[1] = 2
    codes[2, ::2] = 2
    q = np.full((2, k), 127)
    q[1] = -127
    got = exact_partials(codes, q)
    assert got[0, 0, 0] == -127 * 128 and got[0, 1, 0] == 127 * 128 and got[1, 1, 2] == -127 * 128
    for t in range(2):
        assert np.array_equal(got[t].astype(np.int64), T.group_partials_int64(codes, q[t]))


def test_every_row_finish_equals_the_oracle_gemm(oracle):
    """finish_all_rows (exact partials + orc_finish) gives orc_gemm_split's bits for every epilogue."""
    from _util import finish_all_rows, make_layer

    rng = np.random.default_rng(5)
    m, k, rows = 9, 1100, 40
    codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=True)
    x = rng.standard_normal((m, k)).astype(np.float32)
    q8, xsum, sx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    q = T.q8_linear(q8, k)
    for epi, width in [(T.EPI_STORE, rows), (T.EPI_RESIDUAL, rows), (T.EPI_SILU_PAIR, rows // 2)]:
        for splits in (1, 3, 8):
            stride = width + 2
            base = rng.standard_normal((m, stride)).astype(np.float32)
            got = finish_all_rows(oracle, 1, splits, epi, codes, q, scale_bits, sx, b, base.copy(), k, stride)
            want = oracle.gemm_split(epi, q8, xsum, sx, packed, scale_bits, b, base.copy(), k, stride, m, splits)
            assert np.array_equal(got, want), (epi, splits)
