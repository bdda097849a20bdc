"""GPU parity at the benchmark's own shapes and statistics, through the C ABI.

* The large-shape stress GEMVs, K=8192->N=28672 and K=28672->N=8192, for every entry point the bench or
  a decoder uses on them (quantize + GEMV, pre-quantized, residual with bias, NORM + silu pair): bit-exact
  against the oracle's restatement of the kernel order, within rel 1e-5 / abs 1e-6 of the reference
  kernel's order and of the fp64 truth.
* Row counts at which every wave of the decode GEMV takes two or more row items, so the refill path of
  the long-row kernel (its carried step registers and hand-placed waits) and the double-buffered
  short-row kernel run in steady state.
* The M sweep on K=4096->N=14336 with p(0)=0.6, p(+-1)=0.2, lognormal(-4, 0.5) scales and Student-t(3)
  activations, M in {1, 2, 4, 8, 16, 32, 64, 128, 512, 2048}: every output row of the token GEMM
  bit-exact against the oracle's split order (from exact partials), and the pre-quantized GEMV for
  single tokens.
* The prefill shapes K=1024->N=4096 and K=4096->N=1024 with the bench's activations (N(0,1), 1% of the
  channels scaled x20), prompts of 32, 128 and 2048 tokens as one launch and as 32-token tiles: every
  output row bit-exact in each launch's own order.
* The secondary boundary ``TernaryLinear.forward`` (reference quantization.py:177-178) at M=1 and M=37.
"""

from __future__ import annotations

import numpy as np
import pytest

import ternary_oracle as T
from _util import (assert_bits_equal, assert_within, big_layer, device_matrix, finish_all_rows, reference_lanes,
                   to_np, token_gemm_order)

pytestmark = pytest.mark.gpu

STRESS = [(8192, 28672), (28672, 8192)]  # K -> N


def _t(array, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(array)).to(device)


_LAYERS: dict = {}


def _stress_layer(k: int, rows: int, bias: bool):
    """One cached host layer per shape (the draw of 235M codes takes a few seconds)."""
    key = (k, rows)
    if key not in _LAYERS:
        _LAYERS.clear()
        rng = np.random.default_rng(3 + k)
        _LAYERS[key] = big_layer(rng, rows, k, sigma=0.01, bias=True)
    codes, packed, scale_bits, b = _LAYERS[key]
    return codes, packed, scale_bits, (b if bias else None)


def _truth(oracle, q8, xsum, sx, packed, scale_bits, bias, k):
    rows = packed.shape[0]
    partials = oracle.group_partials(q8, xsum, packed, rows, k)
    return T.truth_fp64(partials, T.half_bits_to_float(scale_bits), sx, bias)


@pytest.mark.parametrize("k,rows", STRESS)
@pytest.mark.parametrize("entry", ["plain_store", "prequant_store", "plain_residual_bias", "norm_silu_pair"])
def test_stress_gemv_full_shape(cuda, oracle, k, rows, entry):
    import torch
    from ivonar_amd import ops, runtime

    print(f"stress gemv {entry} K={k} N={rows}", flush=True)
    bias = entry == "plain_residual_bias"
    codes, packed, scale_bits, b = _stress_layer(k, rows, bias)
    rng = np.random.default_rng(k + rows + len(entry))
    x = rng.standard_normal(k).astype(np.float32)
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    lanes, _ = runtime.gemv_plan(rows, k)
    xd = _t(x, cuda)
    if entry == "norm_silu_pair":
        weight = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
        out = torch.empty(rows // 2, dtype=torch.float32, device=cuda)
        ops.gemv(matrix, xd, out=out, mode="norm", epilogue="silu_pair", aux=_t(weight, cuda), eps=1e-6)
        q8, xsum, sx = oracle.quantize_rows(T.MODE_NORM, x, k, aux=weight, eps=1e-6)
        expected = oracle.gemv_pairs(T.EPI_SILU_PAIR, q8[0], xsum[0], sx[0], packed, scale_bits, None,
                                     np.zeros(rows // 2, np.float32), k, lanes)
        assert_bits_equal(to_np(out), expected, "silu pair vs oracle (kernel order)")
        ref = oracle.reforder(T.EPI_SILU_PAIR, False, q8, xsum, sx, packed, scale_bits, None,
                              np.zeros(rows // 2, np.float32), k, reference_lanes(k, rows, 16), rows // 2, 1)
        assert_within(to_np(out), ref, what="silu pair vs reference-kernel order")
        return
    q8, xsum, sx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    base = rng.standard_normal(rows).astype(np.float32)
    if entry == "plain_store":
        y = to_np(ops.gemv(matrix, xd))
        epi, start = T.EPI_STORE, np.zeros(rows, np.float32)
    elif entry == "prequant_store":
        y = to_np(ops.gemv_prequant(matrix, _t(q8, cuda), _t(xsum, cuda), _t(sx, cuda)))
        epi, start = T.EPI_STORE, np.zeros(rows, np.float32)
    else:
        out = _t(base, cuda)
        ops.gemv(matrix, xd, out=out, epilogue="residual")
        y = to_np(out)
        epi, start = T.EPI_RESIDUAL, base.copy()
    expected = oracle.gemv_pairs(epi, q8[0], xsum[0], sx[0], packed, scale_bits, b, start.copy(), k, lanes)
    assert_bits_equal(y, expected, f"{entry} vs oracle (kernel order)")
    ref = oracle.reforder(epi, False, q8, xsum, sx, packed, scale_bits, b, start.copy(), k,
                          reference_lanes(k, rows), rows, 1)
    assert_within(y, ref, what=f"{entry} vs reference-kernel order")
    truth = _truth(oracle, q8[0], xsum[0], sx[0], packed, scale_bits, b, k)
    if epi == T.EPI_RESIDUAL:
        truth = truth + base.astype(np.float64)
    assert_within(y, truth, what=f"{entry} vs fp64 truth")


# Every wave takes at least two row items: the long-row kernel (K 8193..32768, one row pair per wave per
# item, at most 2048 waves) at 12290 rows (6145 pairs, a ragged last pair) and on a K that is not a
# multiple of 4096 (clamped chunks); the short-row kernel (K=8192, two rows per wave per item, at most 4096
# waves) at 20000 rows.
@pytest.mark.parametrize("k,rows", [(28672, 12290), (8192, 20000), (20000, 9000)])
@pytest.mark.parametrize("epilogue", ["store", "residual_bias"])
def test_gemv_waves_take_several_items(cuda, oracle, k, rows, epilogue):
    from ivonar_amd import ops, runtime

    print(f"gemv several items K={k} N={rows} {epilogue}", flush=True)
    rng = np.random.default_rng(k * 3 + rows)
    bias = epilogue == "residual_bias"
    codes, packed, scale_bits, b = big_layer(rng, rows, k, sigma=0.01, bias=bias)
    x = rng.standard_normal(k).astype(np.float32)
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    lanes, _ = runtime.gemv_plan(rows, k)
    q8, xsum, sx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    if bias:
        base = rng.standard_normal(rows).astype(np.float32)
        out = _t(base, cuda)
        ops.gemv(matrix, _t(x, cuda), out=out, epilogue="residual")
        expected = oracle.gemv_pairs(T.EPI_RESIDUAL, q8[0], xsum[0], sx[0], packed, scale_bits, b, base.copy(), k,
                                     lanes)
        assert_bits_equal(to_np(out), expected, "residual")
    else:
        y = to_np(ops.gemv_prequant(matrix, _t(q8, cuda), _t(xsum, cuda), _t(sx, cuda)))
        expected = oracle.gemv_pairs(T.EPI_STORE, q8[0], xsum[0], sx[0], packed, scale_bits, None,
                                     np.zeros(rows, np.float32), k, lanes)
        assert_bits_equal(y, expected, "prequant store")


_SWEEP: dict = {}


def _sweep():
    if not _SWEEP:
        from ivonar_amd import synthetic

        k, rows = synthetic.SWEEP_SHAPE
        rng = np.random.default_rng(4)
        codes, packed, scale_bits, _ = big_layer(rng, rows, k, p=(0.2, 0.6, 0.2), scale="lognormal", mu=-4.0,
                                                 sigma=0.5)
        x = synthetic.student_t(rng, (max(synthetic.SWEEP_M), k))
        _SWEEP.update(k=k, rows=rows, codes=codes, packed=packed, scale_bits=scale_bits, x=x)
    return _SWEEP


@pytest.mark.parametrize("m", [1, 2, 4, 8, 16, 32, 64, 128, 256, 512, 2048])
def test_m_sweep_every_row(cuda, oracle, m):
    """K=4096->N=14336 with the sweep's statistics; every output row of every token bit-exact.

    M=1 runs the decode GEMV on the pre-quantized row, M=256 the 64-token long-prompt tiles (the
    128-token grid has 112 blocks), M=512 and 2048 the 128-token tiles, M=128 the split-K kernel."""
    from ivonar_amd import ops, runtime

    print(f"m sweep m={m}", flush=True)
    s = _sweep()
    k, rows, codes, packed, scale_bits = s["k"], s["rows"], s["codes"], s["packed"], s["scale_bits"]
    x = np.ascontiguousarray(s["x"][:m])
    assert np.abs(x).max() > 10 * np.abs(x).std()  # heavy tails: the absmax is set by outliers
    matrix = device_matrix(packed, scale_bits, k, device=cuda)
    dq8, dxsum, dsx = ops.quantize_rows(_t(x, cuda))
    q8, xsum, sx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    assert_bits_equal(to_np(dq8), q8, "q8")
    assert_bits_equal(to_np(dsx), sx, "token scales")
    y = to_np(ops.gemm(matrix, dq8, dxsum, dsx))
    splits = runtime.gemm_plan(m, rows, k)
    if m in (256, 512, 2048):
        assert splits == 1, "long-prompt tiles (one fmaf chain per output)"
    if m == 128:
        assert splits == 4, "split-K kernel"
    if m == 1:
        assert splits == 0, "one token runs the decode GEMV"
    order, param = token_gemm_order(m, rows, k)
    q = T.q8_linear(q8, k)
    expected = finish_all_rows(oracle, order, param, T.EPI_STORE, codes, q, scale_bits, sx, None,
                               np.zeros((m, rows), np.float32), k, rows)
    assert_bits_equal(y, expected, f"gemm m={m} (order {order}, {param}), every row")
    truth = T.truth_fp64(oracle.group_partials(q8[0], xsum[0], packed, rows, k), T.half_bits_to_float(scale_bits),
                         sx[0])
    assert_within(y[0], truth, what="token 0 vs fp64 truth")
    if m <= 2:
        lanes, _ = runtime.gemv_plan(rows, k)
        for t in range(m):
            g = to_np(ops.gemv_prequant(matrix, dq8[t:t + 1], dxsum[t:t + 1], dsx[t:t + 1]))
            exp = oracle.gemv_pairs(T.EPI_STORE, q8[t], xsum[t], sx[t], packed, scale_bits, None,
                                    np.zeros(rows, np.float32), k, lanes)
            assert_bits_equal(g, exp, f"gemv_prequant token {t}")


@pytest.mark.parametrize("m", [1, 37])
def test_ternary_linear_forward(cuda, oracle, m):
    """TernaryLinear.forward on the single-linear shape K=1024 -> N=4096 (with a bias)."""
    import torch
    from ivonar_amd import runtime
    from ivonar_amd.quantization import TernaryLinear

    rng = np.random.default_rng(100 + m)
    k, rows = 1024, 4096
    codes, packed, scale_bits, b = big_layer(rng, rows, k, bias=True)
    raw = np.ascontiguousarray(packed[:, : (k + 3) // 4])
    layer = TernaryLinear(torch.from_numpy(raw), torch.from_numpy(scale_bits.view(np.float16)), k,
                          bias=torch.from_numpy(b)).to(cuda)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = to_np(layer(_t(x, cuda).reshape(1, m, k))).reshape(m, rows)
    q8, xsum, sx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    if m == 1:
        lanes, _ = runtime.gemv_plan(rows, k)
        expected = oracle.gemv_pairs(T.EPI_STORE, q8[0], xsum[0], sx[0], packed, scale_bits, b,
                                     np.zeros(rows, np.float32), k, lanes)[None]
    else:
        expected = oracle.gemm_split(T.EPI_STORE, q8, xsum, sx, packed, scale_bits, b, np.zeros((m, rows), np.float32),
                                     k, rows, m, runtime.gemm_plan(m, rows, k))
    assert_bits_equal(y, expected, f"TernaryLinear.forward m={m}")
    for t in (0, m - 1):
        truth = T.truth_fp64(oracle.group_partials(q8[t], xsum[t], packed, rows, k), T.half_bits_to_float(scale_bits),
                             sx[t], b)
        assert_within(y[t], truth, what=f"token {t} vs fp64 truth")


@pytest.mark.parametrize("shape", [(1024, 4096), (4096, 1024)])
@pytest.mark.parametrize("length", [32, 128, 512, 2048])
def test_prefill_outlier_channels_every_row(cuda, oracle, shape, length):
    """Prompts with the bench's outlier channels, as one launch and as the reference's 32-token tiles."""
    import torch
    from ivonar_amd import ops, runtime, synthetic

    k, rows = shape
    print(f"prefill {k}->{rows} length={length}", flush=True)
    rng = np.random.default_rng(40 + length + k)
    codes, packed, scale_bits, _ = big_layer(rng, rows, k)
    x = synthetic.prefill_activations(rng, length, k)
    matrix = device_matrix(packed, scale_bits, k, device=cuda)
    dq8, dxsum, dsx = ops.quantize_rows(_t(x, cuda))
    q8, xsum, sx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    assert_bits_equal(to_np(dq8), q8, "q8")
    assert_bits_equal(to_np(dsx), sx, "token scales")
    q = T.q8_linear(q8, k)

    def expected(lo, hi):
        splits = runtime.gemm_plan(hi - lo, rows, k)
        return finish_all_rows(oracle, 1, splits, T.EPI_STORE, codes, q[lo:hi], scale_bits, sx[lo:hi], None,
                               np.zeros((hi - lo, rows), np.float32), k, rows)

    y = to_np(ops.gemm(matrix, dq8, dxsum, dsx))
    assert_bits_equal(y, expected(0, length), f"one launch of {length} tokens")
    tiles = torch.empty((length, rows), dtype=torch.float32, device=cuda)
    for lo in range(0, length, 32):
        ops.gemm(matrix, dq8[lo:lo + 32], dxsum[lo:lo + 32], dsx[lo:lo + 32], out=tiles[lo:lo + 32])
    tiled = to_np(tiles)
    for lo in range(0, length, 32):
        assert_bits_equal(tiled[lo:lo + 32], expected(lo, lo + 32), f"32-token tile at {lo}")
