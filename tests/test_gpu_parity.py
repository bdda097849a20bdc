"""GPU parity of the HIP ternary kernels against the CPU oracle, through the C ABI.

Integer work (q8, xsum, scales, per-128-group partials, embeddings) must be
bit-exact.  fp32 outputs must equal the oracle's restatement of the kernel's
own summation order bit for bit, and lie within rel 1e-5 / abs 1e-6 of both
the reference kernel's order and the fp64 truth.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

import ternary_oracle as T
from _util import (ATOL, RTOL, assert_bits_equal, assert_within, device_matrix, finish_all_rows, make_layer,
                   reference_lanes, to_np, token_gemm_expected, token_gemm_order)

pytestmark = pytest.mark.gpu

EDGE_K = [8, 16, 24, 32, 64, 96, 100, 256, 1024, 1100]


def _t(array, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(array)).to(device)


def _every_row(oracle, codes, x, k, scale_bits, bias, plan, epi=None, out=None, stride=None):
    """The token GEMM's expected output for every token and row, in the kernel's fp32 order: `plan` is
    the K-splits of the split order, or (order, param) as token_gemm_order gives them."""
    order, param = plan if isinstance(plan, tuple) else (1, plan)
    m, rows = x.shape[0], codes.shape[0]
    eq8, exsum, esx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    epi = T.EPI_STORE if epi is None else epi
    out = np.zeros((m, rows), np.float32) if out is None else out
    return finish_all_rows(oracle, order, param, epi, codes, T.q8_linear(eq8, k), scale_bits, esx, bias, out, k,
                           rows if stride is None else stride)


# ------------------------------------------------------------------ quantizer


def _edge_rows(n: int, rng) -> np.ndarray:
    rows = [
        rng.standard_normal(n).astype(np.float32),
        np.zeros(n, dtype=np.float32),                                      # s = 1e-5, q = 0
        (rng.standard_normal(n) * 1e-4).astype(np.float32),                 # amax < 1.27e-3: floor applies
        (rng.standard_normal(n) * 50).astype(np.float32),
    ]
    ties = np.zeros(n, dtype=np.float32)                                    # amax 127 -> s = 1: exact halves
    ties[: min(n, 8)] = np.float32([127.0, 2.5, -3.5, 0.5, -0.5, 1.5, -126.5, -0.0])[: min(n, 8)]
    rows.append(ties)
    return np.stack(rows)


@pytest.mark.parametrize("n", EDGE_K + [4096, 4097, 28672])
def test_quantize_plain_rows_bit_exact(cuda, oracle, n):
    from ivonar_amd import ops

    rng = np.random.default_rng(n)
    x = _edge_rows(n, rng)
    q8, xsum, scale = ops.quantize_rows(_t(x, cuda))
    eq8, exsum, escale = oracle.quantize_rows(T.MODE_PLAIN, x, n)
    assert_bits_equal(to_np(q8), eq8, "q8")
    assert_bits_equal(to_np(xsum), exsum, "xsum")
    assert_bits_equal(to_np(scale), escale, "scale")
    q, s = T.quantize_closed_form(x[0])
    assert s == escale[0]
    assert_bits_equal(eq8[0], T.q8_layout(q)[0], "oracle vs closed form")


@pytest.mark.parametrize("n", [16, 96, 1024, 1100, 4096, 8192])
def test_quantize_norm_bit_exact(cuda, oracle, n):
    from ivonar_amd import ops

    rng = np.random.default_rng(7 + n)
    x = (rng.standard_normal((3, n)) * np.float32(3.0)).astype(np.float32)
    x[2, ::7] *= 40.0  # rows whose normalised values reach the +-8 clip
    weight = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    q8, xsum, scale = ops.quantize_rows(_t(x, cuda), mode=ops.MODE_NORM, aux=_t(weight, cuda), eps=1e-6)
    eq8, exsum, escale = oracle.quantize_rows(T.MODE_NORM, x, n, aux=weight, eps=1e-6)
    assert_bits_equal(to_np(scale), escale, "scale")
    assert_bits_equal(to_np(q8), eq8, "q8")
    assert_bits_equal(to_np(xsum), exsum, "xsum")


@pytest.mark.parametrize("head_dim,heads,splits", [(4, 4, 3), (16, 4, 4), (64, 16, 4)])
def test_quantize_attn_bit_exact(cuda, oracle, head_dim, heads, splits):
    from ivonar_amd import ops, runtime

    rng = np.random.default_rng(head_dim * 31 + splits)
    check = runtime.library().ivonar_define(b"HEAD_DIM", head_dim)
    assert check == 0
    try:
        parts = rng.standard_normal((2, heads, splits, head_dim + 2)).astype(np.float32)
        parts[..., 1] = np.abs(parts[..., 1]) + 0.5
        parts[0, 0, 0, 0] = -np.inf  # an empty split
        n = heads * head_dim
        stride = heads * splits * (head_dim + 2)
        flat = parts.reshape(2, stride)
        q8, xsum, scale = ops.quantize_rows(_t(flat, cuda), mode=ops.MODE_ATTN, splits=splits, n=n)
        eq8, exsum, escale = oracle.quantize_rows(T.MODE_ATTN, flat, n, splits=splits, head_dim=head_dim, m=2,
                                                  in_stride=stride)
        assert_bits_equal(to_np(scale), escale, "scale")
        assert_bits_equal(to_np(q8), eq8, "q8")
        assert_bits_equal(to_np(xsum), exsum, "xsum")
    finally:
        runtime.library().ivonar_define(b"HEAD_DIM", 64)


# ------------------------------------------------------------ integer core


@pytest.mark.parametrize("rows,k", [(1, 8), (7, 16), (9, 24), (64, 96), (130, 100), (33, 1024), (64, 4096),
                                    (16, 8192), (8, 28672)])
def test_group_partials_bit_exact_against_brute_force(cuda, oracle, rows, k):
    from ivonar_amd import ops

    rng = np.random.default_rng(rows * 1000 + k)
    codes, packed, scale_bits, _ = make_layer(rng, rows, k)
    x = rng.standard_normal(k).astype(np.float32)
    q, _ = T.quantize_closed_form(x)
    q8, xsum = T.q8_layout(q)
    matrix = device_matrix(packed, scale_bits, k, device=cuda)
    got = to_np(ops.group_partials(matrix, _t(q8, cuda), _t(xsum, cuda)))
    expected = T.group_partials_int64(codes, q)
    assert np.abs(expected).max() <= 127 * 128
    assert_bits_equal(got.astype(np.int64), expected, "partials")
    assert_bits_equal(oracle.group_partials(q8, xsum, packed, rows, k).astype(np.int64), expected, "oracle partials")


# ------------------------------------------------------------------- GEMV


def _gemv_case(rng, rows, k, bias=False, p=(0.3, 0.4, 0.3)):
    codes, packed, scale_bits, b = make_layer(rng, rows, k, p=p, bias=bias)
    x = rng.standard_normal(k).astype(np.float32)
    return codes, packed, scale_bits, b, x


def _check_gemv_store(cuda, oracle, rows, k, bias):
    from ivonar_amd import ops, runtime

    rng = np.random.default_rng(rows + 17 * k + int(bias))
    codes, packed, scale_bits, b, x = _gemv_case(rng, rows, k, bias)
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    y = to_np(ops.gemv(matrix, _t(x, cuda)))
    q8, xsum, sx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    lanes, _ = runtime.gemv_plan(rows, k)
    mine = oracle.gemv_pairs(T.EPI_STORE, q8[0], xsum[0], sx[0], packed, scale_bits, b,
                             np.zeros(rows, np.float32), k, lanes)
    assert_bits_equal(y, mine, "gemv vs oracle (kernel order)")
    ref = oracle.reforder(T.EPI_STORE, False, q8, xsum, sx, packed, scale_bits, b, np.zeros(rows, np.float32), k,
                          reference_lanes(k, rows), rows, 1)
    assert_within(y, ref, what="gemv vs reference-kernel order")
    q, s = T.quantize_closed_form(x)
    truth = T.truth_fp64(T.group_partials_int64(codes, q), T.half_bits_to_float(scale_bits), s, b)
    assert_within(y, truth, what="gemv vs fp64 truth")


@pytest.mark.parametrize("k", EDGE_K)
@pytest.mark.parametrize("rows", [1, 6, 64, 257])
def test_gemv_plain_store_edge_shapes(cuda, oracle, rows, k):
    _check_gemv_store(cuda, oracle, rows, k, bias=rows == 6)


@pytest.mark.parametrize("rows,k", [(4096, 1024), (1024, 4096), (3072, 1024), (512, 8192), (256, 28672),
                                    (333, 5000), (64, 8193), (128, 12288), (96, 32768), (40, 32769)])
def test_gemv_plain_store_model_shapes(cuda, oracle, rows, k):
    _check_gemv_store(cuda, oracle, rows, k, bias=False)


@pytest.mark.parametrize("k", [24, 1024, 1102, 2048, 4096])
def test_fused_gemv_vector_and_scalar_row_loads(cuda, oracle, k):
    """Rows of up to 4096 inputs are quantized in the GEMV launch's prologue: a 16-byte aligned PLAIN row
    with K a multiple of 4 is read as float4, other rows one input per load (an input shifted by one
    float, and K=1102).  Both give the oracle's bits, for rows of 4, 8 and 16 inputs per thread."""
    import torch
    from ivonar_amd import ops, runtime

    print(f"fused gemv_plain_store row loads K={k}", flush=True)
    rows = 600
    rng = np.random.default_rng(k + 11)
    codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=False)
    matrix = device_matrix(packed, scale_bits, k, bias=None, device=cuda)
    lanes, _ = runtime.gemv_plan(rows, k)
    x = (rng.standard_normal(k) * 3.0).astype(np.float32)
    x[rng.integers(0, k)] = 40.0
    aligned = _t(x, cuda)
    shifted = torch.zeros(k + 1, dtype=torch.float32, device=cuda)
    shifted[1:] = aligned
    q8, xsum, sx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    expected = oracle.gemv_pairs(T.EPI_STORE, q8[0], xsum[0], sx[0], packed, scale_bits, None,
                                 np.zeros(rows, np.float32), k, lanes)
    assert_bits_equal(to_np(ops.gemv(matrix, aligned)), expected, "aligned input")
    assert_bits_equal(to_np(ops.gemv(matrix, shifted[1:])), expected, "input shifted by one float")


@pytest.mark.parametrize("k", [5000, 8192, 28672, 40000])
@pytest.mark.parametrize("rows", [2, 600])
def test_gemv_long_rows_back_to_back(cuda, oracle, rows, k):
    """Rows of 4097..32768 inputs are quantized inside the GEMV launch, by every block into its own LDS
    (40000 inputs: by the separate quantizer).  Eight calls with inputs of magnitudes 1e-3 .. 1e3 go
    out back to back on one stream (two rows: most blocks have no row and still quantize); each output
    must be the oracle's for its own input.  The same rows read from an input that is not 16-byte
    aligned take the separate quantizer launch and give the same bits."""
    import torch
    from ivonar_amd import ops, runtime

    print(f"back-to-back gemv_plain_store K={k} N={rows}", flush=True)
    rng = np.random.default_rng(rows + 3 * k)
    codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=True)
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    lanes, _ = runtime.gemv_plan(rows, k)
    calls = 8
    xs = (rng.standard_normal((calls, k)) * np.geomspace(1e-3, 1e3, calls)[:, None]).astype(np.float32)
    inputs = _t(xs, cuda)
    shifted = torch.zeros(calls * k + 1, dtype=torch.float32, device=cuda)
    shifted[1:] = inputs.reshape(-1)
    outs = torch.empty((2, calls, rows), dtype=torch.float32, device=cuda)
    torch.cuda.synchronize()
    for i in range(calls):
        ops.gemv(matrix, inputs[i], out=outs[0, i])
    for i in range(calls):
        ops.gemv(matrix, shifted[1 + i * k:1 + (i + 1) * k], out=outs[1, i])
    torch.cuda.synchronize()
    got = to_np(outs)
    for i in range(calls):
        q8, xsum, sx = oracle.quantize_rows(T.MODE_PLAIN, xs[i], k)
        mine = oracle.gemv_pairs(T.EPI_STORE, q8[0], xsum[0], sx[0], packed, scale_bits, b,
                                 np.zeros(rows, np.float32), k, lanes)
        assert_bits_equal(got[0, i], mine, f"aligned input, call {i}")
        assert_bits_equal(got[1, i], mine, f"unaligned input, call {i}")


# Rows the GEMV quantizes inside its own launch (16-byte aligned PLAIN rows of 4097..32768 inputs, and
# rows of up to 4096 inputs through the fused prologue), with the values both quantizers treat
# specially: their u = fma(x, 1/s, 128) rounding decides every value except those within 3e-5 of a
# half-integer, which take the exact division.
@pytest.mark.parametrize("k", [24, 1024, 1100, 4096, 4100, 8192, 12288, 28672, 32768])
def test_gemv_in_launch_quantizer_edge_rows(cuda, oracle, k):
    """Zero row (scale floor 1e-5, every q 0), a row below the floor, exact ties x/s = j + 1/2 (s a power
    of two, so x/s is exact and rint goes to even), values one float step either side of those ties, -0.0
    entries, and a single outlier over tiny values: every output the oracle's bits, and q8 from the
    separate quantizer fed to gemv_prequant_store gives the same bits."""
    from ivonar_amd import ops, runtime

    rows = 600
    print(f"in-launch quantizer edge rows K={k} N={rows}", flush=True)
    rng = np.random.default_rng(k + 5)
    codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=True)
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    lanes, _ = runtime.gemv_plan(rows, k)
    s = np.float32(0.125)  # amax = 127 * s makes the scale exactly s
    ties = (rng.integers(-126, 126, k) + np.float32(0.5)) * s
    ties[rng.integers(0, k)] = 127 * s
    near = ties.copy()
    near[0::2] = np.nextafter(near[0::2], np.float32(np.inf))
    near[1::2] = np.nextafter(near[1::2], np.float32(-np.inf))
    near[np.argmax(np.abs(ties))] = 127 * s
    signed_zero = rng.standard_normal(k).astype(np.float32)
    signed_zero[::3] = -0.0
    outlier = (rng.standard_normal(k) * 1e-6).astype(np.float32)
    outlier[k // 3] = 500.0
    cases = {"zeros": np.zeros(k, np.float32), "below floor": (rng.standard_normal(k) * 1e-4).astype(np.float32),
             "exact ties": ties.astype(np.float32), "next to ties": near.astype(np.float32),
             "signed zeros": signed_zero, "outlier": outlier}
    for name, x in cases.items():
        q8, xsum, sx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
        expected = oracle.gemv_pairs(T.EPI_STORE, q8[0], xsum[0], sx[0], packed, scale_bits, b,
                                     np.zeros(rows, np.float32), k, lanes)
        xd = _t(x, cuda)
        assert_bits_equal(to_np(ops.gemv(matrix, xd)), expected, f"{name}: gemv_plain_store")
        dq8, dxsum, dsx = ops.quantize_rows(xd[None])
        assert_bits_equal(to_np(dq8), q8, f"{name}: q8")
        assert_bits_equal(to_np(ops.gemv_prequant(matrix, dq8, dxsum, dsx)), expected, f"{name}: prequant")


@pytest.mark.parametrize("k", [24, 1024, 4096, 5000, 8192, 8200, 28672, 40000, 49152])
def test_gemv_residual_and_silu_pair(cuda, oracle, k):
    import torch
    from ivonar_amd import ops, runtime

    rng = np.random.default_rng(k + 5)
    rows = 64
    codes, packed, scale_bits, b, x = _gemv_case(rng, rows, k, bias=True)
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    q8, xsum, sx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    lanes, _ = runtime.gemv_plan(rows, k)
    base = rng.standard_normal(rows).astype(np.float32)
    out = _t(base, cuda)
    ops.gemv(matrix, _t(x, cuda), out=out, epilogue="residual")
    expected = oracle.gemv_pairs(T.EPI_RESIDUAL, q8[0], xsum[0], sx[0], packed, scale_bits, b, base.copy(), k, lanes)
    assert_bits_equal(to_np(out), expected, "residual")
    # silu pair on interleaved rows: output[j] = silu(row 2j) * row 2j+1
    weight = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    half = torch.empty(rows // 2, dtype=torch.float32, device=cuda)
    ops.gemv(matrix, _t(x, cuda), out=half, mode="norm", epilogue="silu_pair", aux=_t(weight, cuda), eps=1e-6)
    nq8, nxsum, nsx = oracle.quantize_rows(T.MODE_NORM, x, k, aux=weight, eps=1e-6)
    expected = oracle.gemv_pairs(T.EPI_SILU_PAIR, nq8[0], nxsum[0], nsx[0], packed, scale_bits, b,
                                 np.zeros(rows // 2, np.float32), k, lanes)
    assert_bits_equal(to_np(half), expected, "silu pair")
    ref = oracle.reforder(T.EPI_SILU_PAIR, False, nq8, nxsum, nsx, packed, scale_bits, b,
                          np.zeros(rows // 2, np.float32), k, reference_lanes(k, rows, 16), rows // 2, 1)
    assert_within(to_np(half), ref, rtol=1e-5, atol=1e-6, what="silu pair vs reference order")


@pytest.mark.parametrize("k", [96, 1024, 4100, 8192, 8193, 40000])
def test_gemv_norm_store_and_prequant(cuda, oracle, k):
    import torch
    from ivonar_amd import ops, runtime

    rng = np.random.default_rng(k + 11)
    rows = 200
    codes, packed, scale_bits, b, x = _gemv_case(rng, rows, k)
    weight = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    matrix = device_matrix(packed, scale_bits, k, device=cuda)
    y = to_np(ops.gemv(matrix, _t(x, cuda), mode="norm", aux=_t(weight, cuda), eps=1e-6))
    q8, xsum, sx = oracle.quantize_rows(T.MODE_NORM, x, k, aux=weight, eps=1e-6)
    lanes, _ = runtime.gemv_plan(rows, k)
    expected = oracle.gemv_pairs(T.EPI_STORE, q8[0], xsum[0], sx[0], packed, scale_bits, None,
                                 np.zeros(rows, np.float32), k, lanes)
    assert_bits_equal(y, expected, "norm store")
    # quantize_norm + gemv_prequant_store (the LM-head pair of launches)
    lib = runtime.library()
    dq8, dxsum, dscale = ops.activation_buffers(1, k, cuda)
    xin, win = _t(x, cuda), _t(weight, cuda)
    runtime.check(lib.quantize_norm(runtime.current_stream(cuda), runtime.pointer(xin), runtime.pointer(win),
                                    k, runtime.float32(1e-6), 1, runtime.pointer(dq8), runtime.pointer(dxsum),
                                    runtime.pointer(dscale)))
    assert_bits_equal(to_np(dq8), q8, "quantize_norm q8")
    head = to_np(ops.gemv_prequant(matrix, dq8, dxsum, dscale))
    assert_bits_equal(head, expected, "prequant")


@pytest.mark.parametrize("head_dim,heads,splits", [(4, 4, 4), (64, 16, 4), (64, 80, 2)])
def test_gemv_attn_residual(cuda, oracle, head_dim, heads, splits):
    from ivonar_amd import ops, runtime

    lib = runtime.library()
    assert lib.ivonar_define(b"HEAD_DIM", head_dim) == 0
    try:
        rng = np.random.default_rng(head_dim + splits)
        k = heads * head_dim
        rows = 48
        codes, packed, scale_bits, b, _ = _gemv_case(rng, rows, k, bias=True)
        parts = rng.standard_normal((heads, splits, head_dim + 2)).astype(np.float32)
        parts[..., 1] = np.abs(parts[..., 1]) + 0.5
        matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
        base = rng.standard_normal(rows).astype(np.float32)
        out = _t(base, cuda)
        ops.gemv(matrix, _t(parts.reshape(-1), cuda), out=out, mode="attn", epilogue="residual", splits=splits)
        q8, xsum, sx = oracle.quantize_rows(T.MODE_ATTN, parts.reshape(-1), k, splits=splits, head_dim=head_dim)
        lanes, _ = runtime.gemv_plan(rows, k)
        expected = oracle.gemv_pairs(T.EPI_RESIDUAL, q8[0], xsum[0], sx[0], packed, scale_bits, b, base.copy(), k,
                                     lanes)
        assert_bits_equal(to_np(out), expected, "attn residual")
    finally:
        lib.ivonar_define(b"HEAD_DIM", 64)


# ------------------------------------------------------------------- GEMM


@pytest.mark.parametrize("m", [1, 5, 16, 32, 33, 70])
@pytest.mark.parametrize("k,rows", [(24, 16), (96, 64), (1024, 256), (4096, 96), (1100, 48)])
def test_gemm_tile_store(cuda, oracle, m, k, rows):
    from ivonar_amd import ops, runtime

    rng = np.random.default_rng(m * 7919 + k + rows)
    codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=(m == 5))
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[:, :: max(1, k // 10)] *= 20.0
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    q8, xsum, sx = ops.quantize_rows(_t(x, cuda))
    y = to_np(ops.gemm(matrix, q8, xsum, sx))
    eq8, exsum, esx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    assert_bits_equal(to_np(q8), eq8, "tile q8")
    expected = token_gemm_expected(oracle, T.EPI_STORE, eq8, exsum, esx, packed, scale_bits, b,
                                   np.zeros((m, rows), np.float32), k, rows, m)
    assert_bits_equal(y, expected, f"gemm vs oracle (kernel order {token_gemm_order(m, rows, k)})")
    if m == 1:
        assert runtime.gemm_plan(m, rows, k) == 0, "one token runs the decode GEMV"
    ref = oracle.reforder(T.EPI_STORE, True, eq8, exsum, esx, packed, scale_bits, b, np.zeros((m, rows), np.float32),
                          k, reference_lanes(k, rows), rows, m)
    assert_within(y, ref, what="gemm vs reference-kernel order")


@pytest.mark.parametrize("epilogue", ["residual", "silu_pair"])
def test_gemm_tile_epilogues(cuda, oracle, epilogue):
    import torch
    from ivonar_amd import ops, runtime

    rng = np.random.default_rng(99 if epilogue == "residual" else 98)
    m, k, rows = 32, 1024, 128
    codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=True)
    x = rng.standard_normal((m, k)).astype(np.float32)
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    q8, xsum, sx = ops.quantize_rows(_t(x, cuda))
    eq8, exsum, esx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    width = rows if epilogue == "residual" else rows // 2
    stride = width + 3
    base = rng.standard_normal((m, stride)).astype(np.float32)
    out = _t(base, cuda)
    ops.gemm(matrix, q8, xsum, sx, out=out, epilogue=epilogue, out_stride=stride)
    epi = T.EPI_RESIDUAL if epilogue == "residual" else T.EPI_SILU_PAIR
    expected = oracle.gemm_split(epi, eq8, exsum, esx, packed, scale_bits, b, base.copy(), k, stride, m,
                                 runtime.gemm_plan(m, rows, k))
    assert_bits_equal(to_np(out), expected, epilogue)
    assert torch.equal(out[:, width:], _t(base[:, width:], cuda)), "the GEMM wrote past its output width"


# ------------------------------------------------------- embedding, argmax


def test_embed_gather_and_argmax(cuda, oracle):
    import torch
    from ivonar_amd import ops, runtime

    rng = np.random.default_rng(3)
    vocab, hidden = 300, 100
    codes, packed, scale_bits, _, _ = _gemv_case(rng, vocab, hidden)
    matrix = device_matrix(packed, scale_bits, hidden, device=cuda)
    tokens = np.array([0, 5, 299, 17, 5], dtype=np.int64)
    got = to_np(ops.embed(matrix, _t(tokens, cuda)))
    expected = oracle.embed(tokens, packed, scale_bits, hidden)
    assert_bits_equal(got, expected, "embed_tile")
    closed = (codes[tokens].astype(np.float32) - 1.0) * np.repeat(T.half_bits_to_float(scale_bits)[tokens], 128,
                                                                 axis=1)[:, :hidden]
    assert_bits_equal(expected, closed, "oracle embed vs closed form")
    lib = runtime.library()
    single = torch.empty(hidden, dtype=torch.float32, device=cuda)
    runtime.check(lib.embed_token(runtime.current_stream(cuda), runtime.pointer(_t(tokens[2:3], cuda)),
                                  runtime.pointer(matrix.packed), runtime.pointer(matrix.scales),
                                  runtime.pointer(single), hidden, matrix.row_bytes, matrix.groups))
    assert_bits_equal(to_np(single), expected[2], "embed_token")
    tile = _t(expected, cuda)
    for valid in (0, 1, 3, 5):
        out = torch.empty(hidden, dtype=torch.float32, device=cuda)
        runtime.check(lib.gather_token(runtime.current_stream(cuda), runtime.pointer(tile), runtime.pointer(out),
                                       hidden, runtime.pointer(_t(np.array([valid], np.int64), cuda))))
        assert_bits_equal(to_np(out), expected[max(valid - 1, 0)], f"gather valid={valid}")
    values = rng.standard_normal(32000).astype(np.float32)
    values[[123, 31000]] = values.max() + 1.0  # tie: the first index wins
    assert int(to_np(ops.argmax(_t(values, cuda)))[0]) == oracle.argmax(values) == 123


@pytest.mark.parametrize("n", [1, 3, 4, 1023, 2048, 2049, 32000, 32001, 100003, 262144])
@pytest.mark.parametrize("offset", [0, 1])
def test_argmax_first_maximum(cuda, oracle, n, offset):
    """Vector and scalar load paths (offset 1 breaks 16-byte alignment), ties, all-negative rows."""
    from ivonar_amd import ops

    rng = np.random.default_rng(n + offset)
    values = (rng.standard_normal(n + offset).astype(np.float32) - 10.0)
    values[offset + rng.integers(0, n, size=min(n, 5))] = -np.inf
    top = values[offset:].max()
    ties = np.sort(rng.integers(0, n, size=min(n, 3)))
    values[offset + ties] = top + 1.0
    device_values = _t(values, cuda)[offset:]
    got = int(to_np(ops.argmax(device_values))[0])
    assert got == oracle.argmax(values[offset:]) == int(ties[0])


def test_argmax_back_to_back(cuda, oracle):
    """Eight argmax calls over different 32000-value rows go out back to back on one stream (the blocks'
    pairs and their count live in the stream's scratch and are reused by every call); each token must be
    the first maximum of its own row, including ties that span blocks."""
    import torch
    from ivonar_amd import ops

    rng = np.random.default_rng(9)
    rows = rng.standard_normal((8, 32000)).astype(np.float32)
    for r in range(8):
        peak = rows[r].max() + 1.0
        rows[r, [int(rng.integers(0, 32000)), int(rng.integers(0, 32000))]] = peak
    device_rows = _t(rows, cuda)
    outs = torch.empty(8, dtype=torch.int64, device=cuda)
    torch.cuda.synchronize()
    for r in range(8):
        ops.argmax(device_rows[r], out=outs[r:r + 1])
    got = to_np(outs)
    for r in range(8):
        assert int(got[r]) == oracle.argmax(rows[r]), f"row {r}"


# ----------------------------------------------------------- graph capture


def test_graph_replays_match_eager(cuda, oracle):
    """A captured GEMV (two-pass: quantize + GEMV) and GEMM replay bit-identically several times."""
    import torch
    from ivonar_amd import ops

    rng = np.random.default_rng(5)
    k, rows, m = 8192, 256, 32
    codes, packed, scale_bits, b, x = _gemv_case(rng, rows, k)
    matrix = device_matrix(packed, scale_bits, k, device=cuda)
    xs = _t(rng.standard_normal((m, k)).astype(np.float32), cuda)
    xv = _t(x, cuda)
    y = torch.empty(rows, dtype=torch.float32, device=cuda)
    q8, xsum, sx = ops.activation_buffers(m, k, cuda)
    out = torch.empty((m, rows), dtype=torch.float32, device=cuda)

    def step():
        ops.gemv(matrix, xv, out=y)
        ops.quantize_rows(xs, out=(q8, xsum, sx))
        ops.gemm(matrix, q8, xsum, sx, out=out)

    step()
    torch.cuda.synchronize()
    eager_y, eager_out = y.clone(), out.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        step()
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step()
    for _ in range(3):
        y.zero_()
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager_y)
        assert torch.equal(out, eager_out)


# ----------------------------------------------------------------- errors


def test_invalid_arguments_raise(cuda):
    import torch
    from ivonar_amd import ops, runtime

    rng = np.random.default_rng(0)
    codes, packed, scale_bits, _, x = _gemv_case(rng, 7, 64)
    matrix = device_matrix(packed, scale_bits, 64, device=cuda)
    with pytest.raises(runtime.KernelError):  # odd row count for a silu pair
        ops.gemv(matrix, _t(x, cuda), out=torch.empty(4, device=cuda), epilogue="silu_pair", mode="norm",
                 aux=_t(np.ones(64, np.float32), cuda))
    lib = runtime.library()
    status = lib.gemv_plain_store(runtime.current_stream(cuda), runtime.pointer(_t(x, cuda)), None, None, None, None,
                                  runtime.pointer(matrix.packed), runtime.pointer(matrix.scales), None,
                                  runtime.pointer(torch.empty(7, device=cuda)), 7, 64, 8, matrix.groups, 2, 1,
                                  runtime.float32(1e-6), None, 0)
    assert status != 0  # row_bytes below 16 * chunks


@pytest.mark.parametrize("m,k,rows", [(2048, 1024, 4096), (2048, 4096, 1024), (512, 1100, 4096), (300, 4096, 2048)])
def test_gemm_large_tiles_every_token(cuda, oracle, m, k, rows):
    """The large block shapes are chosen only at big M: every output bit for bit against the oracle's
    split order, from exact partials."""
    from ivonar_amd import ops, runtime

    rng = np.random.default_rng(m + k + rows)
    codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=(m == 300))
    x = rng.standard_normal((m, k)).astype(np.float32)
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    q8, xsum, sx = ops.quantize_rows(_t(x, cuda))
    y = to_np(ops.gemm(matrix, q8, xsum, sx))
    plan = token_gemm_order(m, rows, k)
    expected = _every_row(oracle, codes, x, k, scale_bits, b, plan)
    assert_bits_equal(y, expected, f"every token (order {plan})")


@pytest.mark.parametrize("m", [1, 3, 16, 32])
@pytest.mark.parametrize("k,rows", [(8192, 512), (28672, 128), (4096, 1024), (1024, 4096)])
def test_gemm_small_m_split_order(cuda, oracle, m, k, rows):
    """Few tokens run the K-split MFMA kernel: bit-exact against the oracle's split order."""
    from ivonar_amd import ops, runtime

    rng = np.random.default_rng(m * 31 + k + rows)
    codes, packed, scale_bits, b = make_layer(rng, rows, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    matrix = device_matrix(packed, scale_bits, k, device=cuda)
    q8, xsum, sx = ops.quantize_rows(_t(x, cuda))
    y = to_np(ops.gemm(matrix, q8, xsum, sx))
    eq8, exsum, esx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    expected = token_gemm_expected(oracle, T.EPI_STORE, eq8, exsum, esx, packed, scale_bits, None,
                                   np.zeros((m, rows), np.float32), k, rows, m)
    assert_bits_equal(y, expected, f"skinny gemm (order {token_gemm_order(m, rows, k)})")
    q, s = T.quantize_closed_form(x[0])
    truth = T.truth_fp64(T.group_partials_int64(codes, q), T.half_bits_to_float(scale_bits), s)
    assert_within(y[0], truth, what="skinny gemm vs fp64 truth")


# The two skinny kernels (M <= 32): the token bytes staged in LDS per wave (8, 4, 2 or 1 K-splits by
# group count; one row tile per wave, two or four from 768 row tiles on) and, when a wave's share does not
# fit there, the token operand read per wave from the caches (one or two row tiles per wave).  Odd
# chunk counts with several groups, ragged rows, bias; every token against the oracle's split
# order.
@pytest.mark.parametrize("m,k,rows,bias,splits", [(7, 4160, 1000, True, 8), (32, 2112, 1000, False, 8),
                                                  (20, 1088, 8200, True, 8), (1, 8192, 8192, False, 8),
                                                  (9, 4096, 12300, True, 8), (32, 2112, 12290, False, 8),
                                                  (32, 4160, 1000, False, 4), (32, 8192, 8200, False, 4),
                                                  (17, 8192, 300, True, 4), (3, 200, 40, True, 2), (1, 28672, 8192, False, 4),
                                                  (5, 40000, 700, True, 0)])
def test_gemm_skinny_kernels(cuda, oracle, m, k, rows, bias, splits):
    from ivonar_amd import ops, runtime

    rng = np.random.default_rng(m * 13 + k + rows)
    codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=bias)
    x = rng.standard_normal((m, k)).astype(np.float32)
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    q8, xsum, sx = ops.quantize_rows(_t(x, cuda))
    y = to_np(ops.gemm(matrix, q8, xsum, sx))
    if m > 16:  # up to 16 tokens the few-token GEMV runs (its own plan, tests/test_gpu_tokens.py)
        assert runtime.gemm_plan(m, rows, k) == splits
    plan = token_gemm_order(m, rows, k)
    assert_bits_equal(y, _every_row(oracle, codes, x, k, scale_bits, b, plan), f"every token (order {plan})")


# Prompts of 33..512 tokens that neither long-prompt tiling takes (few row blocks, few groups) run the
# LDS-staged skinny kernel in 32-token slices; 513 tokens fall back to the tiled kernel (one split).
@pytest.mark.parametrize("m,k,rows,bias,splits", [(300, 1088, 1000, True, 8), (130, 2112, 500, False, 8),
                                                  (45, 200, 40, True, 2), (512, 1024, 96, False, 8),
                                                  (513, 1088, 300, False, 1)])
def test_gemm_sliced_skinny(cuda, oracle, m, k, rows, bias, splits):
    from ivonar_amd import ops, runtime

    rng = np.random.default_rng(m * 17 + k + rows)
    codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=bias)
    x = rng.standard_normal((m, k)).astype(np.float32)
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    q8, xsum, sx = ops.quantize_rows(_t(x, cuda))
    y = to_np(ops.gemm(matrix, q8, xsum, sx))
    assert runtime.gemm_plan(m, rows, k) == splits
    assert_bits_equal(y, _every_row(oracle, codes, x, k, scale_bits, b, splits), f"every token ({splits} splits)")


@pytest.mark.parametrize("epilogue", ["residual", "silu_pair"])
def test_gemm_sliced_skinny_epilogues(cuda, oracle, epilogue):
    import torch
    from ivonar_amd import ops, runtime

    rng = np.random.default_rng(93 if epilogue == "residual" else 92)
    m, k, rows = 70, 1024, 600
    codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=True)
    x = rng.standard_normal((m, k)).astype(np.float32)
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    q8, xsum, sx = ops.quantize_rows(_t(x, cuda))
    width = rows if epilogue == "residual" else rows // 2
    stride = width + 3
    base = rng.standard_normal((m, stride)).astype(np.float32)
    out = _t(base, cuda)
    ops.gemm(matrix, q8, xsum, sx, out=out, epilogue=epilogue, out_stride=stride)
    assert runtime.gemm_plan(m, rows, k) == 8
    eq8, exsum, esx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    epi = T.EPI_RESIDUAL if epilogue == "residual" else T.EPI_SILU_PAIR
    expected = oracle.gemm_split(epi, eq8, exsum, esx, packed, scale_bits, b, base.copy(), k, stride, m, 8)
    assert_bits_equal(to_np(out), expected, epilogue)
    assert torch.equal(out[:, width:], _t(base[:, width:], cuda)), "the GEMM wrote past its output width"


@pytest.mark.parametrize("epilogue", ["residual", "silu_pair"])
def test_gemm_skinny_four_row_tiles_epilogues(cuda, oracle, epilogue):
    import torch
    from ivonar_amd import ops, runtime

    rng = np.random.default_rng(97 if epilogue == "residual" else 96)
    m, k, rows = 24, 2048, 12304
    codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=True)
    x = rng.standard_normal((m, k)).astype(np.float32)
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    q8, xsum, sx = ops.quantize_rows(_t(x, cuda))
    width = rows if epilogue == "residual" else rows // 2
    stride = width + 3
    base = rng.standard_normal((m, stride)).astype(np.float32)
    out = _t(base, cuda)
    ops.gemm(matrix, q8, xsum, sx, out=out, epilogue=epilogue, out_stride=stride)
    assert runtime.gemm_plan(m, rows, k) == 8
    eq8, exsum, esx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    epi = T.EPI_RESIDUAL if epilogue == "residual" else T.EPI_SILU_PAIR
    expected = oracle.gemm_split(epi, eq8, exsum, esx, packed, scale_bits, b, base.copy(), k, stride, m, 8)
    assert_bits_equal(to_np(out), expected, epilogue)
    assert torch.equal(out[:, width:], _t(base[:, width:], cuda)), "the GEMM wrote past its output width"


# Long prompts with many row blocks run the long-prompt kernel (m >= 128; 128-token x 256-row tiles
# from 2048 inputs on with >= 192 blocks, 64-token tiles below with >= 96 blocks, 32-token tiles where
# 64-token tiles give fewer than 192: 700 tokens over 4096 rows): ragged token and row counts, an odd
# chunk count, a single-chunk K, bias, and every epilogue with a padded output stride.
@pytest.mark.parametrize("m,k,rows,bias", [(1000, 1088, 8200, True), (2048, 64, 4096, False),
                                          (128, 4096, 65536, False), (1537, 1100, 5120, True),
                                          (700, 1024, 4096, True), (130, 1024, 24576, False)])
def test_gemm_wide_tiles_edges(cuda, oracle, m, k, rows, bias):
    from ivonar_amd import ops, runtime

    rng = np.random.default_rng(m * 7 + k + rows)
    codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=bias)
    x = rng.standard_normal((m, k)).astype(np.float32)
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    q8, xsum, sx = ops.quantize_rows(_t(x, cuda))
    y = to_np(ops.gemm(matrix, q8, xsum, sx))
    assert runtime.gemm_plan(m, rows, k) == 1
    assert_bits_equal(y, _every_row(oracle, codes, x, k, scale_bits, b, 1), "every token")


@pytest.mark.parametrize("epilogue", ["store", "residual", "silu_pair"])
def test_gemm_wide_32_token_tiles_epilogues(cuda, oracle, epilogue):
    """32-token long-prompt tiles (K=1024 -> N=8192 at 200 tokens: 128 blocks of 64 tokens, 224 of 32)
    with a ragged last tile, a bias and a padded output stride."""
    import torch
    from ivonar_amd import ops, runtime

    rng = np.random.default_rng(98 + len(epilogue))
    m, k, rows = 200, 1024, 8192
    codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=True)
    x = rng.standard_normal((m, k)).astype(np.float32)
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    q8, xsum, sx = ops.quantize_rows(_t(x, cuda))
    width = rows // 2 if epilogue == "silu_pair" else rows
    stride = width + 3
    base = rng.standard_normal((m, stride)).astype(np.float32)
    out = _t(base, cuda)
    ops.gemm(matrix, q8, xsum, sx, out=out, epilogue=epilogue, out_stride=stride)
    assert runtime.gemm_plan(m, rows, k) == 1
    epi = {"store": T.EPI_STORE, "residual": T.EPI_RESIDUAL, "silu_pair": T.EPI_SILU_PAIR}[epilogue]
    expected = _every_row(oracle, codes, x, k, scale_bits, b, 1, epi, base.copy(), stride)
    assert_bits_equal(to_np(out), expected, epilogue)
    assert torch.equal(out[:, width:], _t(base[:, width:], cuda)), "the GEMM wrote past its output width"


@pytest.mark.parametrize("epilogue", ["residual", "silu_pair"])
def test_gemm_wide_tiles_epilogues(cuda, oracle, epilogue):
    import torch
    from ivonar_amd import ops

    rng = np.random.default_rng(97 if epilogue == "residual" else 96)
    m, k, rows = 300, 1024, 24576
    codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=True)
    x = rng.standard_normal((m, k)).astype(np.float32)
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    q8, xsum, sx = ops.quantize_rows(_t(x, cuda))
    width = rows if epilogue == "residual" else rows // 2
    stride = width + 3
    base = rng.standard_normal((m, stride)).astype(np.float32)
    out = _t(base, cuda)
    ops.gemm(matrix, q8, xsum, sx, out=out, epilogue=epilogue, out_stride=stride)
    epi = T.EPI_RESIDUAL if epilogue == "residual" else T.EPI_SILU_PAIR
    expected = _every_row(oracle, codes, x, k, scale_bits, b, 1, epi, base.copy(), stride)
    assert_bits_equal(to_np(out), expected, epilogue)
    assert torch.equal(out[:, width:], _t(base[:, width:], cuda)), "the GEMM wrote past its output width"


# 128-token tiles (2048 inputs and more) with both epilogues, every token: 192 blocks of 128
# tokens x 256 rows.
@pytest.mark.parametrize("epilogue", ["residual", "silu_pair"])
def test_gemm_wide_128_token_tiles_epilogues(cuda, oracle, epilogue):
    import torch
    from ivonar_amd import ops, runtime

    rng = np.random.default_rng(91 if epilogue == "residual" else 90)
    m, k, rows = 1024, 2048, 6144
    codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=True)
    x = rng.standard_normal((m, k)).astype(np.float32)
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    q8, xsum, sx = ops.quantize_rows(_t(x, cuda))
    width = rows if epilogue == "residual" else rows // 2
    stride = width + 3
    base = rng.standard_normal((m, stride)).astype(np.float32)
    out = _t(base, cuda)
    ops.gemm(matrix, q8, xsum, sx, out=out, epilogue=epilogue, out_stride=stride)
    assert runtime.gemm_plan(m, rows, k) == 1
    epi = T.EPI_RESIDUAL if epilogue == "residual" else T.EPI_SILU_PAIR
    expected = _every_row(oracle, codes, x, k, scale_bits, b, 1, epi, base.copy(), stride)
    assert_bits_equal(to_np(out), expected, epilogue)
    assert torch.equal(out[:, width:], _t(base[:, width:], cuda)), "the GEMM wrote past its output width"


# 64-token tiles at 2048 inputs and more: 850 tokens x 6144 rows give 168 blocks of 128 tokens (too
# few) and 336 of 64 tokens, so the long-prompt kernel runs 64-token tiles over 16 groups rather than
# the split-K kernel.  A ragged last token tile, bias, all three epilogues, every token.
@pytest.mark.parametrize("epilogue", ["store", "residual", "silu_pair"])
def test_gemm_wide_64_token_tiles_long_k(cuda, oracle, epilogue):
    import torch
    from ivonar_amd import ops, runtime

    rng = np.random.default_rng({"store": 81, "residual": 82, "silu_pair": 83}[epilogue])
    m, k, rows = 850, 2048, 6144
    codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=True)
    x = rng.standard_normal((m, k)).astype(np.float32)
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    q8, xsum, sx = ops.quantize_rows(_t(x, cuda))
    assert runtime.gemm_plan(m, rows, k) == 1
    width = rows // 2 if epilogue == "silu_pair" else rows
    stride = width + 3
    base = rng.standard_normal((m, stride)).astype(np.float32)
    out = _t(base, cuda)
    ops.gemm(matrix, q8, xsum, sx, out=out, epilogue=epilogue, out_stride=stride)
    epi = {"store": T.EPI_STORE, "residual": T.EPI_RESIDUAL, "silu_pair": T.EPI_SILU_PAIR}[epilogue]
    expected = _every_row(oracle, codes, x, k, scale_bits, b, 1, epi, base.copy(), stride)
    assert_bits_equal(to_np(out), expected, epilogue)
    assert torch.equal(out[:, width:], _t(base[:, width:], cuda)), "the GEMM wrote past its output width"


# Long prompts with few output rows run the split-K kernel (S waves per 128, 64 or 32-token x 64-row
# tile, each a contiguous 1/S of the groups, added in order): its plan reports S = 4, or 8 for 32-token
# tiles with at least 32 groups.  Ragged tokens and rows, an odd chunk count with a group count not
# divisible by four, bias, and both epilogues; the cases cover all three token tiles (M=2048 and 70
# tokens over 14336 rows: 128 with two stages; 1000 and 1024 tokens and the epilogues: 64 with three
# stages; 33, 127, 300 and 512 tokens: 32 with three stages), eight waves (512 and 300 tokens; at
# K=4160 the eighth wave's range is empty and the seventh has 3 of 5 groups, so padding steps run
# with zero scales).  Prompts of 33..127 tokens fill one partial token tile (the rows past the prompt
# read zeros).
@pytest.mark.parametrize("m,k,rows,bias,splits", [(1000, 4160, 1000, True, 4), (2048, 2048, 1024, False, 4),
                                                 (2048, 4096, 1024, True, 4), (33, 2048, 2048, False, 4),
                                                 (70, 4096, 14336, True, 4), (127, 2176, 3000, False, 4),
                                                 (512, 4096, 1024, True, 8), (300, 4160, 1000, False, 8),
                                                 (1024, 4096, 1024, False, 4)])
def test_gemm_split_k_edges(cuda, oracle, m, k, rows, bias, splits):
    from ivonar_amd import ops, runtime

    rng = np.random.default_rng(m * 3 + k + rows)
    codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=bias)
    x = rng.standard_normal((m, k)).astype(np.float32)
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    q8, xsum, sx = ops.quantize_rows(_t(x, cuda))
    y = to_np(ops.gemm(matrix, q8, xsum, sx))
    assert runtime.gemm_plan(m, rows, k) == splits
    assert_bits_equal(y, _every_row(oracle, codes, x, k, scale_bits, b, splits), f"every token ({splits} splits)")
    sample = np.unique(np.array([0, 1, 31, 32, 95, 127, 128, 129, m // 2, m - 2, m - 1]) % m)
    eq8, exsum, esx = oracle.quantize_rows(T.MODE_PLAIN, x[sample], k)
    ref = oracle.reforder(T.EPI_STORE, True, eq8, exsum, esx, packed, scale_bits, b,
                          np.zeros((len(sample), rows), np.float32), k, reference_lanes(k, rows), rows, len(sample))
    assert_within(y[sample], ref, what="split-K GEMM vs reference-kernel order")


@pytest.mark.parametrize("epilogue", ["residual", "silu_pair"])
def test_gemm_split_k_epilogues(cuda, oracle, epilogue):
    import torch
    from ivonar_amd import ops, runtime

    rng = np.random.default_rng(95 if epilogue == "residual" else 94)
    m, k, rows = 256, 4096, 4096
    codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=True)
    x = rng.standard_normal((m, k)).astype(np.float32)
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    q8, xsum, sx = ops.quantize_rows(_t(x, cuda))
    width = rows if epilogue == "residual" else rows // 2
    stride = width + 3
    base = rng.standard_normal((m, stride)).astype(np.float32)
    out = _t(base, cuda)
    ops.gemm(matrix, q8, xsum, sx, out=out, epilogue=epilogue, out_stride=stride)
    assert runtime.gemm_plan(m, rows, k) == 4
    epi = T.EPI_RESIDUAL if epilogue == "residual" else T.EPI_SILU_PAIR
    expected = _every_row(oracle, codes, x, k, scale_bits, b, 4, epi, base.copy(), stride)
    assert_bits_equal(to_np(out), expected, epilogue)
    assert torch.equal(out[:, width:], _t(base[:, width:], cuda)), "the GEMM wrote past its output width"
