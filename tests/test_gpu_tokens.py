"""GPU parity of the token GEMV: 1..16 tokens against one packed matrix with K a multiple of 256 and the
tokens' q8 rows within the LDS budget (the gemm_tile_* entry points route those calls to it).

Every output of every token is checked bit for bit against the oracle's split order (S = the library's
plan, contiguous group ranges folded in order and added in order), and token 0 within rel 1e-5 / abs 1e-6
of the fp64 truth.  Two tokens of 4097..32768 inputs run the long-row decode GEMV over each token's copy
(plan 0) and are checked in its lane order.  Cases: the planner's span choices (1, 2, 4, 8, 14 and 16 spans per wave), ragged row
counts, a bias, both epilogues with a padded output stride, token counts that are not a multiple of four
(the last lane group's slots past M), and rows too long for the tokens' q8 bytes in LDS, where K is cut
into 2, 4 or 8 slices across blocks and a second kernel adds the wave chains in order."""

from __future__ import annotations

import numpy as np
import pytest

import ternary_oracle as T
from _util import assert_bits_equal, assert_within, device_matrix, finish_all_rows, make_layer, to_np, token_gemm_order

pytestmark = pytest.mark.gpu


def _t(array, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(array)).to(device)


def _case(oracle, cuda, m, k, rows, bias, seed, epilogue="store", pad=0):
    import torch
    from ivonar_amd import ops, runtime

    print(f"token gemv m={m} k={k} rows={rows} bias={bias} {epilogue}", flush=True)
    rng = np.random.default_rng(seed)
    codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=bias)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[:, :: max(1, k // 50)] *= 20.0  # outlier channels set the absmax
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    q8, xsum, sx = ops.quantize_rows(_t(x, cuda))
    eq8, exsum, esx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    assert_bits_equal(to_np(q8), eq8, "q8")
    width = rows // 2 if epilogue == "silu_pair" else rows
    stride = width + pad
    base = rng.standard_normal((m, stride)).astype(np.float32) if epilogue == "residual" else np.zeros(
        (m, stride), np.float32)
    out = _t(base, cuda)
    ops.gemm(matrix, q8, xsum, sx, out=out, epilogue=epilogue, out_stride=stride)
    order, param = token_gemm_order(m, rows, k)
    splits = param if order == 1 else runtime.gemm_plan(m, rows, k)
    epi = {"store": T.EPI_STORE, "residual": T.EPI_RESIDUAL, "silu_pair": T.EPI_SILU_PAIR}[epilogue]
    q = T.q8_linear(eq8, k)
    expected = finish_all_rows(oracle, order, param, epi, codes, q, scale_bits, esx, b, base.copy(), k, stride)
    got = to_np(out)
    assert_bits_equal(got, expected, f"token gemv m={m} k={k} rows={rows} ({splits} splits)")
    if pad:
        assert torch.equal(out[:, width:], _t(base[:, width:], cuda)), "wrote past the output width"
    if epilogue == "store":
        truth = T.truth_fp64(oracle.group_partials(eq8[0], exsum[0], packed, rows, k), T.half_bits_to_float(scale_bits),
                             esx[0], b)
        assert_within(got[0, :rows], truth, what="token 0 vs fp64 truth")
    return splits


# (m, k, rows, bias, K-splits of the plan on a 256-CU device): the plan takes the longest span range
# per wave that still gives every CU eight waves, else one span per wave.
@pytest.mark.parametrize("m,k,rows,bias,splits", [
    (1, 1024, 4096, False, 0),     # one token: the decode GEMV (plan 0, its lane order)
    (2, 1024, 4096, False, 4),     # 4 spans, 1 per wave
    (5, 4096, 1000, True, 16),     # ragged rows, 16 waves per row tile
    (4, 8192, 8200, True, 4),      # 8 spans per wave, ragged rows
    (8, 2048, 16384, False, 2),    # 4 spans per wave
    (4, 28672, 8192, False, 7),    # the long-row stress shape, 16 spans per wave
    (16, 8192, 2000, False, 16),   # 2 spans per wave, 128 KB of token bytes
    (4, 28672, 1000, True, 14),    # 8 spans per wave (no range reaches eight waves per CU)
    (4, 7168, 16384, False, 2),    # 14 spans per wave
    (16, 256, 40, True, 1),        # one span, one wave per row tile
    (13, 3584, 4100, False, 14),   # 14 spans, one per wave
])
def test_token_gemv_store(cuda, oracle, m, k, rows, bias, splits):
    got = _case(oracle, cuda, m, k, rows, bias, seed=m * 1009 + k + rows)
    assert got == splits


# (m, k, rows, bias): two tokens of 4097..32768 inputs run the long-row decode GEMV over each token's copy
# (plan 0): every token's outputs in its own GEMV's lane order.  K a multiple of 4096 (no clamped chunks)
# and not (4160, 6000, 20000: the last step's lanes partly dead), 2..8 steps per row, ragged row counts,
# one row pair per wave and several.  Three tokens stay on the token GEMV.
@pytest.mark.parametrize("m,k,rows,bias", [
    (2, 8192, 28672, False),   # the stress shape, two blocks per CU
    (2, 8192, 1000, True),
    (2, 28672, 8192, False),   # the other stress shape, seven steps per row
    (2, 28672, 130, True),
    (2, 4160, 700, True),      # two steps, the second with one live lane pair
    (2, 6000, 4097, False),
    (2, 20000, 3001, True),    # five steps
    (2, 32768, 514, False),    # eight steps, 68 KB of copies in LDS
])
def test_gemv_tokens_store(cuda, oracle, m, k, rows, bias):
    assert _case(oracle, cuda, m, k, rows, bias, seed=m * 211 + k + rows) == 0


def test_three_tokens_stay_on_the_token_gemv(cuda):
    from ivonar_amd import runtime

    assert runtime.gemm_plan(2, 1000, 8192) == 0
    assert runtime.gemm_plan(3, 1000, 8192) > 0
    assert runtime.gemm_plan(2, 1000, 4096) > 0, "4096 inputs and fewer: the token GEMV"


@pytest.mark.parametrize("epilogue", ["residual", "silu_pair"])
@pytest.mark.parametrize("m,k,rows", [(2, 8192, 1000), (2, 28672, 514), (2, 6000, 258)])
def test_gemv_tokens_epilogues(cuda, oracle, epilogue, m, k, rows):
    assert _case(oracle, cuda, m, k, rows, True, seed=m * 37 + k + rows + (5 if epilogue == "residual" else 0),
                 epilogue=epilogue, pad=3) == 0


@pytest.mark.parametrize("epilogue", ["residual", "silu_pair"])
@pytest.mark.parametrize("m,k,rows", [(7, 2048, 1000), (16, 4096, 514), (1, 8192, 3000)])
def test_token_gemv_epilogues(cuda, oracle, epilogue, m, k, rows):
    _case(oracle, cuda, m, k, rows, True, seed=m * 31 + k + rows + (7 if epilogue == "residual" else 0),
          epilogue=epilogue, pad=3)


def test_token_gemv_stress_shape_sixteen_tokens(cuda, oracle):
    """K=8192 -> N=28672 with 16 tokens: 128 KB of token bytes in LDS, the planner's largest fill."""
    assert _case(oracle, cuda, 16, 8192, 28672, False, seed=5) == 2


# (m, k, rows, bias, K-splits = slices x waves per row tile): the tokens' whole q8 rows exceed the LDS budget.
@pytest.mark.parametrize("m,k,rows,bias,splits", [
    (16, 28672, 512, True, 56),    # 4 slices x 14 waves (448 KB of q8 in all)
    (5, 28672, 1000, True, 28),    # 2 slices x 14
    (12, 28672, 4100, False, 8),   # 4 slices x 2, ragged rows
    (9, 20480, 3000, True, 20),    # 2 slices x 10
    (3, 65536, 700, False, 32),    # 2 slices x 16
    (16, 65536, 1024, False, 32),  # 8 slices x 4, sixteen fill pieces per thread
    (13, 28672, 130, True, 56),    # fewer row tiles than blocks of one slice
    (11, 28672, 8192, False, 8),   # 2 slices, LDS within 1 KB of the budget
])
def test_token_gemv_sliced(cuda, oracle, m, k, rows, bias, splits):
    assert _case(oracle, cuda, m, k, rows, bias, seed=m * 7 + k + rows) == splits


@pytest.mark.parametrize("epilogue", ["residual", "silu_pair"])
def test_token_gemv_sliced_epilogues(cuda, oracle, epilogue):
    assert _case(oracle, cuda, 16, 28672, 514, True, seed=61 if epilogue == "residual" else 62, epilogue=epilogue,
                 pad=3) == 56


@pytest.mark.parametrize("epilogue", ["store", "residual", "silu_pair"])
def test_token_gemv_sliced_second_kernel(cuda, oracle, epilogue):
    """With the in-launch finish switched off (ivonar_token_finish_limit(0), as for calls with more row-tile
    groups than the scratch has counters), the K-sliced token GEMV adds its chains in token_finish_kernel:
    the same bits in the same order."""
    from ivonar_amd import runtime

    lib = runtime.library()
    previous = lib.ivonar_token_finish_limit(0)
    assert previous == 992
    try:
        assert _case(oracle, cuda, 16, 28672, 514, True, seed=63, epilogue=epilogue,
                     pad=0 if epilogue == "store" else 3) == 56
    finally:
        assert lib.ivonar_token_finish_limit(previous) == 0


def test_token_gemv_sliced_stress_shapes(cuda, oracle):
    """K=28672 -> N=8192 with 8 and 16 tokens: two and four slices of two or four waves per row tile."""
    assert _case(oracle, cuda, 8, 28672, 8192, False, seed=7) == 8
    assert _case(oracle, cuda, 16, 28672, 8192, False, seed=8) == 8


def test_token_gemv_graph_replays(cuda, oracle):
    """One-slice and sliced token GEMVs and the two-token GEMV captured in a HIP graph replay bit-identically
    to the eager calls, with eager calls of the same kernels (on the default stream) between the replays."""
    import torch
    from ivonar_amd import ops, runtime

    rng = np.random.default_rng(77)
    cases = []
    for m, k, rows in ((5, 4096, 1000), (16, 28672, 512), (2, 8192, 1000)):
        codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=True)
        matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
        q8, xsum, sx = ops.quantize_rows(_t(rng.standard_normal((m, k)).astype(np.float32), cuda))
        other = ops.quantize_rows(_t(rng.standard_normal((m, k)).astype(np.float32), cuda))
        cases.append((matrix, (q8, xsum, sx), other, torch.empty((m, rows), dtype=torch.float32, device=cuda),
                      torch.empty((m, rows), dtype=torch.float32, device=cuda)))
    assert runtime.gemm_plan(16, 512, 28672) == 56
    assert runtime.gemm_plan(2, 1000, 8192) == 0

    def step():
        for matrix, (q8, xsum, sx), _, out, _ in cases:
            ops.gemm(matrix, q8, xsum, sx, out=out)

    step()
    torch.cuda.synchronize()
    eager = [case[3].clone() for case in cases]
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        step()
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step()
    torch.cuda.synchronize()
    other_expected = []
    for matrix, _, (q8, xsum, sx), _, side in cases:
        ops.gemm(matrix, q8, xsum, sx, out=side)
    torch.cuda.synchronize()
    other_expected = [case[4].clone() for case in cases]
    for replay in range(4):
        for case in cases:
            case[3].zero_()
            case[4].zero_()
        torch.cuda.synchronize()
        graph.replay()
        for matrix, _, (q8, xsum, sx), _, side in cases:  # eager work between and during the replays
            ops.gemm(matrix, q8, xsum, sx, out=side)
        torch.cuda.synchronize()
        for i, case in enumerate(cases):
            assert torch.equal(case[3], eager[i]), f"replay {replay}, case {i}"
            assert torch.equal(case[4], other_expected[i]), f"eager call after replay {replay}, case {i}"


class _PaddedScales:
    """A device matrix whose fp16 scale rows carry `extra` unused groups past ceil(K/128) (the C ABI accepts
    groups >= ceil(K/128)); the q8 rows of the tokens stay K wide."""

    def __init__(self, matrix, extra: int):
        import torch

        self.packed, self.bias = matrix.packed, matrix.bias
        self.rows, self.in_features, self.row_bytes, self.lanes = (matrix.rows, matrix.in_features,
                                                                    matrix.row_bytes, matrix.lanes)
        self.groups = matrix.groups + extra
        padded = torch.full((matrix.rows, self.groups), float("nan"), dtype=torch.float16,
                            device=matrix.scales.device)
        padded[:, :matrix.groups] = matrix.scales.view(matrix.rows, matrix.groups)
        self.scales = padded


# (m, k, rows): the token GEMV in one slice and in K slices, the skinny kernel, the 32-token slices and the
# long-prompt and split-K tilings, all with one or three unused scale groups per row.
@pytest.mark.parametrize("m,k,rows", [(5, 4096, 1000), (12, 28672, 4100), (3, 1024, 300), (32, 4096, 1024),
                                      (100, 2048, 700), (512, 4096, 1024), (300, 4096, 14336), (2, 8192, 1000),
                                      (2, 20480, 300)])
@pytest.mark.parametrize("extra", [1, 2])
def test_token_gemm_padded_scale_rows(cuda, oracle, m, k, rows, extra):
    from ivonar_amd import ops, runtime

    print(f"token gemm padded scales m={m} k={k} rows={rows} extra={extra}", flush=True)
    rng = np.random.default_rng(m * 13 + k + rows + extra)
    codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=True)
    x = rng.standard_normal((m, k)).astype(np.float32)
    matrix = _PaddedScales(device_matrix(packed, scale_bits, k, bias=b, device=cuda), extra)
    q8, xsum, sx = ops.quantize_rows(_t(x, cuda))
    eq8, _, esx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    out = ops.gemm(matrix, q8, xsum, sx)
    order, param = token_gemm_order(m, rows, k)
    expected = finish_all_rows(oracle, order, param, T.EPI_STORE, codes, T.q8_linear(eq8, k), scale_bits, esx, b,
                               np.zeros((m, rows), np.float32), k, rows)
    assert_bits_equal(to_np(out), expected, f"padded scales m={m} k={k} rows={rows} (order {order}, {param})")


@pytest.mark.parametrize("k", [1024, 8192, 28672])
def test_gemv_padded_scale_rows(cuda, oracle, k):
    from ivonar_amd import ops, runtime

    rows = 1000
    print(f"gemv padded scales k={k} rows={rows}", flush=True)
    rng = np.random.default_rng(k + 3)
    codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=True)
    x = rng.standard_normal(k).astype(np.float32)
    matrix = _PaddedScales(device_matrix(packed, scale_bits, k, bias=b, device=cuda), 2)
    got = to_np(ops.gemv(matrix, _t(x, cuda)))
    eq8, _, esx = oracle.quantize_rows(T.MODE_PLAIN, x[None], k)
    lanes, _ = runtime.gemv_plan(rows, k)
    expected = finish_all_rows(oracle, 0, lanes, T.EPI_STORE, codes, T.q8_linear(eq8, k), scale_bits, esx, b,
                               np.zeros((1, rows), np.float32), k, rows)
    assert_bits_equal(got, expected[0], f"gemv padded scales k={k}")
