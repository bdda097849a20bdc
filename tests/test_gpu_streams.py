"""GPU calls that go through the library's scratch, issued on several streams at once.

A decode GEMV on a row longer than 4096 inputs that it does not quantize itself (here: read from an
address that is not 16-byte aligned) quantizes the row into a scratch buffer in one launch and reads
it in the next; a token GEMM of up to 16 tokens whose q8 rows exceed LDS writes its wave chains to a
scratch buffer and adds them in a second launch.  Each stream has its own scratch, so calls on two
streams, interleaved without synchronisation, must each give the oracle's bits, in every repetition
(a shared buffer would let one stream's quantizer or chains overwrite the other's between its two
launches); so must calls on 40 streams, more than any fixed table of per-stream scratch would hold."""

from __future__ import annotations

import numpy as np
import pytest

import ternary_oracle as T
from _util import assert_bits_equal, device_matrix, finish_all_rows, make_layer, to_np

pytestmark = pytest.mark.gpu

REPEATS = 24


def _t(array, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(array)).to(device)


def _unaligned(x):
    """The same values one float past a 16-byte boundary (the GEMV's separate-quantizer path)."""
    import torch

    padded = torch.zeros(x.numel() + 1, dtype=torch.float32, device=x.device)
    padded[1:] = x
    assert padded[1:].data_ptr() % 16 != 0
    return padded[1:]


def test_long_row_gemv_on_two_streams(cuda, oracle):
    import torch
    from ivonar_amd import ops, runtime

    k, rows = 8192, 3000
    print(f"two-stream gemv_plain_store K={k} N={rows}", flush=True)
    rng = np.random.default_rng(41)
    codes, packed, scale_bits, _ = make_layer(rng, rows, k)
    matrix = device_matrix(packed, scale_bits, k, device=cuda)
    lanes, _ = runtime.gemv_plan(rows, k)
    xs = [rng.standard_normal(k).astype(np.float32) * scale for scale in (1.0, 37.0)]
    expected = []
    for x in xs:
        q8, xsum, sx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
        expected.append(oracle.gemv_pairs(T.EPI_STORE, q8[0], xsum[0], sx[0], packed, scale_bits, None,
                                          np.zeros(rows, np.float32), k, lanes))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    inputs = [_unaligned(_t(x, cuda)) for x in xs]
    outs = [torch.empty((REPEATS, rows), dtype=torch.float32, device=cuda) for _ in xs]
    torch.cuda.synchronize()
    for rep in range(REPEATS):
        for side in (0, 1):
            with torch.cuda.stream(streams[side]):
                ops.gemv(matrix, inputs[side], out=outs[side][rep])
    torch.cuda.synchronize()
    for side in (0, 1):
        got = to_np(outs[side])
        for rep in range(REPEATS):
            assert_bits_equal(got[rep], expected[side], f"stream {side}, repetition {rep}")


def test_sliced_token_gemm_on_two_streams(cuda, oracle):
    import torch
    from ivonar_amd import ops, runtime

    m, k, rows = 16, 28672, 512
    print(f"two-stream sliced token gemm m={m} K={k} N={rows}", flush=True)
    rng = np.random.default_rng(42)
    codes, packed, scale_bits, b = make_layer(rng, rows, k, bias=True)
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    splits = runtime.gemm_plan(m, rows, k)
    assert splits == 56, "four K slices of 14 waves per row tile"
    operands, expected = [], []
    for scale in (1.0, 5.0):
        x = (rng.standard_normal((m, k)) * scale).astype(np.float32)
        q8, xsum, sx = ops.quantize_rows(_t(x, cuda))
        eq8, _, esx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
        operands.append((q8, xsum, sx))
        expected.append(finish_all_rows(oracle, 1, splits, T.EPI_STORE, codes, T.q8_linear(eq8, k), scale_bits, esx,
                                        b, np.zeros((m, rows), np.float32), k, rows))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [torch.empty((REPEATS, m, rows), dtype=torch.float32, device=cuda) for _ in operands]
    torch.cuda.synchronize()
    for rep in range(REPEATS):
        for side in (0, 1):
            with torch.cuda.stream(streams[side]):
                q8, xsum, sx = operands[side]
                ops.gemm(matrix, q8, xsum, sx, out=outs[side][rep])
    torch.cuda.synchronize()
    for side in (0, 1):
        got = to_np(outs[side])
        for rep in range(REPEATS):
            assert_bits_equal(got[rep], expected[side], f"stream {side}, repetition {rep}")


def test_scratch_calls_on_forty_streams(cuda, oracle):
    """40 streams, each with its own input, make scratch-using GEMV calls (unaligned K=8192 rows) three
    times each, interleaved without synchronisation: every stream gets a scratch of its own (no table
    limit, no shared fallback), so every output is the oracle's for its stream's input."""
    import torch
    from ivonar_amd import ops, runtime

    k, rows, count = 8192, 1024, 40
    print(f"{count}-stream gemv_plain_store K={k} N={rows}", flush=True)
    rng = np.random.default_rng(43)
    codes, packed, scale_bits, _ = make_layer(rng, rows, k)
    matrix = device_matrix(packed, scale_bits, k, device=cuda)
    lanes, _ = runtime.gemv_plan(rows, k)
    xs = [(rng.standard_normal(k) * (1.0 + i)).astype(np.float32) for i in range(count)]
    expected = []
    for x in xs:
        q8, xsum, sx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
        expected.append(oracle.gemv_pairs(T.EPI_STORE, q8[0], xsum[0], sx[0], packed, scale_bits, None,
                                          np.zeros(rows, np.float32), k, lanes))
    streams = [torch.cuda.Stream() for _ in range(count)]
    inputs = [_unaligned(_t(x, cuda)) for x in xs]
    outs = torch.empty((count, 3, rows), dtype=torch.float32, device=cuda)
    torch.cuda.synchronize()
    for rep in range(3):
        for i in range(count):
            with torch.cuda.stream(streams[i]):
                ops.gemv(matrix, inputs[i], out=outs[i, rep])
    torch.cuda.synchronize()
    got = to_np(outs)
    for i in range(count):
        for rep in range(3):
            assert_bits_equal(got[i, rep], expected[i], f"stream {i}, repetition {rep}")
