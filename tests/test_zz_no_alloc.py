"""The no-allocation GEMV entry point (ivonar_gemv_plain_store_noalloc): through the C ABI, its outputs
equal gemv_plain_store's bit for bit (and the oracle's) on two calls in a row, the second with a smaller
input, for rows longer than the fused limit (quantized into the library's static array) and shorter
ones; rows above its 32768-input limit are refused."""

from __future__ import annotations

import numpy as np
import pytest

import ternary_oracle as T
from _util import assert_bits_equal, big_layer, device_matrix, to_np

pytestmark = pytest.mark.gpu


def _call(lib, name, runtime, matrix, x, out):
    return getattr(lib, name)(
        runtime.current_stream(x.device), runtime.pointer(x), None, None, None, None, runtime.pointer(matrix.packed),
        runtime.pointer(matrix.scales), runtime.pointer(matrix.bias), runtime.pointer(out), matrix.rows,
        matrix.in_features, matrix.row_bytes, matrix.groups, matrix.lanes, 1, runtime.float32(1e-6), None, 0)


@pytest.mark.parametrize("shapes", [((28672, 4096), (8192, 1024)), ((32768, 700), (5000, 333)),
                                    ((2048, 512), (1024, 100))])
def test_noalloc_matches_gemv_plain_store_twice(cuda, oracle, shapes):
    import torch
    from ivonar_amd import runtime

    lib = runtime.library()
    for call, (k, rows) in enumerate(shapes):
        print(f"noalloc call {call}: K={k} N={rows}", flush=True)
        rng = np.random.default_rng(k + rows + call)
        codes, packed, scale_bits, b = big_layer(rng, rows, k, sigma=0.01, bias=call == 1)
        matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
        x = torch.from_numpy(rng.standard_normal(k).astype(np.float32)).to(cuda)
        mine = torch.full((rows,), float("nan"), dtype=torch.float32, device=cuda)
        reference = torch.full((rows,), float("nan"), dtype=torch.float32, device=cuda)
        runtime.check(_call(lib, "ivonar_gemv_plain_store_noalloc", runtime, matrix, x, mine), "noalloc")
        runtime.check(_call(lib, "gemv_plain_store", runtime, matrix, x, reference), "gemv_plain_store")
        torch.cuda.synchronize()
        assert_bits_equal(to_np(mine), to_np(reference), f"call {call}: noalloc vs gemv_plain_store")
        q8, xsum, sx = oracle.quantize_rows(T.MODE_PLAIN, to_np(x), k)
        lanes, _ = runtime.gemv_plan(rows, k)
        expected = oracle.gemv_pairs(T.EPI_STORE, q8[0], xsum[0], sx[0], packed, scale_bits, b,
                                     np.zeros(rows, np.float32), k, lanes)
        assert_bits_equal(to_np(mine), expected, f"call {call}: noalloc vs oracle")


def test_noalloc_refuses_rows_beyond_its_array(cuda):
    import torch
    from ivonar_amd import runtime

    rng = np.random.default_rng(0)
    k, rows = 32769, 8
    codes, packed, scale_bits, _ = big_layer(rng, rows, k)
    matrix = device_matrix(packed, scale_bits, k, device=cuda)
    x = torch.zeros(k, dtype=torch.float32, device=cuda)
    out = torch.zeros(rows, dtype=torch.float32, device=cuda)
    status = _call(runtime.library(), "ivonar_gemv_plain_store_noalloc", runtime, matrix, x, out)
    assert status != 0
    torch.cuda.synchronize()
    assert not out.any()
