"""The no-allocation GEMV entry point (ivonar_gemv_plain_store_noalloc): through the C ABI, its outputs
equal gemv_plain_store's bit for bit (and the oracle's) on two calls in a row, the second with a smaller
input, for rows longer than the fused limit (aligned: quantized inside the GEMV launch; unaligned:
quantized into the library's static array) and shorter ones; rows above its 32768-input limit are
refused; on a stream the library has not seen it allocates nothing (free device memory unchanged, and
a capture in global mode, where an allocation is an error, replays bit-identically)."""

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


def _unaligned(x):
    """The same values read one float past a 16-byte boundary: the GEMV then quantizes them in a launch of
    its own (into the static array for the no-allocation entry point)."""
    import torch

    padded = torch.zeros(x.numel() + 1, dtype=torch.float32, device=x.device)
    padded[1:] = x
    return padded[1:]


@pytest.mark.parametrize("k,rows", [(8192, 1000), (28672, 300)])
def test_noalloc_unaligned_rows_take_the_static_array(cuda, oracle, k, rows):
    """Unaligned rows longer than the fused limit go through the library's static array: the outputs equal
    gemv_plain_store's (which quantizes into the stream's scratch) and the oracle's, twice in a row."""
    import torch
    from ivonar_amd import runtime

    lib = runtime.library()
    print(f"noalloc unaligned K={k} N={rows}", flush=True)
    rng = np.random.default_rng(k + rows)
    codes, packed, scale_bits, b = big_layer(rng, rows, k, sigma=0.01, bias=True)
    matrix = device_matrix(packed, scale_bits, k, bias=b, device=cuda)
    lanes, _ = runtime.gemv_plan(rows, k)
    for call in range(2):
        host = (rng.standard_normal(k) * (10.0 if call else 0.1)).astype(np.float32)
        x = _unaligned(torch.from_numpy(host).to(cuda))
        assert x.data_ptr() % 16 != 0
        mine = torch.full((rows,), float("nan"), dtype=torch.float32, device=cuda)
        reference = torch.full((rows,), float("nan"), dtype=torch.float32, device=cuda)
        runtime.check(_call(lib, "ivonar_gemv_plain_store_noalloc", runtime, matrix, x, mine), "noalloc")
        runtime.check(_call(lib, "gemv_plain_store", runtime, matrix, x, reference), "gemv_plain_store")
        torch.cuda.synchronize()
        assert_bits_equal(to_np(mine), to_np(reference), f"call {call}: noalloc vs gemv_plain_store")
        q8, xsum, sx = oracle.quantize_rows(T.MODE_PLAIN, host, k)
        expected = oracle.gemv_pairs(T.EPI_STORE, q8[0], xsum[0], sx[0], packed, scale_bits, b,
                                     np.zeros(rows, np.float32), k, lanes)
        assert_bits_equal(to_np(mine), expected, f"call {call}: noalloc vs oracle")


def test_noalloc_allocates_nothing_on_a_fresh_stream(cuda, oracle):
    """On a new stream, the no-allocation entry point leaves the device's free memory unchanged (aligned
    rows quantized in the GEMV launch, unaligned ones into the static array).  The measurement sees an
    allocation of the size a stream's scratch would make: a 16 MB hipMalloc (the scratch's token-partials
    block) lowers the free memory it reports.  Smaller blocks can come from memory the runtime already
    holds for small allocations, so they need not show once earlier calls have run."""
    import ctypes

    import torch
    from ivonar_amd import runtime
    from ivonar_amd.build import torch_hip_runtime

    lib = runtime.library()
    rng = np.random.default_rng(11)
    k, rows = 8192, 512
    codes, packed, scale_bits, _ = big_layer(rng, rows, k)
    matrix = device_matrix(packed, scale_bits, k, device=cuda)
    aligned = torch.from_numpy(rng.standard_normal(k).astype(np.float32)).to(cuda)
    unaligned = _unaligned(aligned)
    outs = torch.empty((3, rows), dtype=torch.float32, device=cuda)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        outs.zero_()  # the runtime's own first-use set-up of the stream happens before the measurement
    torch.cuda.synchronize()
    free_before, _ = torch.cuda.mem_get_info()
    with torch.cuda.stream(stream):
        runtime.check(_call(lib, "ivonar_gemv_plain_store_noalloc", runtime, matrix, aligned, outs[0]), "noalloc")
        runtime.check(_call(lib, "ivonar_gemv_plain_store_noalloc", runtime, matrix, unaligned, outs[1]), "noalloc")
    torch.cuda.synchronize()
    free_after, _ = torch.cuda.mem_get_info()
    assert free_after == free_before, f"the no-allocation calls changed free memory by {free_before - free_after} B"
    runtime.check(_call(lib, "gemv_plain_store", runtime, matrix, aligned, outs[2]), "gemv_plain_store")
    torch.cuda.synchronize()
    assert_bits_equal(to_np(outs[0]), to_np(outs[2]), "aligned noalloc vs gemv_plain_store")
    assert_bits_equal(to_np(outs[1]), to_np(outs[2]), "unaligned noalloc vs gemv_plain_store")

    hip = ctypes.CDLL(str(torch_hip_runtime()))
    block = ctypes.c_void_p()
    assert hip.hipMalloc(ctypes.byref(block), ctypes.c_size_t(16 << 20)) == 0
    try:
        free_control, _ = torch.cuda.mem_get_info()
    finally:
        assert hip.hipFree(block) == 0
    assert free_control < free_after, "a 16 MB hipMalloc did not show in the device's free memory"


def test_noalloc_captured_on_a_fresh_stream_replays(cuda, oracle):
    """Captured (global capture mode, where an allocation is an error) on a stream the library has not
    seen, the no-allocation call replays bit-identically to its eager result four times, with eager
    calls of the same entry point between the replays."""
    import torch
    from ivonar_amd import runtime

    lib = runtime.library()
    rng = np.random.default_rng(12)
    k, rows = 28672, 256
    codes, packed, scale_bits, _ = big_layer(rng, rows, k)
    matrix = device_matrix(packed, scale_bits, k, device=cuda)
    x = _unaligned(torch.from_numpy(rng.standard_normal(k).astype(np.float32)).to(cuda))
    other = _unaligned(torch.from_numpy(rng.standard_normal(k).astype(np.float32)).to(cuda))
    eager = torch.empty(rows, dtype=torch.float32, device=cuda)
    side = torch.empty(rows, dtype=torch.float32, device=cuda)
    captured = torch.full((rows,), float("nan"), dtype=torch.float32, device=cuda)
    runtime.check(_call(lib, "ivonar_gemv_plain_store_noalloc", runtime, matrix, x, eager), "noalloc")
    runtime.check(_call(lib, "ivonar_gemv_plain_store_noalloc", runtime, matrix, other, side), "noalloc")
    torch.cuda.synchronize()
    side_expected = side.clone()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    with torch.cuda.graph(graph, stream=stream, capture_error_mode="global"):
        runtime.check(_call(lib, "ivonar_gemv_plain_store_noalloc", runtime, matrix, x, captured), "noalloc")
    for replay in range(4):
        captured.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert_bits_equal(to_np(captured), to_np(eager), f"replay {replay}")
        side.zero_()
        runtime.check(_call(lib, "ivonar_gemv_plain_store_noalloc", runtime, matrix, other, side), "noalloc")
        torch.cuda.synchronize()
        assert_bits_equal(to_np(side), to_np(side_expected), f"eager call after replay {replay}")
