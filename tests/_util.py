"""Shared helpers for the parity tests: host layers, device matrices and oracle calls."""

from __future__ import annotations

import math

import numpy as np

RTOL, ATOL = 1e-5, 1e-6  # fp32 output tolerance against the reference's order and the fp64 truth


def make_layer(rng: np.random.Generator, rows: int, k: int, p=(0.3, 0.4, 0.3), sigma: float = 0.02,
               bias: bool = False):
    """(codes uint8 [rows,k], packed16 uint8 [rows, rb16], scale bits uint16 [rows,G], bias or None)."""
    import ternary_oracle as T

    u = rng.random((rows, k))
    codes = ((u >= p[0]).astype(np.uint8) + (u >= p[0] + p[1]).astype(np.uint8))
    packed = T.pad_rows16(T.pack_codes(codes))
    groups = math.ceil(k / 128)
    scales = (np.abs(rng.normal(0.0, sigma, size=(rows, groups))) + 1e-4).astype(np.float16)
    b = (rng.normal(0.0, 0.02, size=rows)).astype(np.float32) if bias else None
    return codes, packed, scales.view(np.uint16), b


def device_matrix(packed16: np.ndarray, scale_bits: np.ndarray, k: int, bias=None, device=None):
    import torch
    from ivonar_amd.matrix import Matrix

    packed_t = torch.from_numpy(np.ascontiguousarray(packed16))
    scales_t = torch.from_numpy(np.ascontiguousarray(scale_bits)).view(torch.float16)
    bias_t = None if bias is None else torch.from_numpy(bias)
    return Matrix.from_tensors(packed_t, scales_t, k, bias_t, device=device)


def reference_lanes(k: int, rows: int, max_lanes: int = 32) -> int:
    from ivonar_amd.matrix import _lanes_for

    return _lanes_for((k + 63) // 64, rows, max_lanes)


def to_np(tensor) -> np.ndarray:
    return tensor.detach().cpu().numpy()


def assert_within(actual, expected, rtol: float = RTOL, atol: float = ATOL, what: str = "") -> None:
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    bad = np.abs(actual - expected) > atol + rtol * np.abs(expected)
    if bad.any():
        index = np.argwhere(bad)[0]
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.size} outside rel {rtol} / abs {atol}; first at {tuple(index)}: "
            f"{actual[tuple(index)]!r} vs {expected[tuple(index)]!r}")


def assert_bits_equal(actual, expected, what: str = "") -> None:
    actual = np.asarray(actual)
    expected = np.asarray(expected)
    if actual.shape != expected.shape:
        raise AssertionError(f"{what}: shape {actual.shape} != {expected.shape}")
    if actual.dtype.kind == "f":
        same = (actual == expected) | (np.isnan(actual) & np.isnan(expected))
    else:
        same = actual == expected
    if not same.all():
        index = np.argwhere(~same)[0]
        raise AssertionError(f"{what}: {int((~same).sum())} of {same.size} differ; first at {tuple(index)}: "
                             f"{actual[tuple(index)]!r} vs {expected[tuple(index)]!r}")


def big_layer(rng: np.random.Generator, rows: int, k: int, p=(0.3, 0.4, 0.3), scale: str = "abs_normal",
              sigma: float = 0.02, mu: float = -4.0, bias: bool = False, block: int = 2048):
    """(codes uint8 [rows, k], packed16, scale bits, bias or None) for matrices of up to a few hundred million
    weights, drawn in row blocks so that no float64 copy of the whole matrix is made."""
    import ternary_oracle as T
    from ivonar_amd import synthetic

    codes = np.empty((rows, k), dtype=np.uint8)
    for start in range(0, rows, block):
        codes[start:start + block] = synthetic.sample_codes(rng, min(block, rows - start), k, p)
    packed = T.pad_rows16(synthetic.pack_codes(codes))
    groups = math.ceil(k / 128)
    if scale == "lognormal":
        scales = synthetic.lognormal_scales(rng, rows, groups, mu, sigma)
    else:
        scales = synthetic.abs_normal_scales(rng, rows, groups, sigma, 1e-4)
    b = (rng.normal(0.0, 0.02, size=rows)).astype(np.float32) if bias else None
    return codes, packed, scales.view(np.uint16), b


def exact_partials(codes: np.ndarray, q: np.ndarray) -> np.ndarray:
    """P[t, r, g] = sum_{i in g} (code[r, i] - 1) * q[t, i] as int32 [M, rows, G], for many tokens at once.

    Computed with float32 matrix products per 128-input group: every term is an integer of magnitude at
    most 127 and a group has at most 128 of them, so every partial sum in any summation order is an
    integer below 2**24 and exact in float32."""
    q = np.atleast_2d(q)
    m, k = q.shape
    rows = codes.shape[0]
    groups = math.ceil(k / 128)
    out = np.empty((m, rows, groups), dtype=np.int32)
    for g in range(groups):
        lo, hi = g * 128, min(k, g * 128 + 128)
        w = codes[:, lo:hi].astype(np.float32) - np.float32(1.0)
        out[:, :, g] = np.rint(q[:, lo:hi].astype(np.float32) @ w.T).astype(np.int32)
    return out


def finish_all_rows(oracle, order: int, param: int, epi: int, codes: np.ndarray, q: np.ndarray, scale_bits,
                    sx: np.ndarray, bias, out: np.ndarray, k: int, out_stride: int) -> np.ndarray:
    """Every output row of a token GEMM (order 1: K-split `param`) or GEMV (order 0: `param` lanes) in the
    kernel's fp32 order, from exact partials; tokens in blocks of at most 64M partials (256 MB)."""
    m = q.shape[0]
    block = max(1, min(m, (64 << 20) // max(1, codes.shape[0] * math.ceil(k / 128))))
    for start in range(0, m, block):
        stop = min(m, start + block)
        partials = exact_partials(codes, q[start:stop])
        oracle.finish(order, param, epi, partials, scale_bits, sx[start:stop], bias, out[start:stop], k, out_stride)
    return out


def token_gemm_order(m: int, rows: int, k: int) -> tuple[int, int]:
    """(order, param) of gemm_tile_* for m tokens, as the oracle's finish takes them: the K-split the plan
    reports (order 1), or for plan 0 (one token, or two tokens of 4097..32768 inputs) the decode
    GEMV's lanes (order 0): the GEMV then runs each token's row."""
    from ivonar_amd import runtime

    splits = runtime.gemm_plan(m, rows, k)
    if splits == 0:
        return 0, runtime.gemv_plan(rows, k)[0]
    return 1, splits


def token_gemm_expected(oracle, epi: int, q8, xsum, sx, packed, scale_bits, bias, out: np.ndarray, k: int,
                        out_stride: int, m: int) -> np.ndarray:
    """gemm_tile_*'s outputs for m tokens in the fp32 order of the kernel that runs them."""
    rows = packed.shape[0]
    order, param = token_gemm_order(m, rows, k)
    if order == 1:
        return oracle.gemm_split(epi, q8, xsum, sx, packed, scale_bits, bias, out, k, out_stride, m, param)
    for t in range(m):
        oracle.gemv_pairs(epi, q8[t], xsum[t], sx[t], packed, scale_bits, bias, out[t], k, param)
    return out
