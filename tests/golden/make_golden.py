"""Writes the known-answer fixtures in tests/golden/ from closed forms (numpy, float64 where noted).

The reference ships no golden vectors for the ternary path, so these are
derived from the mathematics the reference states, independently of the C
oracle they pin (reference paths relative to src/ivonar_inference/):

* packing: quantization.py:13-18 (input 4b+k in bits 2k..2k+1, code = w + 1);
* plain quantizer: quantization.py:35-38 / ternary.cu:178-186 in IEEE fp32;
* group partials: int64 brute force of sum (code-1)*q per 128 inputs;
* GEMV output: fp64 truth s_x * sum_g P*scale (+ bias);
* NORM quantizer: RMSNorm with clip (layers.py:10-25, ternary.cu:169-176) in
  fp64; inputs are resampled until no value lies within 1e-3 of a rounding
  tie, so the fp64 codes are the codes any faithful fp32 evaluation gives;
* ATTN quantizer: the split-softmax merge (ternary.cu:128-146) in fp64, with
  the same tie margin;
* embedding rows: (code-1) * scale, exact.

Run: python tests/golden/make_golden.py   (rewrites golden.npz)
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def pack(codes: np.ndarray) -> np.ndarray:
    rows, k = codes.shape
    width = math.ceil(k / 4)
    padded = np.ones((rows, width * 4), dtype=np.uint8)
    padded[:, :k] = codes
    q = padded.reshape(rows, width, 4).astype(np.uint16)
    return (q[..., 0] | (q[..., 1] << 2) | (q[..., 2] << 4) | (q[..., 3] << 6)).astype(np.uint8)


def quantize_f32(values: np.ndarray):
    v = values.astype(np.float32)
    amax = np.float32(np.abs(v).max()) if v.size else np.float32(0)
    s = np.float32(max(np.float32(amax / np.float32(127.0)), np.float32(1e-5)))
    return np.rint(v / s).astype(np.int64), s


def quantize_f64_clear_of_ties(values64: np.ndarray, margin: float = 1e-3):
    amax = float(np.abs(values64).max())
    s = max(amax / 127.0, 1e-5)
    ratio = values64 / s
    frac = np.abs(ratio - np.floor(ratio) - 0.5)
    return np.rint(ratio).astype(np.int64), s, bool((frac > margin).all())


def partials(codes: np.ndarray, q: np.ndarray) -> np.ndarray:
    rows, k = codes.shape
    groups = math.ceil(k / 128)
    w = np.zeros((rows, groups * 128), dtype=np.int64)
    w[:, :k] = codes.astype(np.int64) - 1
    qp = np.zeros(groups * 128, dtype=np.int64)
    qp[:k] = q
    return (w.reshape(rows, groups, 128) * qp.reshape(groups, 128)).sum(-1)


def main() -> None:
    rng = np.random.default_rng(20240601)
    out: dict[str, np.ndarray] = {}

    # Packing known answers: codes (0,1,2,0) -> 0b00_10_01_00 = 0x24 and friends.
    known_codes = np.array([[0, 1, 2, 0, 2, 2, 2, 2, 1, 1, 1, 1, 0, 0, 0, 0, 2, 0]], dtype=np.uint8)
    out["pack_codes"] = known_codes
    out["pack_bytes"] = np.array([[0x24, 0xAA, 0x55, 0x00, 0x52]], dtype=np.uint8)  # last byte padded with code 1
    assert np.array_equal(pack(known_codes), out["pack_bytes"])

    # Plain quantizer + partials + fp64 outputs over the edge widths.
    cases = []
    for index, (rows, k) in enumerate([(1, 8), (5, 16), (3, 24), (64, 96), (7, 100), (16, 256), (64, 1024), (9, 1100)]):
        codes = (rng.random((rows, k)) >= 0.3).astype(np.uint8) + (rng.random((rows, k)) >= 0.5).astype(np.uint8)
        scales = (np.abs(rng.normal(0, 0.02, (rows, math.ceil(k / 128)))) + 1e-4).astype(np.float16)
        bias = rng.normal(0, 0.02, rows).astype(np.float32) if index % 2 else np.zeros(0, np.float32)
        x = rng.standard_normal(k).astype(np.float32) * np.float32(rng.choice([0.5, 1.0, 30.0]))
        q, s = quantize_f32(x)
        p = partials(codes, q)
        y = (p.astype(np.float64) * scales.astype(np.float64)).sum(-1) * float(s)
        if bias.size:
            y = y + bias.astype(np.float64)
        prefix = f"plain{index}_"
        out[prefix + "codes"] = codes
        out[prefix + "packed"] = pack(codes)
        out[prefix + "scales"] = scales.view(np.uint16)
        out[prefix + "bias"] = bias
        out[prefix + "x"] = x
        out[prefix + "q"] = q.astype(np.int8)
        out[prefix + "scale"] = np.array([s], np.float32)
        out[prefix + "partials"] = p.astype(np.int32)
        out[prefix + "y64"] = y
        cases.append(prefix)
    out["plain_cases"] = np.array(cases)

    # Quantizer special cases (plain): zero row, tiny row, exact ties, negative zero.
    special = np.zeros((4, 16), np.float32)
    special[1] = np.float32(1e-4) * rng.standard_normal(16).astype(np.float32)
    special[2, :8] = [127.0, 2.5, -3.5, 0.5, -0.5, 1.5, -126.5, 3.4999998]
    special[3, :3] = [-0.0, 0.0, -0.0]
    out["special_x"] = special
    out["special_q"] = np.stack([quantize_f32(row)[0] for row in special]).astype(np.int8)
    out["special_scale"] = np.array([quantize_f32(row)[1] for row in special], np.float32)
    assert list(out["special_q"][2, :8]) == [127, 2, -4, 0, 0, 2, -126, 3]
    assert out["special_scale"][0] == np.float32(1e-5)

    # NORM quantizer (fp64 closed form, tie-free inputs).
    norms = []
    for index, n in enumerate([16, 96, 1024, 3000]):
        while True:
            x = (rng.standard_normal(n) * 2.0).astype(np.float32)
            if index == 1:
                x[::5] *= 30.0  # reach the +-8 clip
            w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
            eps = 1e-6
            inv = 1.0 / math.sqrt(float((x.astype(np.float64) ** 2).sum()) / n + eps)
            v = np.clip(x.astype(np.float64) * inv, -8.0, 8.0) * w.astype(np.float64)
            q, s, clear = quantize_f64_clear_of_ties(v)
            if clear:
                break
        prefix = f"norm{index}_"
        out[prefix + "x"] = x
        out[prefix + "w"] = w
        out[prefix + "q"] = q.astype(np.int8)
        out[prefix + "scale64"] = np.array([s])
        norms.append(prefix)
    out["norm_cases"] = np.array(norms)

    # ATTN quantizer (fp64 merge, tie-free).
    while True:
        heads, splits, head_dim = 4, 3, 8
        parts = rng.standard_normal((heads, splits, head_dim + 2)).astype(np.float32)
        parts[..., 1] = np.abs(parts[..., 1]) + 0.5
        parts[1, 2, 0] = -np.inf
        merged = np.zeros((heads, head_dim))
        for h in range(heads):
            peak = parts[h, :, 0].astype(np.float64).max()
            weights = np.where(np.isneginf(parts[h, :, 0]), 0.0, np.exp(parts[h, :, 0].astype(np.float64) - peak))
            merged[h] = (weights[:, None] * parts[h, :, 2:].astype(np.float64)).sum(0) / (
                weights * parts[h, :, 1].astype(np.float64)).sum()
        q, s, clear = quantize_f64_clear_of_ties(merged.reshape(-1))
        if clear:
            break
    out["attn_parts"] = parts
    out["attn_q"] = q.astype(np.int8)
    out["attn_shape"] = np.array([heads, splits, head_dim])

    # Embedding rows (exact).
    codes = (rng.random((10, 40)) * 3).astype(np.uint8)
    scales = (np.abs(rng.normal(0, 0.05, (10, 1))) + 1e-3).astype(np.float16)
    out["embed_codes"] = codes
    out["embed_packed"] = pack(codes)
    out["embed_scales"] = scales.view(np.uint16)
    out["embed_rows"] = ((codes.astype(np.float32) - 1) * scales.astype(np.float32)).astype(np.float32)

    np.savez_compressed(HERE / "golden.npz", **out)
    print(f"wrote {HERE / 'golden.npz'} ({len(out)} arrays)")


if __name__ == "__main__":
    main()
