"""The CPU oracle pinned against closed forms, golden vectors and planted mistakes (CPU only)."""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest

import ternary_oracle as T
from _util import assert_bits_equal, assert_within

GOLDEN = np.load(Path(__file__).resolve().parent / "golden" / "golden.npz", allow_pickle=False)


def _golden_cases(key: str) -> list[str]:
    return [str(name) for name in GOLDEN[key]]


# ------------------------------------------------------------------ format


def test_packing_known_bytes_and_round_trip():
    codes = GOLDEN["pack_codes"]
    assert_bits_equal(T.pack_codes(codes)[:, :4], GOLDEN["pack_bytes"][:, :4], "known bytes")
    rng = np.random.default_rng(0)
    for k in (1, 3, 4, 5, 64, 127, 1000):
        sample = rng.integers(0, 3, size=(3, k), dtype=np.uint8)
        assert_bits_equal(T.unpack_codes(T.pack_codes(sample), k), sample, f"round trip k={k}")
        assert ((T.unpack_codes(T.pack_codes(sample), k)) != 3).all()


def test_row_padding_to_sixteen_bytes():
    packed = np.arange(10 * 5, dtype=np.uint8).reshape(10, 5)
    padded = T.pad_rows16(packed)
    assert padded.shape == (10, 16)
    assert_bits_equal(padded[:, :5], packed)
    assert not padded[:, 5:].any()


def test_half_conversion_is_exact(oracle):
    bits = np.arange(0, 1 << 16, 97, dtype=np.uint16)
    expected = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.h2f(int(b)) for b in bits], dtype=np.float32)
    assert_bits_equal(got, expected, "h2f")


# --------------------------------------------------------------- quantizer


@pytest.mark.parametrize("case", _golden_cases("plain_cases"))
def test_plain_quantizer_matches_golden(oracle, case):
    x = GOLDEN[case + "x"]
    q8, xsum, scale = oracle.quantize_rows(T.MODE_PLAIN, x, x.shape[0])
    eq8, exsum = T.q8_layout(GOLDEN[case + "q"].astype(np.int64))
    assert scale[0] == GOLDEN[case + "scale"][0]
    assert_bits_equal(q8[0], eq8, "q8")
    assert_bits_equal(xsum[0], exsum, "xsum")


def test_quantizer_special_cases(oracle):
    x = GOLDEN["special_x"]
    q8, xsum, scale = oracle.quantize_rows(T.MODE_PLAIN, x, x.shape[1])
    assert_bits_equal(scale, GOLDEN["special_scale"], "scales")
    for row in range(x.shape[0]):
        assert_bits_equal(q8[row], T.q8_layout(GOLDEN["special_q"][row].astype(np.int64))[0], f"row {row}")
    assert scale[0] == np.float32(1e-5) and not q8[0].any()            # all-zero row
    assert scale[1] == np.float32(1e-5)                                  # floor applies below 1.27e-3
    assert abs(int(q8[2][T.q8_index(16)[0]])) == 127                    # argmax element is +-127


def test_q8_layout_pairs_with_the_packed_word_fields():
    """Word k of quad w holds inputs {16w+k+4b}: exactly the bytes of (word >> 2k) & 0x03030303."""
    index = T.q8_index(64)
    for i in range(64):
        quad, k, b = i // 16, i % 4, (i % 16) // 4
        assert index[i] == quad * 16 + k * 4 + b
    assert sorted(index) == list(range(64))


@pytest.mark.parametrize("case", _golden_cases("norm_cases"))
def test_norm_quantizer_matches_fp64_closed_form(oracle, case):
    x, w = GOLDEN[case + "x"], GOLDEN[case + "w"]
    q8, _, scale = oracle.quantize_rows(T.MODE_NORM, x, x.shape[0], aux=w, eps=1e-6)
    assert_bits_equal(q8[0], T.q8_layout(GOLDEN[case + "q"].astype(np.int64))[0], "norm q8")
    assert abs(float(scale[0]) - float(GOLDEN[case + "scale64"][0])) <= 4e-7 * float(GOLDEN[case + "scale64"][0])


def test_attn_quantizer_matches_fp64_closed_form(oracle):
    heads, splits, head_dim = (int(v) for v in GOLDEN["attn_shape"])
    parts = GOLDEN["attn_parts"]
    q8, _, _ = oracle.quantize_rows(T.MODE_ATTN, parts.reshape(-1), heads * head_dim, splits=splits,
                                    head_dim=head_dim)
    assert_bits_equal(q8[0], T.q8_layout(GOLDEN["attn_q"].astype(np.int64))[0], "attn q8")


def test_reference_tree_sum_of_squares(oracle):
    rng = np.random.default_rng(4)
    for n in (1, 31, 256, 257, 1024, 5000):
        v = rng.standard_normal(n).astype(np.float32)
        tree = float(oracle.ref_sum_squares(v))
        exact = float((v.astype(np.float64) ** 2).sum())
        assert abs(tree - exact) <= 1e-6 * exact
    # The tree is a specific order: on these inputs it differs from the sequential fp32 sum (the
    # numba order, cpu_decoder.py:58-61), so a restatement that summed sequentially would fail.
    differs = 0
    for seed in range(20):
        v = np.random.default_rng(100 + seed).standard_normal(4096).astype(np.float32)
        sequential = np.float32(0)
        for value in v:
            sequential = np.float32(sequential + np.float32(value * value))
        differs += float(oracle.ref_sum_squares(v)) != float(sequential)
    assert differs > 0


# ------------------------------------------------------------ integer core


@pytest.mark.parametrize("case", _golden_cases("plain_cases"))
def test_group_partials_match_brute_force(oracle, case):
    codes, x = GOLDEN[case + "codes"], GOLDEN[case + "x"]
    k = x.shape[0]
    packed = T.pad_rows16(GOLDEN[case + "packed"])
    q8, xsum, _ = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    got = oracle.group_partials(q8[0], xsum[0], packed, codes.shape[0], k)
    assert_bits_equal(got, GOLDEN[case + "partials"], "partials")
    assert_bits_equal(T.group_partials_int64(codes, GOLDEN[case + "q"].astype(np.int64)).astype(np.int32),
                      GOLDEN[case + "partials"], "numpy brute force")


def test_planted_mistakes_are_caught(oracle):
    """A transposed q8 layout, a dropped xsum term or a wrong code offset all break the partials."""
    case = "plain6_"
    codes, x = GOLDEN[case + "codes"], GOLDEN[case + "x"]
    k = x.shape[0]
    packed = T.pad_rows16(GOLDEN[case + "packed"])
    expected = GOLDEN[case + "partials"]
    q8, xsum, _ = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    transposed = q8[0].reshape(-1, 4, 4, 4).transpose(0, 1, 3, 2).copy().reshape(-1)
    assert not np.array_equal(oracle.group_partials(transposed, xsum[0], packed, codes.shape[0], k), expected)
    assert not np.array_equal(oracle.group_partials(q8[0], np.zeros_like(xsum[0]), packed, codes.shape[0], k),
                              expected)
    q = GOLDEN[case + "q"].astype(np.int64)
    assert not np.array_equal(T.group_partials_int64(codes.astype(np.int64) + 1, q), expected.astype(np.int64))


# ---------------------------------------------------------------- outputs


@pytest.mark.parametrize("case", _golden_cases("plain_cases"))
@pytest.mark.parametrize("lanes", [2, 8, 64])
def test_fp32_orders_agree_with_fp64_truth(oracle, case, lanes):
    codes, x = GOLDEN[case + "codes"], GOLDEN[case + "x"]
    rows, k = codes.shape
    packed = T.pad_rows16(GOLDEN[case + "packed"])
    scales = GOLDEN[case + "scales"]
    bias = GOLDEN[case + "bias"] if GOLDEN[case + "bias"].size else None
    q8, xsum, sx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    truth = GOLDEN[case + "y64"]
    pairs = oracle.gemv_pairs(T.EPI_STORE, q8[0], xsum[0], sx[0], packed, scales, bias, np.zeros(rows, np.float32),
                              k, lanes)
    seq = oracle.gemm_seq(T.EPI_STORE, q8, xsum, sx, packed, scales, bias, np.zeros((1, rows), np.float32), k, rows,
                          1)
    ref = oracle.reforder(T.EPI_STORE, False, q8, xsum, sx, packed, scales, bias, np.zeros((1, rows), np.float32), k,
                          lanes, rows, 1)
    for name, value in (("pairs", pairs), ("seq", seq[0]), ("reforder", ref[0])):
        assert_within(value, truth, what=name)
    if lanes == 2:
        assert_bits_equal(pairs, seq[0], "two lanes = one pair = the sequential chain")


def test_epilogues_follow_their_definitions(oracle):
    case = "plain6_"
    codes, x = GOLDEN[case + "codes"], GOLDEN[case + "x"]
    rows, k = codes.shape
    packed = T.pad_rows16(GOLDEN[case + "packed"])
    scales = GOLDEN[case + "scales"]
    q8, xsum, sx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    y = oracle.gemv_pairs(T.EPI_STORE, q8[0], xsum[0], sx[0], packed, scales, None, np.zeros(rows, np.float32), k, 8)
    base = np.linspace(-1, 1, rows).astype(np.float32)
    residual = oracle.gemv_pairs(T.EPI_RESIDUAL, q8[0], xsum[0], sx[0], packed, scales, None, base.copy(), k, 8)
    assert_bits_equal(residual, (base + y).astype(np.float32), "residual")
    pair = oracle.gemv_pairs(T.EPI_SILU_PAIR, q8[0], xsum[0], sx[0], packed, scales, None,
                             np.zeros(rows // 2, np.float32), k, 8)
    gate, up = y[0::2].astype(np.float64), y[1::2].astype(np.float64)
    assert_within(pair, gate / (1 + np.exp(-gate)) * up, rtol=1e-6, atol=1e-7, what="silu pair")


def test_expf_is_within_one_ulp(oracle):
    xs = np.concatenate([np.linspace(-100, 88.7, 20001, dtype=np.float32), np.float32([0.0, -0.0, 1e-8, -88.0])])
    got = oracle.expf_array(xs).astype(np.float64)
    truth = np.exp(xs.astype(np.float64))
    normal = truth > np.finfo(np.float32).tiny
    ulp = np.spacing(truth.astype(np.float32)).astype(np.float64)
    assert (np.abs(got - truth)[normal] <= ulp[normal]).all()
    assert oracle.expf(100.0) == math.inf and oracle.expf(-200.0) == 0.0 and oracle.expf(0.0) == 1.0


@pytest.mark.parametrize("index", range(10))
def test_embedding_rows_are_exact(oracle, index):
    tokens = np.array([index, (index * 7) % 10], dtype=np.int64)
    got = oracle.embed(tokens, T.pad_rows16(GOLDEN["embed_packed"]), GOLDEN["embed_scales"], 40)
    assert_bits_equal(got, GOLDEN["embed_rows"][tokens], "embed")


def test_argmax_takes_the_first_maximum(oracle):
    values = np.array([0.5, 2.0, -1.0, 2.0], dtype=np.float32)
    assert oracle.argmax(values) == 1


# ----------------------------------------------------------- CPU baseline


def test_cpu_baseline_agrees_with_the_oracle():
    """The numba GEMV restated in C++ (planes layout) matches the fp64 truth by tolerance."""
    cb = T.CpuBaseline()
    case = "plain7_"
    codes, x = GOLDEN[case + "codes"], GOLDEN[case + "x"]
    rows, k = codes.shape
    planes = cb.planes_of(T.pad_rows16(GOLDEN[case + "packed"]), k)
    scales = GOLDEN[case + "scales"].view(np.float16).astype(np.float32)
    bias = GOLDEN[case + "bias"]
    out = cb.gemv(np.ascontiguousarray(x), planes, scales, bias, np.zeros(rows, np.float32))
    assert_within(out, GOLDEN[case + "y64"], rtol=1e-5, atol=1e-5, what="cpu baseline")


@pytest.mark.parametrize("splits", [1, 2, 3, 8])
def test_split_order_agrees_with_fp64_truth(oracle, splits):
    case = "plain6_"
    codes, x = GOLDEN[case + "codes"], GOLDEN[case + "x"]
    rows, k = codes.shape
    packed = T.pad_rows16(GOLDEN[case + "packed"])
    scales = GOLDEN[case + "scales"]
    q8, xsum, sx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    got = oracle.gemm_split(T.EPI_STORE, q8, xsum, sx, packed, scales, None, np.zeros((1, rows), np.float32), k, rows,
                            1, splits)
    assert_within(got[0], GOLDEN[case + "y64"] - 0.0, what=f"{splits} splits")
    if splits == 1:
        seq = oracle.gemm_seq(T.EPI_STORE, q8, xsum, sx, packed, scales, None, np.zeros((1, rows), np.float32), k,
                              rows, 1)
        assert_bits_equal(got, seq, "one split is the sequential chain")


# ------------------------------------------------------- stack fast paths


def test_q8_linear_inverts_the_layout(rng):
    q = rng.integers(-127, 128, size=200)
    q8, _ = T.q8_layout(q)
    np.testing.assert_array_equal(T.q8_linear(q8, 200), q.astype(np.int8))


@pytest.mark.parametrize("case", ["plain3_", "plain6_", "plain7_"])
def test_int8_partials_match_the_packed_core(oracle, case):
    codes, x = GOLDEN[case + "codes"], GOLDEN[case + "x"]
    rows, k = codes.shape
    q8, xsum, _ = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    got = oracle.partials_i8(codes.astype(np.int8) - 1, T.q8_linear(q8[0], k))
    packed = oracle.group_partials(q8[0], xsum[0], T.pad_rows16(GOLDEN[case + "packed"]), rows, k)
    np.testing.assert_array_equal(got, packed)
    q, _ = T.quantize_closed_form(x)
    np.testing.assert_array_equal(got, T.group_partials_int64(codes, q))


@pytest.mark.parametrize("epi", [T.EPI_STORE, T.EPI_RESIDUAL, T.EPI_SILU_PAIR])
def test_finish_restates_the_kernel_orders(oracle, epi, rng):
    """orc_finish (partials -> fp32) gives the bits of orc_gemv_pairs and orc_gemm_split."""
    rows, k, m = 48, 1000, 3
    codes = rng.integers(0, 3, size=(rows, k)).astype(np.uint8)
    packed = T.pad_rows16(T.pack_codes(codes))
    scales = (np.abs(rng.normal(0, 0.02, (rows, 8))) + 1e-4).astype(np.float16).view(np.uint16)
    x = rng.standard_normal((m, k)).astype(np.float32)
    q8, xsum, sx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
    partials = np.stack([oracle.partials_i8(codes.astype(np.int8) - 1, T.q8_linear(q8[t], k)) for t in range(m)])
    width = rows // 2 if epi == T.EPI_SILU_PAIR else rows
    base = np.linspace(-1, 1, m * width).astype(np.float32).reshape(m, width)
    for lanes in (2, 4, 16, 64):
        expected = oracle.gemv_pairs(epi, q8[1], xsum[1], sx[1], packed, scales, None, base[1].copy(), k, lanes)
        got = oracle.finish(0, lanes, epi, partials[1], scales, sx[1:2], None, base[1].copy(), k, width)
        assert_bits_equal(got, expected, f"lanes {lanes}")
    for splits in (1, 2, 3, 8):
        expected = oracle.gemm_split(epi, q8, xsum, sx, packed, scales, None, base.copy(), k, width, m, splits)
        got = oracle.finish(1, splits, epi, partials, scales, sx, None, base.copy(), k, width)
        assert_bits_equal(got, expected, f"{splits} splits")
