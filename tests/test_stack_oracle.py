"""The stack oracle's wiring against an independent float64 forward of the same stack (CPU only)."""

from __future__ import annotations

import numpy as np
import pytest

import ternary_oracle as T
from ivonar_amd.synthetic import StackConfig, decoder_stack, prompt_ids
from stack_oracle import StackOracle

CONFIG = StackConfig(vocab=500, hidden=192, layers=2, dense=320)


def _lanes(rows: int, k: int) -> int:
    return 8


def _splits(m: int, rows: int, k: int) -> int:
    return 2


def _linear64(layer, x: np.ndarray) -> np.ndarray:
    """sx * sum_g P[r, g] * scale[r, g] with the closed-form fp32 quantizer and exact partials."""
    q, sx = T.quantize_closed_form(x.astype(np.float32))
    codes = T.unpack_codes(layer.packed, layer.in_features)
    partials = T.group_partials_int64(codes, q)
    return T.truth_fp64(partials, layer.scales.astype(np.float32), sx)


def _norm64(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    inv = 1.0 / np.sqrt(np.mean(x.astype(np.float64) ** 2) + eps)
    return np.clip(x * inv, -8.0, 8.0) * weight


def _forward64(weights, token: int) -> np.ndarray:
    config = weights.config
    hidden = config.hidden
    codes = T.unpack_codes(weights.token.packed, hidden)[token].astype(np.float64) - 1
    scales = np.repeat(weights.token.scales[token].astype(np.float64), 128)[:hidden]
    h = codes * scales
    for layer in weights.layers:
        mixed = _linear64(layer.qkv, _norm64(h, layer.mixer_norm, config.eps))
        h = h + _linear64(layer.out, mixed[2 * hidden:])
        x = _norm64(h, layer.ffn_norm, config.eps)
        gate, up = _linear64(layer.gate, x), _linear64(layer.up, x)
        h = h + _linear64(layer.down, gate / (1.0 + np.exp(-gate)) * up)
    return _linear64(weights.token, _norm64(h, weights.final_norm, config.eps))


@pytest.fixture(scope="module")
def stack():
    weights = decoder_stack(CONFIG, seed=7)
    return weights, StackOracle(weights, _lanes, _splits)


@pytest.mark.parametrize("token", [2, 77, 499])
def test_step_logits_follow_the_float64_forward(stack, token):
    weights, oracle = stack
    got = oracle.step_logits(token)
    truth = _forward64(weights, token)
    scale = np.abs(truth).max()
    assert np.abs(got - truth).max() <= 2e-3 * scale
    # and the tile order gives the same logits up to fp32 rounding
    tile = oracle.prefill_logits([5, token])
    assert np.abs(tile - got).max() <= 1e-4 * scale


def test_planted_wiring_mistake_is_caught(stack):
    """Swapping gate and up in the forward changes the logits far beyond the tolerance."""
    weights, oracle = stack
    layer = weights.layers[0]
    swapped = decoder_stack(CONFIG, seed=7)
    swapped.layers[0].gate, swapped.layers[0].up = layer.up, layer.gate
    truth = _forward64(weights, 77)
    wrong = _forward64(swapped, 77)
    assert np.abs(wrong - truth).max() > 2e-3 * np.abs(truth).max()


def test_generate_is_greedy(stack):
    weights, oracle = stack
    prompt = prompt_ids(CONFIG.vocab, 5, seed=3)
    tokens, logits = oracle.generate(prompt, 4, keep_logits=True)
    assert tokens == [int(np.argmax(row)) for row in logits]
    np.testing.assert_array_equal(logits[1], oracle.step_logits(tokens[0]))
