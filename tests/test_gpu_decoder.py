"""Greedy decoding of ternary linear stacks on the MI355X against the stack oracle (tokens and logits)."""

from __future__ import annotations

import numpy as np
import pytest

from ivonar_amd.synthetic import StackConfig, decoder_stack, prompt_ids

pytestmark = pytest.mark.gpu

CONFIGS = {
    "narrow": StackConfig(vocab=3000, hidden=256, layers=3, dense=768),
    "wide": StackConfig(vocab=1000, hidden=1280, layers=2, dense=2304),
    "ragged": StackConfig(vocab=700, hidden=320, layers=2, dense=448),
}


def _oracle(weights):
    from ivonar_amd import runtime
    from stack_oracle import StackOracle

    return StackOracle(weights, lambda rows, k: runtime.gemv_plan(rows, k)[0], runtime.gemm_plan)


@pytest.fixture(scope="module", params=sorted(CONFIGS))
def pair(request, cuda):
    from ivonar_amd.decoder import StackDecoder

    weights = decoder_stack(CONFIGS[request.param], seed=5, keep_codes=True)
    print(f"decoder stack {request.param}: {CONFIGS[request.param]}", flush=True)
    return StackDecoder(weights, cuda, burst=8), _oracle(weights)


@pytest.mark.parametrize("length", [1, 32, 40])
def test_prefill_logits_are_bit_exact(pair, length):
    decoder, oracle = pair
    prompt = prompt_ids(decoder.config.vocab, length, seed=length)
    logits = decoder.prefill(prompt).cpu().numpy()
    expected = oracle.prefill_logits(prompt)
    np.testing.assert_array_equal(logits, expected)
    assert int(decoder.history[decoder.burst - 1]) == oracle.oracle.argmax(expected)


def test_eager_greedy_tokens_and_logits_match(pair):
    decoder, oracle = pair
    prompt = prompt_ids(decoder.config.vocab, 36, seed=1)
    tokens = decoder.generate(prompt, 12)
    expected, logits = oracle.generate(prompt, 12, keep_logits=True)
    assert tokens == expected
    np.testing.assert_array_equal(decoder.logits.cpu().numpy(), logits[-1])


def test_graph_bursts_match_eager_steps(pair):
    import torch

    decoder, oracle = pair
    prompt = prompt_ids(decoder.config.vocab, 36, seed=2)
    decoder.prefill(prompt)
    decoder.capture()
    first = int(decoder.history[decoder.burst - 1])
    replayed = [first] + decoder.advance_many(2 * decoder.burst + 3)
    torch.cuda.synchronize()
    assert replayed == oracle.generate(prompt, len(replayed))
    # a second prefill and replay over the same graph gives the same tokens
    decoder.prefill(prompt)
    again = [int(decoder.history[decoder.burst - 1])] + decoder.advance_many(2 * decoder.burst + 3)
    assert again == replayed


def test_out_of_range_prompt_is_rejected(pair):
    decoder, _ = pair
    with pytest.raises(IndexError):
        decoder.prefill([0, decoder.config.vocab])
    with pytest.raises(ValueError):
        decoder.prefill([])


def test_full_size_stack_greedy_tokens_are_identical(cuda):
    """24 layers, d=1024, ffn 4096, vocab 32000, 36-token prompt, 256 greedy tokens through graph bursts."""
    from ivonar_amd.decoder import StackDecoder

    config = StackConfig()
    weights = decoder_stack(config, seed=1, keep_codes=True)
    prompt = prompt_ids(config.vocab, 36, seed=1)
    decoder = StackDecoder(weights, cuda, burst=16)
    decoder.prefill(prompt)
    decoder.capture()
    tokens = decoder.generate(prompt, 256)
    last_logits = decoder.logits.cpu().numpy()
    del decoder
    expected, logits = _oracle(weights).generate(prompt, 256, keep_logits=True)
    assert tokens == expected
    np.testing.assert_array_equal(last_logits, logits[-1])
