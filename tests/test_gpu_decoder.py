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


@pytest.mark.parametrize("name", ["narrow", "ragged"])
def test_sampled_tokens_match_the_oracle(cuda, name):
    """Sampling (temperature 0.8, top_k 40, repetition penalty 1.3, two penalized ids): the first token
    after the prompt, two graph bursts and three eager steps, each drawn with the uniform the device
    generated, against the oracle's draws with the same uniforms."""
    import torch

    from ivonar_amd.decoder import StackDecoder

    weights = decoder_stack(CONFIGS[name], seed=6, keep_codes=True)
    decoder = StackDecoder(weights, cuda, burst=8, sampling=True, max_top_k=64)
    decoder.configure_sampling(temperature=0.8, top_k=40, repetition_penalty=1.3, penalized_ids=[3, 17, -1])
    prompt = prompt_ids(decoder.config.vocab, 36, seed=3)
    decoder.prefill(prompt)
    uniforms = [float(decoder.uniforms[decoder.burst - 1])]
    tokens = [int(decoder.history[decoder.burst - 1])]
    decoder.capture()
    decoder.drawn_uniforms.clear()
    tokens += decoder.advance_many(2 * decoder.burst + 3)
    uniforms += decoder.drawn_uniforms
    torch.cuda.synchronize()
    assert len(set(uniforms)) == len(uniforms)
    expected = _oracle(weights).generate_sampled(prompt, uniforms, 0.8, 40, 1.3, [3, 17, -1], max_top_k=64)
    assert tokens == expected
    seen = np.flatnonzero(decoder.sampler.seen.cpu().numpy().reshape(-1))
    assert set(seen.tolist()) == {3, 17} | set(tokens)


def test_prefill_tile_graph_matches_the_oracle(pair):
    """After capture() every 32-token tile of a prefill is one replay of the captured tile program: the
    logits stay bit-exact for prompts of 40, 1 and 32 tokens (two replays, then one, with eager decode steps
    between), and greedy steps after a graph prefill give the oracle's tokens."""
    decoder, oracle = pair
    decoder.prefill(prompt_ids(decoder.config.vocab, 8, seed=9))
    decoder.capture()
    assert decoder._tile_graph is not None
    for length in (40, 1, 32):
        prompt = prompt_ids(decoder.config.vocab, length, seed=100 + length)
        logits = decoder.prefill(prompt).cpu().numpy()
        np.testing.assert_array_equal(logits, oracle.prefill_logits(prompt), err_msg=f"prompt of {length}")
        first = int(decoder.history[decoder.burst - 1])
        assert [first] + decoder.advance_many(3) == oracle.generate(prompt, 4)


def test_self_check_passes_and_resets(pair):
    """The load-time self-check (kernel_decoder.py:524-549): the prompt through the tile GEMMs and through
    single GEMV steps agree; afterwards the decoder is at position 0 with an empty ring and still gives the
    oracle's logits."""
    decoder, oracle = pair
    decoder.self_check()
    assert decoder.position == 0
    assert int(decoder.history.abs().sum()) == 0
    prompt = prompt_ids(decoder.config.vocab, 33, seed=21)
    np.testing.assert_array_equal(decoder.prefill(prompt).cpu().numpy(), oracle.prefill_logits(prompt))


def test_self_check_refuses_invalid_or_disagreeing_results(pair, monkeypatch):
    """Failures forced from the host: a prefill whose logits are not finite, then single steps whose logits
    are scaled away from the prefill's, each raise KernelError with the reference's message."""
    import torch
    from ivonar_amd.runtime import KernelError

    decoder, _ = pair
    real_prefill, real_step = decoder.prefill, decoder.step

    def nan_prefill(ids):
        out = real_prefill(ids)
        out.fill_(float("nan"))
        return out

    monkeypatch.setattr(decoder, "prefill", nan_prefill)
    with pytest.raises(KernelError, match="invalid numbers"):
        decoder.self_check()
    monkeypatch.setattr(decoder, "prefill", real_prefill)

    def scaled_step():
        real_step()
        decoder.logits.mul_(torch.tensor(3.0, device=decoder.logits.device))

    monkeypatch.setattr(decoder, "step", scaled_step)
    with pytest.raises(KernelError, match="disagree"):
        decoder.self_check()
    monkeypatch.setattr(decoder, "step", real_step)
    decoder.self_check()
