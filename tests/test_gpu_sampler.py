"""The device sampler (logit_bounds + sample_token) against the sampling oracle: tokens, seen flags,
history and bounds bit for bit, and the reference's own distribution test."""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _sampler(cuda, vocab: int, max_top_k: int = 1024):
    from ivonar_amd.sampling import DeviceSampler

    return DeviceSampler(vocab, cuda, max_top_k=max_top_k)


def _logits(rng, vocab: int, kind: str) -> np.ndarray:
    if kind == "ties":  # integer values: ties everywhere, including at the top-k cut
        return rng.integers(-4, 5, size=vocab).astype(np.float32)
    if kind == "flat":  # one value everywhere: more candidates than the LDS list holds
        return np.full(vocab, 0.25, np.float32)
    return (rng.standard_normal(vocab) * 3).astype(np.float32)


def _draw(sampler, logits_t, seen_np, temperature, penalty, top_k, u, history=None):
    import torch

    sampler.temperature.fill_(float(temperature))
    sampler.penalty.fill_(float(penalty))
    sampler.inverse_penalty.fill_(float(np.float32(1.0) / np.float32(penalty)))
    sampler.top_k.fill_(int(top_k))
    sampler.seen.copy_(torch.from_numpy(seen_np.astype(bool)).reshape(1, -1))
    sampler.uniform.fill_(float(u))
    sampler.launch(logits_t, history=history)
    torch.cuda.synchronize()
    return int(sampler.token[0]), sampler.seen.cpu().numpy().reshape(-1).astype(np.uint8)


@pytest.mark.parametrize("kind", ["normal", "ties"])
@pytest.mark.parametrize("top_k", [1, 2, 40, 256, 1024])
@pytest.mark.parametrize("vocab", [1, 7, 64, 65, 300, 4097, 32000, 262144])
def test_draws_match_the_oracle(cuda, oracle, vocab, top_k, kind):
    import torch

    rng = np.random.default_rng(vocab * 7 + top_k)
    print(f"sampler vocab={vocab} top_k={top_k} kind={kind}", flush=True)
    sampler = _sampler(cuda, vocab)
    logits = _logits(rng, vocab, kind)
    logits_t = torch.from_numpy(logits).to(cuda)
    seen = (rng.random(vocab) < 0.1).astype(np.uint8)
    temperature, penalty = 0.7, 1.4
    inverse = np.float32(1.0) / np.float32(penalty)
    bounds = oracle.logit_bounds(logits, seen, np.float32(temperature), np.float32(penalty), inverse)
    for u in (0.0, 0.1234, 0.5, 0.9, 0.99999, 1.0):
        history = torch.full((1,), -1, dtype=torch.int64, device=cuda)
        token, seen_after = _draw(sampler, logits_t, seen, temperature, penalty, top_k, u, history)
        np.testing.assert_array_equal(sampler.bounds.cpu().numpy(), bounds)
        expected_seen = seen.copy()
        expected, _, _ = oracle.sample_token(logits, expected_seen, np.float32(temperature), np.float32(penalty),
                                             inverse, top_k, 1024, np.float32(u))
        assert token == expected, (u, token, expected)
        assert int(history[0]) == expected
        np.testing.assert_array_equal(seen_after, expected_seen)


@pytest.mark.parametrize("vocab,top_k", [(32000, 40), (5000, 1024), (262144, 8)])
def test_flat_logits_take_the_lowest_indices(cuda, oracle, vocab, top_k):
    """Every score equal: the candidate list overflows LDS and the picks are the k lowest indices."""
    import torch

    sampler = _sampler(cuda, vocab)
    logits = _logits(None, vocab, "flat")
    logits_t = torch.from_numpy(logits).to(cuda)
    seen = np.zeros(vocab, np.uint8)
    for u in (0.0, 0.37, 0.999):
        token, _ = _draw(sampler, logits_t, seen, 1.0, 1.0, top_k, u)
        expected, picks, _ = oracle.sample_token(logits, seen.copy(), np.float32(1.0), np.float32(1.0),
                                                 np.float32(1.0), top_k, 1024, np.float32(u))
        assert list(picks) == list(range(top_k))
        assert token == expected


def test_special_values(cuda, oracle):
    import torch

    vocab = 1000
    sampler = _sampler(cuda, vocab)
    cases = {
        "all -inf": np.full(vocab, -np.inf, np.float32),
        "one finite": np.where(np.arange(vocab) == 613, 2.0, -np.inf).astype(np.float32),
        "+inf present": np.where(np.arange(vocab) % 97 == 5, np.inf, 0.0).astype(np.float32),
        "large": (np.random.default_rng(0).standard_normal(vocab) * 1e30).astype(np.float32),
        "signed zeros": np.where(np.arange(vocab) % 2 == 0, 0.0, -0.0).astype(np.float32),
    }
    for name, logits in cases.items():
        logits_t = torch.from_numpy(logits).to(cuda)
        for top_k in (1, 5, 300):
            for u in (0.0, 0.6):
                token, _ = _draw(sampler, logits_t, np.zeros(vocab, np.uint8), 1.0, 1.0, top_k, u)
                expected, _, _ = oracle.sample_token(logits, np.zeros(vocab, np.uint8), np.float32(1.0),
                                                     np.float32(1.0), np.float32(1.0), top_k, 1024, np.float32(u))
                assert token == expected, (name, top_k, u)


def test_top_k_is_clamped_by_max_topk(cuda, oracle):
    import torch

    from ivonar_amd import runtime

    vocab = 3000
    rng = np.random.default_rng(4)
    logits = _logits(rng, vocab, "normal")
    logits_t = torch.from_numpy(logits).to(cuda)
    sampler = _sampler(cuda, vocab, max_top_k=16)
    try:
        for top_k, u in [(40, 0.99), (0, 0.5), (-3, 0.2), (1 << 40, 0.7)]:
            token, _ = _draw(sampler, logits_t, np.zeros(vocab, np.uint8), 1.0, 1.0, top_k, u)
            expected, _, _ = oracle.sample_token(logits, np.zeros(vocab, np.uint8), np.float32(1.0),
                                                 np.float32(1.0), np.float32(1.0), top_k, 16, np.float32(u))
            assert token == expected, (top_k, u)
    finally:
        runtime.check(runtime.library().ivonar_define(b"MAX_TOPK", 256), "define MAX_TOPK")


def test_sample_token_follows_the_top_k_distribution(cuda):
    """Reference tests/test_kernels.py:131-161 with the device's own uniform_()."""
    import torch

    torch.manual_seed(21)
    vocab = 300
    sampler = _sampler(cuda, vocab, max_top_k=16)
    logits = torch.randn(vocab, device=cuda) * 3
    sampler.configure_sampling(temperature=0.7, top_k=8, repetition_penalty=1.0)
    draws = 4000
    counts = torch.zeros(vocab)
    for _ in range(draws):
        sampler.seen.zero_()
        counts[sampler.sample(logits)] += 1
    values, indices = torch.topk(logits / 0.7, 8)
    expected = torch.softmax(values, dim=0).cpu()
    assert counts.sum() == draws
    assert counts[[i for i in range(vocab) if i not in indices.tolist()]].sum() == 0
    frequencies = counts[indices.cpu()] / draws
    tolerance = 5 * (expected * (1 - expected) / draws).sqrt() + 0.005
    assert bool(((frequencies - expected).abs() <= tolerance).all())
    sampler.configure_sampling(temperature=0.7, top_k=8, repetition_penalty=2.0, penalized_ids=[int(indices[0])])
    penalized = 0
    for _ in range(draws):
        sampler.seen.zero_()
        sampler.seen[0, int(indices[0])] = True
        penalized += int(sampler.sample(logits) == int(indices[0]))
    assert penalized / draws < float(expected[0]) * 0.8
    sampler.configure_sampling(temperature=1.0, top_k=1, repetition_penalty=1.0)
    assert sampler.sample(logits) == int(indices[0])


def test_greedy_penalty_known_answer(cuda):
    """Reference tests/test_decoder.py:128-139."""
    import torch

    sampler = _sampler(cuda, 40, max_top_k=8)
    logits = torch.zeros(40, device=cuda)
    logits[5], logits[9] = 6.0, 5.0
    sampler.configure_sampling(temperature=1.0, top_k=1, repetition_penalty=1.5)
    assert sampler.sample(logits) == 5
    assert bool(sampler.seen[0, 5]) and not bool(sampler.seen[0, 9])
    assert sampler.sample(logits) == 9
    sampler.configure_sampling(temperature=1.0, top_k=1, repetition_penalty=1.0)
    assert sampler.sample(logits) == 5


def test_sampler_in_a_graph_replays_fresh_draws(cuda, oracle):
    """uniform_() + both launches captured once; every replay draws a new uniform, and each token is the
    oracle's for that replay's uniform and seen set."""
    import torch

    vocab = 32000
    rng = np.random.default_rng(9)
    logits = _logits(rng, vocab, "normal")
    logits_t = torch.from_numpy(logits).to(cuda)
    sampler = _sampler(cuda, vocab, max_top_k=256)
    sampler.configure_sampling(temperature=0.9, top_k=40, repetition_penalty=1.2)
    stream = torch.cuda.Stream()

    def step():
        sampler.uniform.uniform_()
        sampler.launch(logits_t)

    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        step()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step()
    torch.cuda.synchronize()
    sampler.seen.zero_()
    seen = np.zeros(vocab, np.uint8)
    uniforms = set()
    for _ in range(6):
        graph.replay()
        torch.cuda.synchronize()
        u = float(sampler.uniform[0])
        uniforms.add(u)
        expected, _, _ = oracle.sample_token(logits, seen, np.float32(0.9), np.float32(1.2),
                                             np.float32(1.0 / 1.2), 40, 256, np.float32(u))
        assert int(sampler.token[0]) == expected
        np.testing.assert_array_equal(sampler.seen.cpu().numpy().reshape(-1).astype(np.uint8), seen)
    assert len(uniforms) == 6
