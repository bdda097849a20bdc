"""The sampler oracle (logit_bounds / sample_token rule) pinned on the CPU.

Checks are chosen so that a plausible mistake fails one of them:
- the reference's own known answers (tests/test_decoder.py:128-155 and tests/test_kernels.py:131-161 of
  the reference: greedy with a repetition penalty, top_k covering a candidate set, the top-k
  distribution at temperature 0.7);
- the top-k set and its order against a brute-force sort;
- the inverse-CDF intervals against float64 softmax probabilities;
- the draw against searchsorted on the oracle's own CDF, and the bounds against numpy maxima.
"""

from __future__ import annotations

import numpy as np
import pytest


def scores_of(logits, seen, temperature, penalty, inverse_penalty):
    """The reference rule in numpy float32 (ternary.cu:990-996; decoder.py:325-327)."""
    inv_t = np.float32(1.0) / np.float32(temperature)
    s = logits.astype(np.float32) * inv_t
    mult = np.where(s > 0, np.float32(inverse_penalty), np.float32(penalty)).astype(np.float32)
    return np.where(seen.astype(bool), s * mult, s).astype(np.float32)


def brute_topk(scores: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest scores, ties lowest index first, returned in ascending index order."""
    order = np.lexsort((np.arange(scores.shape[0]), -scores.astype(np.float64)))
    return np.sort(order[:k])


def sample(oracle, logits, seen, temperature=1.0, penalty=1.0, top_k=1, max_topk=256, uniform=0.5):
    return oracle.sample_token(logits, seen, temperature, penalty, np.float32(1.0) / np.float32(penalty), top_k,
                               max_topk, uniform)


def test_greedy_with_repetition_penalty_known_answer(oracle):
    """Reference tests/test_decoder.py:128-139: logits 0 except [5]=6, [9]=5."""
    logits = np.zeros(40, np.float32)
    logits[5], logits[9] = 6.0, 5.0
    seen = np.zeros(40, np.uint8)
    token, _, _ = sample(oracle, logits, seen, penalty=1.5, top_k=1)
    assert token == 5 and seen[5] == 1 and seen[9] == 0
    token, _, _ = sample(oracle, logits, seen, penalty=1.5, top_k=1)
    assert token == 9  # 6 / 1.5 = 4 < 5
    seen[:] = 0
    token, _, _ = sample(oracle, logits, seen, penalty=1.0, top_k=1)
    assert token == 5


def test_top_k_covers_the_candidate_set(oracle):
    """Reference tests/test_decoder.py:145-155: four equal logits, the rest -50, top_k = max_top_k = 4."""
    logits = np.full(40, -50.0, np.float32)
    logits[:4] = 1.0
    draws = {sample(oracle, logits, np.zeros(40, np.uint8), temperature=0.5, top_k=4, max_topk=4, uniform=u)[0]
             for u in np.linspace(0.0, 1.0, 64, dtype=np.float32)}
    assert draws == {0, 1, 2, 3}


def test_top_k_distribution_known_answer(oracle):
    """Reference tests/test_kernels.py:131-161: 300 logits ~ 3 N(0,1), temperature 0.7, top_k 8.  The
    inverse-CDF intervals are the top-8 softmax probabilities; a penalty of 2 on the favourite lowers it."""
    rng = np.random.default_rng(21)
    logits = (rng.standard_normal(300) * 3).astype(np.float32)
    _, picks, cdf = sample(oracle, logits, np.zeros(300, np.uint8), temperature=0.7, top_k=8, max_topk=16)
    scaled = logits.astype(np.float64) / 0.7
    top = np.argsort(-scaled)[:8]
    assert set(picks.tolist()) == set(top.tolist())
    expected = np.exp(scaled[picks] - scaled[top[0]])
    expected /= expected.sum()
    widths = np.diff(np.concatenate([[0.0], cdf.astype(np.float64)])) / float(cdf[-1])
    np.testing.assert_allclose(widths, expected, rtol=0, atol=2e-7)
    seen = np.zeros(300, np.uint8)
    seen[top[0]] = 1
    _, picks2, cdf2 = sample(oracle, logits, seen, temperature=0.7, penalty=2.0, top_k=8, max_topk=16)
    if top[0] in picks2:
        j = int(np.flatnonzero(picks2 == top[0])[0])
        share = (cdf2[j] - (cdf2[j - 1] if j else 0.0)) / cdf2[-1]
    else:
        share = 0.0
    assert share < expected[list(picks).index(top[0])] * 0.8
    token, _, _ = sample(oracle, logits, np.zeros(300, np.uint8), temperature=1.0, top_k=1, max_topk=16)
    assert token == int(top[0])


@pytest.mark.parametrize("vocab", [1, 7, 64, 65, 300, 1000, 4097])
@pytest.mark.parametrize("top_k", [1, 2, 8, 40, 256, 1024])
def test_picks_match_brute_force(oracle, vocab, top_k):
    rng = np.random.default_rng(vocab * 31 + top_k)
    # integer-valued logits make ties common, including at the cut
    logits = rng.integers(-6, 7, size=vocab).astype(np.float32) if top_k % 2 == 0 else \
        rng.standard_normal(vocab).astype(np.float32) * 4
    seen = (rng.random(vocab) < 0.2).astype(np.uint8)
    temperature, penalty = 0.8, 1.3
    s = scores_of(logits, seen, temperature, penalty, np.float32(1) / np.float32(penalty))
    for max_topk in (top_k, 1024):
        k = max(1, min(top_k, max_topk, vocab))
        u = float(rng.random())
        token, picks, cdf = sample(oracle, logits, seen.copy(), temperature, penalty, top_k, max_topk, u)
        np.testing.assert_array_equal(picks, brute_topk(s, k))
        assert np.all(np.diff(cdf.astype(np.float64)) >= -1e-6 * cdf[-1])
        target = np.float32(min(u, np.float32(0.99999994))) * cdf[-1]
        j = min(int(np.searchsorted(cdf, target, side="right")), k - 1)
        assert token == picks[j]


def test_scores_and_bounds(oracle):
    rng = np.random.default_rng(3)
    logits = rng.standard_normal(1000).astype(np.float32) * 5
    seen = (rng.random(1000) < 0.3).astype(np.uint8)
    bounds = oracle.logit_bounds(logits, seen, 0.7, 1.7, np.float32(1) / np.float32(1.7))
    s = scores_of(logits, seen, 0.7, 1.7, np.float32(1) / np.float32(1.7))
    padded = np.concatenate([s, np.full(-len(s) % 64, -np.inf, np.float32)]).reshape(-1, 64)
    np.testing.assert_array_equal(bounds, padded.max(axis=1))
    # the penalty divides positive scores and multiplies negative ones
    one = np.array([2.0, -2.0], np.float32)
    assert oracle.logit_bounds(one[:1], np.ones(1, np.uint8), 1.0, 2.0, 0.5)[0] == 1.0
    assert oracle.logit_bounds(one[1:], np.ones(1, np.uint8), 1.0, 2.0, 0.5)[0] == -4.0


def test_draw_edges(oracle):
    rng = np.random.default_rng(5)
    logits = rng.standard_normal(500).astype(np.float32)
    picks0 = sample(oracle, logits, np.zeros(500, np.uint8), top_k=20, uniform=0.0)
    assert picks0[0] == picks0[1][0]  # u = 0: first pick
    last = sample(oracle, logits, np.zeros(500, np.uint8), top_k=20, uniform=1.0)
    assert last[0] == last[1][-1]  # u = 1 is clamped below 1: last pick
    # all -inf: every weight is NaN, the draw falls back to the last pick
    inf = np.full(100, -np.inf, np.float32)
    token, picks, _ = sample(oracle, inf, np.zeros(100, np.uint8), top_k=5, uniform=0.3)
    assert list(picks) == [0, 1, 2, 3, 4] and token == 4
    # one finite logit among -inf: it is drawn for every u
    inf[37] = 1.0
    for u in (0.0, 0.5, 0.999):
        assert sample(oracle, inf, np.zeros(100, np.uint8), top_k=5, uniform=u)[0] == 37


def test_planted_mistake_is_caught(oracle):
    """Drawing from the picks in descending-score order gives the same distribution but other tokens for
    the same u: the brute-force order check above is what tells them apart."""
    rng = np.random.default_rng(8)
    logits = rng.standard_normal(256).astype(np.float32)
    _, picks, cdf = sample(oracle, logits, np.zeros(256, np.uint8), top_k=16)
    wrong = picks[np.argsort(-logits[picks], kind="stable")]
    assert not np.array_equal(wrong, picks)
