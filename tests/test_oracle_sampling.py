"""Logit processing and token selection of the oracle (oracle/sampling.py), pinned by closed
forms, brute force over tiny vocabularies, and the reference's stated rules
(kernels.rs:176-221, 248-263, 408-426; sampling.rs:57-118)."""
import itertools

import numpy as np
import pytest

from oracle import sampling as S


def test_argmax_ties_take_lowest_index():
    assert S.argmax_lowest(np.array([1.0, 3.0, 3.0, 2.0])) == 1
    assert S.argmax_lowest(np.array([-np.inf, -1.0, -np.inf])) == 1


def test_suppression_mask():
    V, eos = 3072, 2150
    out = S.suppress(np.zeros(V), eos)
    assert np.all(out[:V - 1024] == 0)
    assert out[eos] == 0
    masked = np.ones(V, bool)
    masked[:V - 1024] = False
    masked[eos] = False
    assert np.all(np.isneginf(out[masked]))


def test_repetition_penalty_once_per_distinct_token():
    l = np.array([2.0, -2.0, 1.0, 0.5])
    out = S.apply_repetition_penalty(l, [0, 1, 0, 0], 2.0)
    np.testing.assert_array_equal(out, [1.0, -4.0, 1.0, 0.5])
    # penalty 1 or empty history: unchanged
    np.testing.assert_array_equal(S.apply_repetition_penalty(l, [0], 1.0), l)
    np.testing.assert_array_equal(S.apply_repetition_penalty(l, [], 2.0), l)


def test_repetition_penalty_per_occurrence_compounds():
    """The crate's GPU kernel applies the penalty once per history entry (kernels.rs:408-426):
    a token seen three times is divided (positive) or multiplied (negative) three times."""
    l = np.array([8.0, -2.0, 1.0, 0.5, 3.0])
    hist = [0, 1, 0, 0, 4, 9, -1]          # out-of-range ids are skipped, as in the kernel
    out = S.apply_repetition_penalty(l, hist, 2.0, per_occurrence=True)
    np.testing.assert_array_equal(out, [1.0, -4.0, 1.0, 0.5, 1.5])
    once = S.apply_repetition_penalty(l, hist, 2.0)
    np.testing.assert_array_equal(once, [4.0, -4.0, 1.0, 0.5, 1.5])
    # a history without repeats gives the same result under both rules
    np.testing.assert_array_equal(S.apply_repetition_penalty(l, [0, 1, 4], 1.3, per_occurrence=True),
                                  S.apply_repetition_penalty(l, [0, 1, 4], 1.3))
    # the order of the history does not matter (each token's logit sees only its own entries)
    np.testing.assert_array_equal(S.apply_repetition_penalty(l, [0, 0, 1, 0, 4], 1.7, per_occurrence=True),
                                  S.apply_repetition_penalty(l, [4, 0, 1, 0, 0], 1.7, per_occurrence=True))


def _brute_distribution(logits, k, p, T):
    """Enumerate the kept set from the definitions, independently of kept_distribution."""
    idx = sorted(range(len(logits)), key=lambda i: (-logits[i], i))
    idx = [i for i in idx if np.isfinite(logits[i])]
    if 0 < k < len(idx):
        idx = idx[:k]
    w = np.array([np.exp((logits[i] - logits[idx[0]]) / T) for i in idx])
    if p < 1.0:
        for m in range(1, len(idx) + 1):
            if w[:m].sum() / w.sum() >= p:
                idx, w = idx[:m], w[:m]
                break
    return idx, w / w.sum()


@pytest.mark.parametrize("k,p,T", [(0, 1.0, 1.0), (3, 1.0, 0.7), (0, 0.6, 1.3), (4, 0.8, 0.9), (1, 1.0, 2.0)])
def test_kept_distribution_matches_brute_force(k, p, T):
    rng = np.random.default_rng(k * 10 + int(p * 10))
    logits = rng.standard_normal(9)
    logits[2] = -np.inf
    tokens, probs = S.kept_distribution(logits, S.SamplingConfig(True, k, p, T))
    bt, bp = _brute_distribution(logits, k, p, T)
    assert list(tokens) == bt
    np.testing.assert_allclose(probs / probs.sum(), bp, rtol=1e-12)


def test_inverse_cdf_selects_by_interval():
    logits = np.log(np.array([0.5, 0.3, 0.2]))
    cfg = S.SamplingConfig(True, 0, 1.0, 1.0)
    assert S.sample(logits, cfg, 0.0) == 0
    assert S.sample(logits, cfg, 0.49) == 0
    assert S.sample(logits, cfg, 0.51) == 1
    assert S.sample(logits, cfg, 0.79) == 1
    assert S.sample(logits, cfg, 0.81) == 2
    assert S.sample(logits, cfg, 0.999999) == 2


def test_sampling_frequencies_match_closed_form():
    """Chi-square of 20k draws with a stratified u grid against p_i ~ exp(l_i / T)."""
    logits = np.array([1.0, 0.2, -0.5, 0.9, -3.0, 0.0])
    cfg = S.SamplingConfig(True, 4, 1.0, 0.8)
    n = 20000
    draws = [S.sample(logits, cfg, (i + 0.5) / n) for i in range(n)]
    tokens, probs = S.kept_distribution(logits, cfg)
    counts = np.array([draws.count(t) for t in tokens])
    expected = probs / probs.sum() * n
    assert set(draws) <= set(int(t) for t in tokens)
    assert np.all(np.abs(counts - expected) <= 1.0)   # stratified u: exact up to one draw


def test_validation_rules():
    S.SamplingConfig(True, 50, 1.0, 0.9).validate("t")
    for bad in [S.SamplingConfig(True, 50, 0.0, 0.9), S.SamplingConfig(True, 50, 1.1, 0.9),
                S.SamplingConfig(True, 50, 1.0, 0.0)]:
        with pytest.raises(ValueError):
            bad.validate("t")


def test_top2_margin():
    assert S.top2_margin(np.array([0.1, 0.5, 0.45, -np.inf])) == pytest.approx(0.05)
