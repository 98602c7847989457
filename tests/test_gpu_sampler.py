"""The fused GPU sampler (top-k / temperature / top-p / Philox), through q3t_sampler_draw.

* 10k draws from fixed logits: chi-square against the closed-form distribution
  p_i ~ exp((l_i - l_max) / T) over the kept set (BASELINE config 3 settings and variants);
* draw-for-draw agreement with the oracle's sampler fed the same Philox uniforms;
* greedy mode is the lowest-index argmax.
"""
import numpy as np
import pytest
from scipy import stats

from oracle import philox
from oracle import sampling as S
from q3t import engine as E
from q3t.workloads import WORKLOADS

pytestmark = pytest.mark.gpu

N_DRAWS = 10000


@pytest.fixture(scope="module")
def eng(models):
    w = WORKLOADS["tiny_greedy"]
    _, d = models.get(w.spec)
    e = E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=64))
    yield e
    e.close()


def _logits(V, seed):
    return (np.random.default_rng(seed).standard_normal(V) * 0.64).astype(np.float32)


@pytest.mark.parametrize("V,top_k,top_p,T", [
    (3072, 50, 1.0, 0.9),     # config 3 Talker
    (2048, 50, 1.0, 0.9),     # config 3 CodePredictor
    (3072, 0, 0.8, 1.0),      # nucleus only
    (2048, 20, 0.7, 0.6),
    (2048, 2048, 1.0, 1.3),   # top_k = V keeps every candidate
])
def test_draws_follow_closed_form(eng, V, top_k, top_p, T):
    logits = _logits(V, V + top_k)
    print(f"[gpu] sampler V={V} k={top_k} p={top_p} T={T}", flush=True)
    draws = eng.sampler_draw(logits, N_DRAWS, True, top_k, top_p, T, seed=123, kind=1)
    cfg = S.SamplingConfig(True, top_k, top_p, T)
    tokens, probs = S.kept_distribution(logits.astype(np.float64), cfg)
    assert set(np.unique(draws)) <= set(tokens.tolist())
    counts = np.array([(draws == t).sum() for t in tokens])
    expected = probs / probs.sum() * N_DRAWS
    # pool the tail so every cell expects >= 5 draws
    order = np.argsort(-expected)
    e_sorted, c_sorted = expected[order], counts[order]
    keep = e_sorted >= 5
    e_cells = np.append(e_sorted[keep], e_sorted[~keep].sum())
    c_cells = np.append(c_sorted[keep], c_sorted[~keep].sum())
    if e_cells[-1] == 0:
        e_cells, c_cells = e_cells[:-1], c_cells[:-1]
    p = stats.chisquare(c_cells, e_cells).pvalue
    print(f"chi-square p = {p:.3g} over {len(e_cells)} cells")
    assert p > 1e-3

    # the same Philox uniforms through the oracle's sampler
    want = np.array([S.sample(logits.astype(np.float64), cfg, philox.sampler_uniform(123, i, 1))
                     for i in range(2000)])
    agree = np.mean(want == draws[:2000])
    assert agree >= 0.999, agree


def test_greedy_is_lowest_index_argmax(eng):
    logits = _logits(3072, 5)
    logits[100] = logits[2000] = logits.max() + 1.0
    out = eng.sampler_draw(logits, 4, do_sample=False)
    assert out.tolist() == [100] * 4


@pytest.mark.parametrize("V,top_k,top_p,T", [(3072, 1, 1.0, 0.9), (2048, 0, 1e-6, 1.0), (3072, 50, 1e-6, 0.7)])
def test_degenerate_settings_draw_the_argmax(eng, V, top_k, top_p, T):
    """top_k = 1, or a nucleus smaller than the top candidate's probability, leaves one
    candidate: every draw is the argmax."""
    logits = _logits(V, 17 + top_k)
    draws = eng.sampler_draw(logits, 500, True, top_k, top_p, T, seed=7)
    assert set(draws.tolist()) == {int(np.argmax(logits))}


def test_masked_logits_never_drawn(eng):
    logits = _logits(3072, 9)
    logits[2048:] = -np.inf
    draws = eng.sampler_draw(logits, 2000, True, 0, 1.0, 2.0, seed=1)
    assert draws.max() < 2048


@pytest.mark.parametrize("V,top_k,top_p,T,mode", [
    (2048, 50, 1.0, 0.9, "gauss"),   # config 3 CodePredictor settings
    (2048, 64, 0.8, 0.7, "ties"),    # ties, -inf, signed zeros, -FLT_MAX
    (2048, 1, 1.0, 1.0, "ties"),
    (1000, 50, 0.9, 0.9, "sparse"),  # fewer finite logits than top_k
])
def test_top64_path_equals_radix_path(eng, V, top_k, top_p, T, mode):
    """Top-k of at most 64 over at most 2048 logits takes the sort-and-merge sampler; the same
    logits padded with -inf to 2049 entries take the radix-select sampler.  The candidates,
    their order and the inverse CDF are the same, so every draw must agree."""
    rng = np.random.default_rng(V + top_k)
    logits = (rng.standard_normal(V) * 3).astype(np.float32)
    if mode == "ties":
        r = rng.integers(0, 16, V)
        logits[r == 0] = -np.inf
        logits[r == 1] = 1.5
        logits[r == 2] = np.where(rng.integers(0, 2, (r == 2).sum()) == 1, 0.0, -0.0)
        logits[r == 3] = -np.finfo(np.float32).max
    elif mode == "sparse":
        logits[np.arange(V) % 37 != 0] = -np.inf
    padded = np.concatenate([logits, np.full(2049 - V, -np.inf, np.float32)])
    print(f"[gpu] sampler paths V={V} k={top_k} p={top_p} T={T} {mode}", flush=True)
    fast = eng.sampler_draw(logits, 4096, True, top_k, top_p, T, seed=77, kind=2)
    radix = eng.sampler_draw(padded, 4096, True, top_k, top_p, T, seed=77, kind=2)
    np.testing.assert_array_equal(fast, radix)
