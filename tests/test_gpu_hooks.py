"""The reference's own parity seams, through the C ABI hooks, against float64-oracle fixtures
with the reference's array names and tolerances:
  talker-prefill-parity.rs:41-110  prefill: token exact, normed hidden max 2e-3 / mean 2e-4,
                                   logits max 5e-3 / mean 5e-4; then one decode step at
                                   offset P from `first_step_input`, same logit bounds;
  code-predictor-parity.rs:21-47   deterministic_hidden(H, 17, 15) / (H, 23, 11) prefix:
                                   tokens exact, embedding_sum max 2e-3 / mean 2e-4.
A token may differ only where the oracle's top-2 margin is below the near-tie tolerance.
"""
import numpy as np
import pytest

from q3t import engine as E
from q3t.workloads import WORKLOADS

from parity import TIE_TOL, fixture_exists, load_fixture

pytestmark = pytest.mark.gpu

SPECS = ["tiny", "tiny-proj", "0.6b", "1.7b"]
HOOK_WORKLOADS = {"tiny": "tiny_greedy", "tiny-proj": "tinyproj_greedy", "0.6b": "cfg2_0.6b_greedy",
                  "1.7b": "cfg4_1.7b_greedy"}


def close(got, want, max_tol, mean_tol, what):
    d = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))
    print(f"  {what}: max {d.max():.2e} mean {d.mean():.2e}")
    assert d.max() <= max_tol and d.mean() <= mean_tol, f"{what}: max {d.max():.3g} mean {d.mean():.3g}"


def same_tokens(got, want, margins, what):
    got, want = np.asarray(got).ravel(), np.asarray(want).ravel()
    bad = np.nonzero(got != want)[0]
    if bad.size:
        i = int(bad[0])
        assert margins[i] < TIE_TOL, f"{what}[{i}]: GPU {got[i]} vs oracle {want[i]} (margin {margins[i]:.3g})"


@pytest.fixture(scope="module", params=SPECS)
def hook_case(request, models):
    spec = request.param
    if not fixture_exists(f"hooks_{spec}"):
        pytest.skip(f"hooks_{spec} fixture not generated")
    fx = load_fixture(f"hooks_{spec}")
    w = WORKLOADS[HOOK_WORKLOADS[spec]]
    model, d = models.get(w.spec, w.weight_seed)
    assert model.checksum() == fx["meta"]["checksum"]
    print(f"[gpu] hooks {spec}", flush=True)
    eng = E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=w.max_cache_steps))
    yield spec, fx, eng, model
    eng.close()


def test_talker_prefill_and_step(hook_case):
    spec, fx, eng, _ = hook_case
    hidden, logits, tok = eng.debug_talker_prefill(fx["prefill"])
    close(hidden, fx["last_hidden"], 2e-3, 2e-4, f"{spec} prefill hidden")
    close(logits, fx["logits"], 5e-3, 5e-4, f"{spec} prefill logits")
    same_tokens([tok], fx["first_semantic"], fx["talker_margins"][:1], "first_semantic")
    P = int(fx["meta"]["prefill_steps"])
    _, next_logits, next_tok = eng.debug_talker_step(fx["first_step_input"], P)
    close(next_logits, fx["forward_next_logits"], 5e-3, 5e-4, f"{spec} decode-step logits")
    same_tokens([next_tok], fx["next_semantic"], fx["talker_margins"][1:], "next_semantic")


def test_code_predictor_deterministic_prefix(hook_case):
    spec, fx, eng, _ = hook_case
    tokens, emb = eng.debug_code_predictor(fx["talker_hidden"], fx["semantic_embed"])
    same_tokens(tokens, fx["acoustic_tokens"], fx["acoustic_margins"], "acoustic_tokens")
    if np.array_equal(tokens, fx["acoustic_tokens"]):
        close(emb, fx["embedding_sum"], 2e-3, 2e-4, f"{spec} embedding_sum")


def test_code_predictor_first_frame(hook_case):
    """The CodePredictor of frame 0 from the prefill's own prefix [hidden ; codec_emb[token]]."""
    spec, fx, eng, model = hook_case
    hidden, _, tok = eng.debug_talker_prefill(fx["prefill"])
    if tok != int(fx["first_semantic"][0]):
        pytest.skip("first semantic token is a near tie")
    sem_embed = model.f32("talker.model.codec_embedding.weight")[tok]
    tokens, _ = eng.debug_code_predictor(hidden, sem_embed)
    same_tokens(tokens, fx["first_acoustic"], fx["first_cp_margins"], "first_acoustic")


def test_hooks_need_a_free_slot(models):
    w = WORKLOADS["tiny_greedy"]
    model, d = models.get(w.spec, w.weight_seed)
    with E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=w.max_cache_steps)) as eng:
        st = eng.start_stream(w.inputs(model), E.GenerateOptions.greedy(4))
        with pytest.raises(E.BusyError):
            eng.debug_code_predictor(np.zeros(512, np.float32), np.zeros(512, np.float32))
        st.close()
        with pytest.raises(E.CapacityError):
            eng.debug_talker_step(np.zeros(512, np.float32), w.max_cache_steps)


def test_kernel_timing_hook_covers_every_class(models):
    """q3t_bench_kernel (the roofline report's timer) runs every kernel class of the 0.6B model
    as a captured graph and reports a positive time and the algorithmic bytes of one launch."""
    w = WORKLOADS["cfg2_0.6b_greedy"]
    _, d = models.get(w.spec, w.weight_seed)
    with E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=w.max_cache_steps)) as eng:
        for k, name in E.HipTtsEngine.KERNELS.items():
            us, b = eng.bench_kernel(k, 64)
            print(f"  class {k} {name}: {us:.3f} us, {b:.0f} B")
            assert 0.0 < us < 1000.0 and b > 0.0, name
        # class 2 sums the fused projection's 8 per-head partials in its 75 CodePredictor launches
        _, b2 = eng.bench_kernel(2, 103)
        assert b2 > 2 * 2 * 3072 * 1024
        with pytest.raises(E.Q3tError):
            eng.bench_kernel(11, 8)


def test_eager_engine_captures_no_graph(models):
    """An engine created with use_graph = False (the form profiled under a kernel tracer)
    refuses the graph-timed kernel hook and still runs the eagerly timed one."""
    w = WORKLOADS["cfg2_0.6b_greedy"]
    _, d = models.get(w.spec, w.weight_seed)
    with E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=w.max_cache_steps, use_graph=False)) as eng:
        with pytest.raises(E.InvalidInputError, match="without graphs"):
            eng.bench_kernel(2, 8)
        us, b = eng.bench_kernel_timed(2, 8)
        assert us > 0 and b > 0
        r = eng.dominant_kernel_roofline(8000.0, iters=8, graph=False)
        assert r["graph_us_per_launch"] is None and r["avg_launch_us"] > 0


def test_phase_timing_and_profiled_rollout_take_the_split_attention(models):
    """Talker steps at positions from 192 on take the split attention + merging O projection
    (q3t_engine_set_fused_attention_rows), also when each frame's phases are timed as their own
    graphs (q3t_debug_phase_times) and in the profiled rollout: a prompt of 190 rows crosses
    that position in its third frame, and every path yields the same codes."""
    model, d = models.get("tiny")
    prompt = np.random.default_rng(3).integers(0, 151643, 181)
    from q3t import textprep
    inputs = textprep.TextPrep(model).prepare(prompt)
    assert inputs.prefill_steps == 190
    opts = E.GenerateOptions.greedy(8)
    print("[gpu] split attention in phase timing and profiled rollout", flush=True)
    with E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=320)) as eng:
        with pytest.raises(E.InvalidInputError):
            eng.set_fused_attention_rows(-1)
        ref = eng.generate_codes(inputs, opts).codes
        with eng.start_stream(inputs, opts) as st:
            timed = []
            while True:
                c, cp_us, tk_us = st.next_codes_chunk_timed(3)
                if c is None:
                    break
                assert len(cp_us) == len(tk_us) == c.frames and (tk_us > 0).all()
                timed.append(c.codes)
        prof = eng.generate_codes_profiled(inputs, opts)
        eng.set_fused_attention_rows(1 << 20)  # fused at every position
        fused = eng.generate_codes(inputs, opts).codes
    np.testing.assert_array_equal(np.concatenate(timed), ref)
    np.testing.assert_array_equal(prof.codes.codes, ref)
    np.testing.assert_array_equal(fused, ref)

