"""GPU parity: the gfx950 token loop, through the C ABI, against the CPU oracle.

Fixtures (tests/golden/*.npz) hold float64-oracle rollouts of the workloads in
q3t/workloads.py; small variants are recomputed here with the oracle directly.
"""
import numpy as np
import pytest

from oracle.model import GenerateOptions as OracleOptions
from oracle.model import Oracle
from q3t import engine as E
from q3t import synth
from q3t.workloads import WORKLOADS

from parity import (LOGIT_TOL, check_codes, check_codes_near_tie, check_cp_logits, check_talker_logits,
                    load_fixture)

pytestmark = pytest.mark.gpu


def run(models, name, chunk=None, use_graph=True, kv_bf16=False, trace=True, options=None, inputs=None,
        model_dir=None, cap=None):
    w = WORKLOADS[name]
    model, d = models.get(w.spec, w.weight_seed)
    inputs = inputs if inputs is not None else w.inputs(model)
    opts = options or E.GenerateOptions(**w.options_kwargs())
    print(f"[gpu] {name} chunk={chunk} graph={use_graph} kv_bf16={kv_bf16}", flush=True)
    eng = E.HipTtsEngine(model_dir or d, E.EngineOptions(max_cache_steps=cap or w.max_cache_steps,
                                                         use_graph=use_graph, kv_bf16=kv_bf16))
    try:
        eng.set_trace(trace)
        st = eng.start_stream(inputs, opts)
        chunks = []
        while True:
            c = st.next_codes_chunk(chunk or w.chunk_frames)
            if c is None:
                break
            chunks.append(c)
        tl = st.talker_logits() if trace else None
        cl = st.cp_logits() if trace else None
        eos = st.ended_by_eos
        st.close()
    finally:
        eng.close()
    codes = np.concatenate([c.codes for c in chunks]) if chunks else np.zeros((0, 16), np.int32)
    return dict(codes=codes, eos=eos, talker_logits=tl, cp_logits=cl, chunks=chunks)


@pytest.mark.parametrize("name", ["tiny_greedy", "tiny_sampled", "tinyproj_greedy"])
def test_small_workloads_match_fixture(models, name):
    fx = load_fixture(name)
    model, _ = models.get(fx["meta"]["spec"], fx["meta"]["weight_seed"])
    assert model.checksum() == fx["meta"]["checksum"]
    r = run(models, name)
    same = check_codes(r["codes"], r["eos"], fx)
    err = check_talker_logits(r["talker_logits"], fx, same)
    cp_err = check_cp_logits(r["cp_logits"], fx)
    print(f"{name}: {same} frames identical, talker logit err {err:.2e}, cp logit err {cp_err:.2e}")


def test_chunking_and_generate_codes_agree(models):
    ref = run(models, "tiny_greedy", chunk=24)["codes"]
    for chunk in (1, 5, 7):
        r = run(models, "tiny_greedy", chunk=chunk, trace=False)
        np.testing.assert_array_equal(r["codes"], ref)
        sizes = [c.frames for c in r["chunks"]]
        assert all(s == chunk for s in sizes[:-1]) and 0 < sizes[-1] <= chunk
        assert [c.total_frames for c in r["chunks"]] == list(np.cumsum(sizes))
    w = WORKLOADS["tiny_greedy"]
    model, d = models.get(w.spec)
    with E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=w.max_cache_steps)) as eng:
        g = eng.generate_codes(w.inputs(model), E.GenerateOptions(**w.options_kwargs()))
    np.testing.assert_array_equal(g.codes, ref)
    assert g.frames == len(ref) and not g.ended_by_eos


@pytest.mark.parametrize("name", ["tiny_greedy", "tiny_sampled"])
def test_generate_codes_profiled(models, name):
    """generate_codes_profiled (generation.rs:395-419): the same codes as generate_codes, and
    a time for every phase the device measures."""
    w = WORKLOADS[name]
    model, d = models.get(w.spec)
    opts = E.GenerateOptions(**w.options_kwargs())
    print(f"[gpu] generate_codes_profiled {name}", flush=True)
    with E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=w.max_cache_steps)) as eng:
        g = eng.generate_codes(w.inputs(model), opts)
        p = eng.generate_codes_profiled(w.inputs(model), opts)
        again = eng.generate_codes(w.inputs(model), opts)  # the slot is free again
    np.testing.assert_array_equal(p.codes.codes, g.codes)
    np.testing.assert_array_equal(again.codes, g.codes)
    assert (p.codes.frames, p.codes.ended_by_eos) == (g.frames, g.ended_by_eos)
    prof = p.profile
    assert prof.upload_seconds > 0 and prof.prefill_seconds > 0
    assert prof.code_predictor_seconds > 0 and prof.talker_decode_seconds > 0
    assert prof.prepare_prefix_seconds == 0 and prof.build_step_input_seconds == 0
    assert prof.total_seconds() == pytest.approx(
        prof.prepare_text_seconds + prof.upload_seconds + prof.prefill_seconds + prof.code_predictor_seconds
        + prof.talker_decode_seconds)
    print(f"{name}: {p.codes.frames} frames; code predictor {1e3 * prof.code_predictor_seconds:.2f} ms, "
          f"talker {1e3 * prof.talker_decode_seconds:.2f} ms, prefill {1e3 * prof.prefill_seconds:.3f} ms")


@pytest.mark.parametrize("use_graph", [True, False])
def test_phase_timed_frames_equal_plain_frames(models, use_graph):
    """q3t_debug_phase_times (the CodePredictor and the Talker step replayed as two graphs, or
    launched eagerly, with events between them) produces the same codes as next_codes_chunk and
    a positive time for every phase of every frame; the timed kernel hook runs too."""
    w = WORKLOADS["tiny_greedy"]
    model, d = models.get(w.spec)
    opts = E.GenerateOptions(**w.options_kwargs())
    print(f"[gpu] phase times graph={use_graph}", flush=True)
    with E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=w.max_cache_steps, use_graph=use_graph)) as eng:
        ref = eng.generate_codes(w.inputs(model), opts).codes
        got, cps, tks = [], [], []
        with eng.start_stream(w.inputs(model), opts) as st:
            while True:
                c, cp, tk = st.next_codes_chunk_timed(5)
                cps += list(cp)
                tks += list(tk)
                if c is None:
                    break
                got.append(c.codes)
                assert len(cp) == c.frames
        us, b = eng.bench_kernel_timed(2, 40)
    np.testing.assert_array_equal(np.concatenate(got), ref)
    assert len(cps) == len(ref) and min(cps) > 0 and min(tks) > 0
    assert us > 0 and b > 0
    print(f"CodePredictor {np.mean(cps):.1f} us, Talker step {np.mean(tks):.1f} us per frame; gate/up {us:.2f} us")


def test_graph_replay_is_bitwise_equal_to_eager(models):
    a = run(models, "tiny_sampled", use_graph=True)
    b = run(models, "tiny_sampled", use_graph=False)
    np.testing.assert_array_equal(a["codes"], b["codes"])
    np.testing.assert_array_equal(a["talker_logits"], b["talker_logits"])
    np.testing.assert_array_equal(a["cp_logits"], b["cp_logits"])


def test_runs_are_deterministic(models):
    a = run(models, "tiny_greedy")
    b = run(models, "tiny_greedy")
    np.testing.assert_array_equal(a["talker_logits"], b["talker_logits"])
    np.testing.assert_array_equal(a["codes"], b["codes"])


def _oracle_rollout(model, inputs, opts: E.GenerateOptions, cap, kv_bf16=False, keep_cp=0):
    o = Oracle(model.tensors, model.config(), max_cache_steps=cap, kv_bf16=kv_bf16)
    oo = OracleOptions(**{k: getattr(opts, k) for k in OracleOptions.__dataclass_fields__})
    return o.rollout(inputs.prefill, inputs.trailing_text, inputs.tts_pad_embed, oo, keep_cp_logits=keep_cp)


def _as_fixture(tr):
    return dict(codes=tr.codes, talker_logits=tr.talker_logits, talker_margins=tr.talker_margins,
                cp_margins=tr.cp_margins, meta=dict(ended_by_eos=tr.ended_by_eos))


@pytest.mark.parametrize("per_occurrence", [False, True])
def test_greedy_repetition_penalty_matches_oracle(models, per_occurrence):
    """Repetition penalty 1.3 on a greedy Talker, counted once per distinct token (HF) or once
    per occurrence (the crate's GPU kernel, kernels.rs:408-426)."""
    w = WORKLOADS["tiny_greedy"]
    model, _ = models.get(w.spec)
    inputs = w.inputs(model)
    opts = E.GenerateOptions.greedy(16, repetition_penalty=1.3, repetition_penalty_per_occurrence=per_occurrence)
    r = run(models, "tiny_greedy", options=opts)
    fx = _as_fixture(_oracle_rollout(model, inputs, opts, w.max_cache_steps))
    same = check_codes(r["codes"], r["eos"], fx)
    check_talker_logits(r["talker_logits"], fx, same)


def test_sampled_talker_with_greedy_subtalker_matches_oracle(models):
    """Talker sampling (top-k 50, T 0.9, penalty 1.05) with a greedy CodePredictor: the greedy
    groups hand their tokens from one LM head to the next group's first GEMV, while the
    Talker's token still goes through its sampler."""
    w = WORKLOADS["tiny_greedy"]
    model, _ = models.get(w.spec)
    inputs = w.inputs(model)
    opts = E.GenerateOptions.greedy(16, do_sample=True, top_k=50, top_p=1.0, temperature=0.9,
                                    repetition_penalty=1.05, seed=11)
    r = run(models, "tiny_greedy", options=opts)
    fx = _as_fixture(_oracle_rollout(model, inputs, opts, w.max_cache_steps))
    same = check_codes(r["codes"], r["eos"], fx)
    check_talker_logits(r["talker_logits"], fx, same)
    print(f"sampled Talker + greedy CodePredictor: {same} frames identical")


@pytest.mark.parametrize("sampled", [False, True])
def test_one_query_head_per_kv_head_matches_oracle(models, sampled):
    """A model with one query head per KV head in both stacks and a 512 -> 1024 projection into
    the CodePredictor: its fused attention + O projection with 1 query head per KV head, after a
    token hand-off (greedy) and after a sampled group."""
    from q3t import textprep
    model, d = models.get("tiny-g1")
    inputs = textprep.TextPrep(model).prepare(np.random.default_rng(5).integers(0, 151643, 20))
    kw = dict(subtalker_dosample=True, subtalker_top_k=50, subtalker_top_p=0.9, subtalker_temperature=0.9,
              seed=3) if sampled else {}
    opts = E.GenerateOptions.greedy(12, **kw)
    r = run(models, "tiny_greedy", options=opts, inputs=inputs, model_dir=d, cap=64)
    fx = _as_fixture(_oracle_rollout(model, inputs, opts, 64))
    same = check_codes(r["codes"], r["eos"], fx)
    err = check_talker_logits(r["talker_logits"], fx, same)
    print(f"tiny-g1 sampled={sampled}: {same} frames identical, talker logit err {err:.2e}")


def test_bf16_kv_cache_matches_bf16_oracle(models):
    """KV stored as bf16 (rounded once at the store), against the oracle's bf16-KV model."""
    w = WORKLOADS["tiny_greedy"]
    model, _ = models.get(w.spec)
    tr = _oracle_rollout(model, w.inputs(model), E.GenerateOptions(**w.options_kwargs()), w.max_cache_steps,
                         kv_bf16=True)
    r = run(models, "tiny_greedy", kv_bf16=True)
    fx = _as_fixture(tr)
    same = check_codes_near_tie(r["codes"], r["eos"], fx)
    check_talker_logits(r["talker_logits"], fx, same)


def test_eos_ends_stream_like_the_reference(models, tmp_path):
    """A model whose EOS row copies (and slightly beats) a token the baseline emits."""
    w = WORKLOADS["tiny_greedy"]
    base, _ = models.get(w.spec)
    inputs = w.inputs(base)
    ref = _oracle_rollout(base, inputs, E.GenerateOptions.greedy(12), w.max_cache_steps)
    sem = ref.codes[:, 0].tolist()
    # the first semantic token that first appears at frame >= 2: EOS takes its place there
    target = next(t for f, t in enumerate(sem) if f >= 2 and t not in sem[:f])
    tensors = dict(base.tensors)
    head = synth.bf16_bits_to_f32(tensors["talker.codec_head.weight"]).copy()
    head[2150] = head[target] * 1.01
    tensors["talker.codec_head.weight"] = synth.f32_to_bf16_bits(head)
    model = synth.SyntheticModel(base.spec, base.seed, tensors)
    model.write(str(tmp_path))
    tr = _oracle_rollout(model, inputs, E.GenerateOptions.greedy(12), w.max_cache_steps)
    assert tr.ended_by_eos and 0 < tr.frames < 12
    r = run(models, "tiny_greedy", options=E.GenerateOptions.greedy(12), model_dir=str(tmp_path), chunk=2)
    np.testing.assert_array_equal(r["codes"], tr.codes)
    assert r["eos"] and r["chunks"][-1].ended_by_eos


@pytest.mark.parametrize("spec,n_ids,cap,frames,kv_bf16,fused_rows", [
    ("tiny", 291, 512, 8, False, 512),      # positions 300-307: two 256-row passes
    ("tiny", 240, 320, 16, False, 320),     # positions 249-264: the second pass starts mid-stream
    ("tiny-g1", 240, 320, 16, False, 320),  # one query head per KV head
    ("tiny", 1000, 1024, 10, False, 1024),  # positions 1009-1018: four passes, the longest cache
    ("tiny", 291, 512, 8, True, 512),       # bf16 cache (every row group loaded)
    # the engine's default: fused below position 192 (fp32 cache) or 256 (bf16), the split
    # attention + merging O from there (positions 189-204 and 254-269 in calls of 4 frames:
    # one call runs both graphs of the slot)
    ("tiny", 180, 320, 16, False, None),
    ("tiny", 1000, 1024, 10, False, None),
    ("tiny", 245, 320, 16, True, None),
])
def test_fused_talker_attention_long_caches_match_oracle(models, spec, n_ids, cap, frames, kv_bf16, fused_rows):
    """The Talker's fused attention + O projection (hidden 512 / 1024, caches of 33 .. 1024
    rows) runs its key rows in passes of 256: caches past one pass, across the pass boundary,
    and at the 1024-row limit (q3t_engine_set_fused_attention_rows at the capacity keeps it at
    every position), against the oracle's rollout of the same prompt; and the engine's
    default, which moves long positions to the split attention mid-stream."""
    model, d = models.get(spec)
    prompt = np.random.default_rng(n_ids + cap).integers(0, 151643, n_ids)
    from q3t import textprep
    inputs = textprep.TextPrep(model).prepare(prompt)
    assert inputs.prefill_steps == n_ids + 9
    opts = E.GenerateOptions.greedy(frames)
    print(f"[gpu] fused attention spec={spec} P={inputs.prefill_steps} cap={cap} kv_bf16={kv_bf16} "
          f"fused_rows={fused_rows}", flush=True)
    with E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=cap, kv_bf16=kv_bf16)) as eng:
        if fused_rows is not None:
            eng.set_fused_attention_rows(fused_rows)
        eng.set_trace(True)
        with eng.start_stream(inputs, opts) as st:
            chunks = []
            while (c := st.next_codes_chunk(4)) is not None:
                chunks.append(c)
            tl, eos = st.talker_logits(), st.ended_by_eos
    codes = np.concatenate([c.codes for c in chunks])
    fx = _as_fixture(_oracle_rollout(model, inputs, opts, cap, kv_bf16=kv_bf16))
    same = (check_codes_near_tie if kv_bf16 else check_codes)(codes, eos, fx)
    err = check_talker_logits(tl, fx, same)
    print(f"{spec} P={inputs.prefill_steps} cap={cap}: {same} frames identical, talker logit err {err:.2e}")


def test_cache_past_1024_rows_matches_oracle(models):
    """A 1,109-row prompt in a 1,152-row cache: the Talker's attention spans 9 chunks of 128
    rows, more than the O projection merges itself, so the merge kernel runs first."""
    w = WORKLOADS["tiny_greedy"]
    model, _ = models.get(w.spec)
    prompt = np.random.default_rng(21).integers(0, 151643, 1100)
    from q3t import textprep
    inputs = textprep.TextPrep(model).prepare(prompt)
    assert inputs.prefill_steps == 1109
    opts = E.GenerateOptions.greedy(6)
    r = run(models, "tiny_greedy", options=opts, inputs=inputs, cap=1152)
    fx = _as_fixture(_oracle_rollout(model, inputs, opts, 1152))
    same = check_codes(r["codes"], r["eos"], fx)
    err = check_talker_logits(r["talker_logits"], fx, same)
    print(f"1152-row cache: {same} frames identical, talker logit err {err:.2e}")


def test_cache_of_33_chunks_matches_oracle(models):
    """A 4,107-row prompt in a 4,224-row cache: 33 key chunks of 128 rows, merged by the merge
    kernel's 64-slot form before the O projection."""
    w = WORKLOADS["tiny_greedy"]
    model, _ = models.get(w.spec)
    prompt = np.random.default_rng(22).integers(0, 151643, 4098)
    from q3t import textprep
    inputs = textprep.TextPrep(model).prepare(prompt)
    assert inputs.prefill_steps == 4107
    opts = E.GenerateOptions.greedy(4)
    r = run(models, "tiny_greedy", options=opts, inputs=inputs, cap=4224)
    fx = _as_fixture(_oracle_rollout(model, inputs, opts, 4224))
    same = check_codes(r["codes"], r["eos"], fx)
    err = check_talker_logits(r["talker_logits"], fx, same)
    print(f"4224-row cache: {same} frames identical, talker logit err {err:.2e}")


def test_largest_cache_matches_oracle_to_its_last_row(models):
    """The largest cache the attention kernels take (64 key chunks of 128 rows, 8,192 rows):
    an 8,186-row prompt and 6 frames, so the last frame's Talker row is row 8,191.  One row
    more is refused when the engine is created, before any kernel runs."""
    w = WORKLOADS["tiny_greedy"]
    model, d = models.get(w.spec)
    with pytest.raises(E.InvalidInputError):
        E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=8193))
    prompt = np.random.default_rng(23).integers(0, 151643, 8177)
    from q3t import textprep
    inputs = textprep.TextPrep(model).prepare(prompt)
    assert inputs.prefill_steps == 8186
    opts = E.GenerateOptions.greedy(6)
    r = run(models, "tiny_greedy", options=opts, inputs=inputs, cap=8192)
    fx = _as_fixture(_oracle_rollout(model, inputs, opts, 8192))
    same = check_codes(r["codes"], r["eos"], fx)
    err = check_talker_logits(r["talker_logits"], fx, same)
    print(f"8192-row cache: {same} frames identical, talker logit err {err:.2e}")


@pytest.mark.parametrize("frames", [1, 2])
def test_shortest_streams_match_oracle(models, frames):
    """One frame (the prefill's logits give its semantic token and the frame's last Talker
    decode is skipped) and two frames, on the graph and the eager path."""
    w = WORKLOADS["tiny_greedy"]
    model, _ = models.get(w.spec)
    inputs = w.inputs(model)
    opts = E.GenerateOptions.greedy(frames)
    fx = _as_fixture(_oracle_rollout(model, inputs, opts, w.max_cache_steps))
    for use_graph in (True, False):
        r = run(models, "tiny_greedy", options=opts, inputs=inputs, use_graph=use_graph)
        assert len(r["codes"]) == frames
        same = check_codes(r["codes"], r["eos"], fx)
        check_talker_logits(r["talker_logits"], fx, same)


def test_capacity_busy_and_exhausted_streams(models):
    w = WORKLOADS["tiny_greedy"]
    model, d = models.get(w.spec)
    inputs = w.inputs(model)
    with E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=64, max_streams=1)) as eng:
        with pytest.raises(E.CapacityError):
            eng.start_stream(inputs, E.GenerateOptions.greedy(64 - inputs.prefill_steps + 1))
        st = eng.start_stream(inputs, E.GenerateOptions.greedy(3))
        with pytest.raises(E.BusyError):
            eng.start_stream(inputs, E.GenerateOptions.greedy(3))
        assert st.next_codes_chunk(6).frames == 3
        assert st.next_codes_chunk(6) is None
        with pytest.raises(E.InvalidInputError):
            st.next_codes_chunk(0)
        st.close()
        st2 = eng.start_stream(inputs, E.GenerateOptions.greedy(2))   # the slot is free again
        assert st2.next_codes_chunk(1).frames == 1
        # finish_codes returns what was produced so far, without draining (generation.rs:991-997)
        assert st2.finish_codes().frames == 1
        with pytest.raises(E.InvalidInputError):
            eng.start_stream(inputs, E.GenerateOptions(top_p=0.0))


def test_two_stream_slots_are_independent(models):
    w = WORKLOADS["tiny_greedy"]
    model, d = models.get(w.spec)
    inputs = w.inputs(model)
    ref = run(models, "tiny_greedy", trace=False)["codes"]
    with E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=w.max_cache_steps, max_streams=2)) as eng:
        opts = E.GenerateOptions(**w.options_kwargs())
        a = eng.start_stream(inputs, opts)
        b = eng.start_stream(inputs, opts)
        out_a, out_b = [], []
        while True:
            ca, cb = a.next_codes_chunk(5), b.next_codes_chunk(3)
            if ca:
                out_a.append(ca.codes)
            if cb:
                out_b.append(cb.codes)
            if ca is None and cb is None:
                break
        a.close()
        b.close()
    np.testing.assert_array_equal(np.concatenate(out_a), ref)
    np.testing.assert_array_equal(np.concatenate(out_b), ref)


@pytest.mark.parametrize("name", ["cfg1_cpu_0.6b", "cfg2_0.6b_greedy", "cfg3_0.6b_sampled", "cfg4_1.7b_greedy"])
def test_baseline_workloads_match_fixture(models, name):
    """BASELINE configs 1-4 against their float64 fixtures: every frame's 16 codes, the frame
    count and the EOS flag identical; Talker logits of every row and the first frames'
    CodePredictor logits within 2e-2.  Config 1 is the reference's CPU case (non-streaming,
    P = 41, 40 frames), run here on the GPU path."""
    fx = load_fixture(name)
    model, _ = models.get(fx["meta"]["spec"], fx["meta"]["weight_seed"])
    assert model.checksum() == fx["meta"]["checksum"]
    r = run(models, name)
    same = check_codes(r["codes"], r["eos"], fx)
    err = check_talker_logits(r["talker_logits"], fx, same)
    cp_err = check_cp_logits(r["cp_logits"], fx)
    print(f"{name}: {same}/{len(fx['codes'])} frames identical, talker logit max err {err:.2e}, "
          f"CodePredictor logit max err {cp_err:.2e}")
    if name.startswith("cfg4"):
        models.drop(fx["meta"]["spec"], fx["meta"]["weight_seed"])
