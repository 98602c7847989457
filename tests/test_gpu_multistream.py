"""GPU parity of the multi-stream path: q3t_streams_start runs one
prefill over every stream's prompt rows, q3t_streams_next_codes advances all listed
streams with one pass over the weights per frame.  Streams are independent, so each must
reproduce its own single-stream oracle rollout (tests/golden/<workload>.npz holds one per
stream) and the single-stream engine path.
"""
import time

import numpy as np
import pytest

from q3t import engine as E
from q3t.workloads import MULTI_WORKLOADS

from parity import LOGIT_TOL, check_codes, load_fixture

pytestmark = pytest.mark.gpu


def stream_fixture(fx, j):
    m = fx["meta"]
    return {"codes": fx[f"codes_{j}"], "talker_margins": fx[f"talker_margins_{j}"],
            "cp_margins": fx[f"cp_margins_{j}"], "talker_logits": fx[f"talker_logits_{j}"],
            "meta": {"ended_by_eos": m["ended_by_eos"][j]}}


def run_batch(models, name, use_graph=True, trace=False, chunk=None, kv_bf16=False):
    w = MULTI_WORKLOADS[name]
    model, d = models.get(w.spec, w.weight_seed)
    inputs = w.inputs(model)
    opts = [E.GenerateOptions(**kw) for kw in w.options_kwargs()]
    print(f"[gpu] batch {name} streams={w.streams} graph={use_graph} chunk={chunk}", flush=True)
    eng = E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=w.max_cache_steps, max_streams=w.streams,
                                            use_graph=use_graph, kv_bf16=kv_bf16))
    try:
        eng.set_trace(trace)
        t0 = time.perf_counter()
        streams = eng.start_streams(inputs, opts, E.StreamOptions(text_lookahead_tokens=1 << 30))
        t1 = time.perf_counter()
        live, sizes, calls = list(streams), [[] for _ in streams], 0
        while live:
            chunks = eng.next_codes_chunks(live, chunk or w.chunk_frames)
            calls += 1
            for s, c in zip(live, chunks):
                if c is not None:
                    sizes[streams.index(s)].append((c.frames, c.total_frames))
            live = [s for s, c in zip(live, chunks) if c is not None]
        eng.synchronize()
        t2 = time.perf_counter()
        logits = [s.talker_logits() for s in streams] if trace else None
        out = [s.finish_codes() for s in streams]
    finally:
        eng.close()
    frames = sum(o.frames for o in out)
    print(f"{name}: prefill {1e3 * (t1 - t0):.1f} ms, {frames} frames in {t2 - t1:.3f} s "
          f"({frames / (t2 - t1):.1f} frames/s aggregate, {calls} calls)", flush=True)
    return dict(codes=[o.codes for o in out], eos=[o.ended_by_eos for o in out], logits=logits, sizes=sizes,
                frames_per_s=frames / (t2 - t1))


def run_single(models, name, j, use_graph=True):
    w = MULTI_WORKLOADS[name]
    model, d = models.get(w.spec, w.weight_seed)
    inp = w.inputs(model)[j]
    opts = E.GenerateOptions(**w.options_kwargs()[j])
    with E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=w.max_cache_steps, use_graph=use_graph)) as eng:
        return eng.generate_codes(inp, opts)


def test_tiny_multistream_matches_oracle(models):
    name = "tiny_multistream"
    fx = load_fixture(name)
    w = MULTI_WORKLOADS[name]
    model, _ = models.get(w.spec, w.weight_seed)
    assert model.checksum() == fx["meta"]["checksum"]
    r = run_batch(models, name, trace=True)
    for j in range(w.streams):
        sf = stream_fixture(fx, j)
        same = check_codes(r["codes"][j], r["eos"][j], sf)
        rows = min(len(sf["talker_logits"]), same + 1)
        err = float(np.abs(r["logits"][j][:rows] - sf["talker_logits"][:rows].astype(np.float32)).max())
        print(f"stream {j}: {same} frames identical, talker logit err {err:.2e}")
        assert err <= LOGIT_TOL


@pytest.mark.parametrize("name", ["tiny_multistream", "tinyproj_multistream", "tiny_multistream_greedy",
                                  "tinyg1_multistream"])
def test_multistream_equals_single_stream_path(models, name):
    r = run_batch(models, name)
    for j in range(MULTI_WORKLOADS[name].streams):
        g = run_single(models, name, j)
        np.testing.assert_array_equal(r["codes"][j], g.codes, err_msg=f"stream {j}")


@pytest.mark.parametrize("name", ["tiny_multistream", "tiny_multistream_greedy", "tinyg1_multistream"])
def test_multistream_graph_replay_equals_eager(models, name):
    a = run_batch(models, name, use_graph=True)
    b = run_batch(models, name, use_graph=False)
    for j, (x, y) in enumerate(zip(a["codes"], b["codes"])):
        np.testing.assert_array_equal(x, y, err_msg=f"stream {j}")


def test_greedy_batch_hand_off_matches_traced_batch(models):
    """All-greedy batches hand tokens over between CodePredictor groups without selection
    kernels; with logit tracing on the batch takes the selection kernels instead.  Both give
    the same codes."""
    a = run_batch(models, "tiny_multistream_greedy")
    b = run_batch(models, "tiny_multistream_greedy", trace=True)
    for j, (x, y) in enumerate(zip(a["codes"], b["codes"])):
        np.testing.assert_array_equal(x, y, err_msg=f"stream {j}")


def test_multistream_chunks_are_per_stream(models):
    w = MULTI_WORKLOADS["tiny_multistream"]
    r = run_batch(models, "tiny_multistream", chunk=4)
    _, frames, _ = w.plan()
    for j, sz in enumerate(r["sizes"]):
        n = [f for f, _ in sz]
        assert all(k == 4 for k in n[:-1]) and 0 < n[-1] <= 4, (j, n)
        assert [t for _, t in sz] == list(np.cumsum(n))
        assert sum(n) == len(r["codes"][j]) <= frames[j]


@pytest.mark.parametrize("name", ["tiny_multistream", "tinyg1_multistream"])
def test_unlisted_stream_is_untouched(models, name):
    """Stepping a subset must leave the other live streams exactly where they were (on
    tinyg1_multistream also through the split O / down GEMMs and the two-position prefix
    pass, whose zeroed buffers a masked row must not disturb)."""
    w = MULTI_WORKLOADS[name]
    model, d = models.get(w.spec, w.weight_seed)
    inputs = w.inputs(model)[:3]
    opts = [E.GenerateOptions(**kw) for kw in w.options_kwargs()[:3]]
    ref = [run_single(models, name, j).codes for j in range(3)]
    with E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=w.max_cache_steps, max_streams=4)) as eng:
        s = eng.start_streams(inputs, opts, E.StreamOptions(text_lookahead_tokens=1 << 30))
        for _ in range(3):
            eng.next_codes_chunks([s[0], s[2]], 3)     # stream 1 waits
        while s[1].next_codes_chunk(5) is not None:    # then runs alone on the single-stream path
            pass
        while any(c is not None for c in eng.next_codes_chunks([s[0], s[2]], 7)):
            pass
        got = [x.finish_codes().codes for x in s]
    for j in range(3):
        np.testing.assert_array_equal(got[j], ref[j], err_msg=f"stream {j}")


@pytest.mark.parametrize("name", ["tiny_multistream", "tinyg1_multistream"])
def test_lone_stream_switches_paths_mid_stream(models, name):
    """q3t_streams_next_codes runs a call with one stream left on the single-stream frame: a
    stream that alternates between batched calls and calls where it runs alone must still
    reproduce its single-stream rollout (the two frames share every piece of per-slot state)."""
    w = MULTI_WORKLOADS[name]
    model, d = models.get(w.spec, w.weight_seed)
    inputs = w.inputs(model)[:2]
    opts = [E.GenerateOptions(**kw) for kw in w.options_kwargs()[:2]]
    ref = [run_single(models, name, j).codes for j in range(2)]
    print(f"[gpu] lone stream path switches {name}", flush=True)
    with E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=w.max_cache_steps, max_streams=3)) as eng:
        s = eng.start_streams(inputs, opts, E.StreamOptions(text_lookahead_tokens=1 << 30))
        for step in range(64):
            listed = [s[0]] if step % 3 == 1 else ([s[1]] if step % 3 == 2 else list(s))
            if all(c is None for c in eng.next_codes_chunks(listed, 2)) and step % 3 == 0:
                break
        got = [x.finish_codes().codes for x in s]
    for j in range(2):
        np.testing.assert_array_equal(got[j], ref[j], err_msg=f"stream {j}")


def test_streams_start_reports_busy_and_capacity(models):
    w = MULTI_WORKLOADS["tiny_multistream"]
    model, d = models.get(w.spec, w.weight_seed)
    inputs = w.inputs(model)
    opts = [E.GenerateOptions(**kw) for kw in w.options_kwargs()]
    lk = E.StreamOptions(text_lookahead_tokens=1 << 30)
    with E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=w.max_cache_steps, max_streams=2)) as eng:
        with pytest.raises(E.BusyError):
            eng.start_streams(inputs[:3], opts[:3], lk)
        one = eng.start_stream(inputs[0], opts[0], lk)
        with pytest.raises(E.BusyError):
            eng.start_streams(inputs[1:3], opts[1:3], lk)
        two = eng.start_streams(inputs[1:2], opts[1:2], lk)
        one.close()
        two[0].close()
        big = E.GenerateOptions(**{**w.options_kwargs()[0], "max_frames": w.max_cache_steps})
        with pytest.raises(E.CapacityError):
            eng.start_streams(inputs[:1], [big], lk)


@pytest.mark.parametrize("trace", [False, True])
def test_cfg5_sixteen_streams_match_oracle(models, trace):
    """every stream's codes equal its float64 single-stream rollout over its
    whole length.  Untraced is the path bench.py times: an all-greedy batch hands each
    CodePredictor group's token to the next group through the LM head's per-row argmax keys
    and the layer-0 q/k/v table rows.  Traced, the batch takes the selection kernels and
    records the Talker logits, which are held to 2e-2."""
    name = "cfg5_0.6b_multistream"
    fx = load_fixture(name)
    w = MULTI_WORKLOADS[name]
    model, _ = models.get(w.spec, w.weight_seed)
    assert model.checksum() == fx["meta"]["checksum"]
    r = run_batch(models, name, trace=trace)
    for j in range(w.streams):
        sf = stream_fixture(fx, j)
        same = check_codes(r["codes"][j], r["eos"][j], sf)
        msg = f"stream {j}: P={fx['meta']['prefill_steps'][j]} {same}/{len(sf['codes'])} frames identical"
        if trace:
            rows = min(len(sf["talker_logits"]), same + 1)
            err = float(np.abs(r["logits"][j][:rows] - sf["talker_logits"][:rows].astype(np.float32)).max())
            msg += f", talker logit err {err:.2e}"
            assert err <= LOGIT_TOL
        print(msg)


def test_batched_stream_ends_by_eos_while_others_continue(models, tmp_path):
    """One stream of a batch hits EOS mid-chunk (a model whose EOS row copies and slightly beats
    a token the baseline emits); the others run to max_frames.  Every stream equals the
    single-stream path on the same model."""
    from q3t import synth
    from q3t.workloads import WORKLOADS
    w = WORKLOADS["tiny_greedy"]
    base, d0 = models.get(w.spec)
    inp = w.inputs(base)
    with E.HipTtsEngine(d0, E.EngineOptions(max_cache_steps=w.max_cache_steps)) as eng:
        sem = eng.generate_codes(inp, E.GenerateOptions.greedy(12)).codes[:, 0].tolist()
    target = next(t for f, t in enumerate(sem) if f >= 2 and t not in sem[:f])
    tensors = dict(base.tensors)
    head = synth.bf16_bits_to_f32(tensors["talker.codec_head.weight"]).copy()
    head[2150] = head[target] * 1.01
    tensors["talker.codec_head.weight"] = synth.f32_to_bf16_bits(head)
    synth.SyntheticModel(base.spec, base.seed, tensors).write(str(tmp_path))
    mw = MULTI_WORKLOADS["tiny_multistream"]
    inputs = [inp] + mw.inputs(base)[:2]
    opts = [E.GenerateOptions.greedy(12), E.GenerateOptions.greedy(10), E.GenerateOptions.greedy(14)]
    cap = max(mw.max_cache_steps, w.max_cache_steps)
    with E.HipTtsEngine(str(tmp_path), E.EngineOptions(max_cache_steps=cap)) as eng:
        ref = [eng.generate_codes(i, o) for i, o in zip(inputs, opts)]
    assert ref[0].ended_by_eos and 0 < ref[0].frames < 12
    with E.HipTtsEngine(str(tmp_path), E.EngineOptions(max_cache_steps=cap, max_streams=3)) as eng:
        s = eng.start_streams(inputs, opts, E.StreamOptions(text_lookahead_tokens=1 << 30))
        live, last = list(s), {}
        while live:
            chunks = eng.next_codes_chunks(live, 5)
            for x, c in zip(live, chunks):
                if c is not None:
                    last[id(x)] = c
            live = [x for x, c in zip(live, chunks) if c is not None]
        got = [x.finish_codes() for x in s]
        assert last[id(s[0])].ended_by_eos and not last[id(s[1])].ended_by_eos
    for j, (g, r) in enumerate(zip(got, ref)):
        np.testing.assert_array_equal(g.codes, r.codes, err_msg=f"stream {j}")
        assert g.ended_by_eos == r.ended_by_eos


def test_batched_bf16_kv_tracks_single_stream(models):
    """bf16 KV caches on the batched path.  The two paths add in different fp32 orders, and a
    bf16 store can round one ulp apart (0.4%), which the model then amplifies; so the runs are
    compared on what must hold.  While the token histories agree, the Talker logits agree
    within the 2e-2 bound.  The first differing frame is no earlier than frame 4."""
    name = "tiny_multistream"
    w = MULTI_WORKLOADS[name]
    model, d = models.get(w.spec, w.weight_seed)
    r = run_batch(models, name, kv_bf16=True, trace=True)
    for j, (inp, kw) in enumerate(zip(w.inputs(model), w.options_kwargs())):
        with E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=w.max_cache_steps, kv_bf16=True)) as eng:
            eng.set_trace(True)
            st = eng.start_stream(inp, E.GenerateOptions(**kw), E.StreamOptions(text_lookahead_tokens=1 << 30))
            while st.next_codes_chunk(8) is not None:
                pass
            logits = st.talker_logits()
            codes = st.finish_codes().codes
        a, b = r["codes"][j], codes
        n = min(len(a), len(b))
        diff = np.nonzero((a[:n] != b[:n]).any(1))[0]
        first = int(diff[0]) if diff.size else n
        rows = min(first + 1, len(logits), len(r["logits"][j]))
        err = float(np.abs(r["logits"][j][:rows] - logits[:rows]).max())
        print(f"stream {j}: first differing frame {first} of {n}, logits over {rows} rows max diff {err:.2e}")
        assert err <= LOGIT_TOL
        assert first >= min(4, n)


@pytest.mark.parametrize("cap,n_ids", [(2304, (2100, 2190)), (4224, (3990, 4098))])
def test_batched_caches_past_2048_rows_match_oracle(models, cap, n_ids):
    """Stream rows in caches longer than 64 chunks of 32 rows: the batched Talker attention
    takes 64-row chunks (2,304-row cache, 36 partials) or 128-row chunks (4,224 rows, 33),
    since k_attn_merge merges at most 64, while the CodePredictor keeps its one 32-row chunk.
    Two greedy streams of 5 and 7 frames (the longer one ends alone, on the single-stream
    frame) each reproduce their float64 oracle rollout."""
    from oracle.model import GenerateOptions as OracleOptions
    from oracle.model import Oracle
    from q3t import textprep
    model, d = models.get("tiny", 0)
    prep = textprep.TextPrep(model)
    inputs = [prep.prepare(np.random.default_rng(30 + j).integers(0, 151643, n)) for j, n in enumerate(n_ids)]
    opts = [E.GenerateOptions.greedy(5), E.GenerateOptions.greedy(7)]
    print(f"[gpu] batched long caches cap={cap}", flush=True)
    with E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=cap, max_streams=2)) as eng:
        streams = eng.start_streams(inputs, opts, E.StreamOptions(text_lookahead_tokens=1 << 30))
        live = list(streams)
        while live:
            chunks = eng.next_codes_chunks(live, 3)
            live = [s for s, c in zip(live, chunks) if c is not None]
        out = [s.finish_codes() for s in streams]
    for j in range(2):
        o = Oracle(model.tensors, model.config(), max_cache_steps=cap)
        oo = OracleOptions(**{k: getattr(opts[j], k) for k in OracleOptions.__dataclass_fields__})
        tr = o.rollout(inputs[j].prefill, inputs[j].trailing_text, inputs[j].tts_pad_embed, oo)
        fx = dict(codes=tr.codes, talker_margins=tr.talker_margins, cp_margins=tr.cp_margins,
                  meta=dict(ended_by_eos=tr.ended_by_eos))
        same = check_codes(out[j].codes, out[j].ended_by_eos, fx)
        print(f"stream {j} (prefill {inputs[j].prefill_steps} rows): {same} frames identical")


def test_batched_1p7b_streams_match_fixture_and_single_stream(models):
    """The 1.7B Talker on the batched frame (hidden 2048 and intermediate 6144 in the skinny
    GEMMs, the CodePredictor input projected to 1024): config 4's stream next to two others
    (40, 25 and 33 frames, so config 4's stream ends alone on the single-stream frame).  Its
    codes repeat the first 40 frames of its float64 fixture; the others repeat their
    single-stream rollouts.  The model stays cached for config 4's parity test."""
    from q3t import textprep
    from q3t.workloads import WORKLOADS
    fx = load_fixture("cfg4_1.7b_greedy")
    w = WORKLOADS["cfg4_1.7b_greedy"]
    model, d = models.get(w.spec, w.weight_seed)
    assert model.checksum() == fx["meta"]["checksum"]
    prep = textprep.TextPrep(model)
    inputs = [w.inputs(model)] + [prep.prepare(textprep.random_prompt(n, 40 + n)) for n in (30, 90)]
    opts = [E.GenerateOptions.greedy(40), E.GenerateOptions.greedy(25), E.GenerateOptions.greedy(33)]
    print("[gpu] batched 1.7B streams", flush=True)
    with E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=w.max_cache_steps, max_streams=3)) as eng:
        streams = eng.start_streams(inputs, opts)
        live = list(streams)
        while live:
            chunks = eng.next_codes_chunks(live, 6)
            live = [s for s, c in zip(live, chunks) if c is not None]
        got = [s.finish_codes().codes for s in streams]
        for s in streams:
            s.close()
        refs = [eng.generate_codes(inputs[j], opts[j]).codes for j in (1, 2)]
    np.testing.assert_array_equal(got[0], fx["codes"][:40])
    for j in (1, 2):
        np.testing.assert_array_equal(got[j], refs[j - 1], err_msg=f"stream {j}")
    print(f"1.7B batched: {[len(g) for g in got]} frames, config 4's stream equal to its fixture")
