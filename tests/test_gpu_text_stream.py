"""Text streams on the device (q3t_text_stream_start / _push / _finish and the open-text cap in
q3t_stream_next_codes), on the tiny model written with its text table, tokenizer and codec.

A text stream's codes depend only on its sequence of content ids (the flush points fix it) and
min_start_tokens, not on when the text arrives: stalls delay frames and change no state the
frames read, the sampler's counters included.  So every stream here is compared with
start_stream over the same ids with text_lookahead_tokens = min_start_tokens, and the first
one also with the CPU oracle's rollout of the same prompt rows."""
import ctypes
import threading
import time

import numpy as np
import pytest

from oracle.model import GenerateOptions as OracleOptions
from oracle.model import Oracle
from oracle.textprep import TextPrepOracle
from q3t import engine as E
from q3t import synth
from q3t import text_stream as TS
from q3t.voice_clone import VoiceClonePrompt

from parity import check_codes

pytestmark = pytest.mark.gpu

TEXT = "hello world, hello world! the quick brown fox jumps over the lazy dog. ok then, bye."


@pytest.fixture(scope="module")
def tiny_text(models):
    model, d = models.get_with_text("tiny")
    rows = lambda ids: synth.text_embedding_rows(model.seed, ids, model.spec.text_hidden)
    oracle = TextPrepOracle(model.tensors, model.config(), rows, synth.TEXT_VOCAB)
    eng = E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=256))
    yield model, oracle, eng, d
    eng.close()


def queue_of(eng, pieces, tso):
    """The content ids a text stream fed `pieces` (then finished) queues, from a stream that
    never starts."""
    shadow = TS.PollingTextStream(eng, E.GenerateOptions.greedy(4), tso)
    for p in pieces:
        shadow.push_text(p)
    shadow.finish_text()
    return list(shadow.queued_tokens)


def drain_text_stream(ts, chunk, got=None):
    """Pulls until Finished; the Finished codes are every chunk's codes, `got` (the chunks pulled
    before) included."""
    got = [] if got is None else got
    while True:
        r = ts.next_codes_chunk(chunk)
        if r.kind == TS.CHUNK:
            got.append(r.chunk.codes)
        elif r.kind == TS.FINISHED:
            cat = np.concatenate(got) if got else np.zeros((0, 16), np.int32)
            np.testing.assert_array_equal(r.codes.codes, cat)
            return r.codes
        else:
            raise AssertionError("the stream asked for more text after finish_text")


def drain_stream(st, chunk=7):
    got = []
    while (c := st.next_codes_chunk(chunk)) is not None:
        got.append(c.codes)
    st.close()
    return (np.concatenate(got) if got else np.zeros((0, 16), np.int32)), st.ended_by_eos


def test_all_text_first_matches_start_stream_and_oracle(tiny_text):
    model, oracle, eng, _ = tiny_text
    tso = TS.TextStreamOptions(min_start_tokens=4)
    opts = E.GenerateOptions.greedy(20)
    print("[gpu] text stream: all text, then pulls", flush=True)
    ts = eng.start_text_stream_polling(opts, tso)
    ts.push_text(TEXT)
    ts.finish_text()
    got = drain_text_stream(ts, 5)
    ids = queue_of(eng, [TEXT], tso)
    ref, eos = drain_stream(eng.start_stream(ids, opts, E.StreamOptions(text_lookahead_tokens=4)))
    np.testing.assert_array_equal(got.codes, ref)
    assert got.ended_by_eos == eos
    ref_in = oracle.prepare(ids, "ryan", "english", 4)
    o = Oracle(model.tensors, model.config(), max_cache_steps=256)
    oo = OracleOptions(**{k: getattr(opts, k) for k in OracleOptions.__dataclass_fields__})
    tr = o.rollout(ref_in.prefill, ref_in.trailing_text, ref_in.tts_pad_embed, oo)
    fx = dict(codes=tr.codes, talker_logits=tr.talker_logits, talker_margins=tr.talker_margins,
              cp_margins=tr.cp_margins, meta=dict(ended_by_eos=tr.ended_by_eos))
    same = check_codes(got.codes, got.ended_by_eos, fx)
    print(f"text stream vs oracle: {same} frames identical")


@pytest.mark.parametrize("min_start,min_resume,sample", [(3, 1, True), (8, 1, False), (2, 3, True)])
def test_incremental_text_matches_start_stream(tiny_text, min_start, min_resume, sample):
    """Words pushed one at a time with pulls in between: the stream waits for text (NeedMoreText)
    and resumes; its codes equal start_stream's over the same ids, sampling included."""
    model, oracle, eng, _ = tiny_text
    tso = TS.TextStreamOptions(min_start_tokens=min_start, min_resume_tokens=min_resume)
    opts = (E.GenerateOptions(max_frames=40, seed=7, repetition_penalty=1.05) if sample
            else E.GenerateOptions.greedy(40))
    pieces = [w + " " for w in TEXT.split(" ")]
    print(f"[gpu] text stream incremental min_start={min_start} min_resume={min_resume} sample={sample}",
          flush=True)
    ts = eng.start_text_stream_polling(opts, tso)
    got, waits, held, done = [], 0, 0, False
    for p in pieces:  # push a word, then pull 2-frame chunks until the stream stops for text
        ts.push_text(p)
        while not done:
            r = ts.next_codes_chunk(2)
            if r.kind == TS.FINISHED:
                done = True
                break
            if r.kind == TS.CHUNK:
                got.append(r.chunk.codes)
            else:
                waits += 1
            if r.kind == TS.NEED_MORE_TEXT or r.chunk.frames < 2:
                s = ts._stream
                if s is not None and not (s.ended_by_eos or s.frame >= opts.max_frames):
                    # started and not ended: it stopped for lack of queued ids
                    assert len(ts.queued_tokens) < min_resume
                    held += len(ts.queued_tokens) > 0
                break
        if done:
            break
    ts.finish_text()
    fin = drain_text_stream(ts, 3, got)
    assert waits > 0
    if min_resume > 1:
        assert held > 0  # stopped although ids were queued: fewer than min_resume_tokens
    ids = queue_of(eng, pieces, tso)
    ref, eos = drain_stream(eng.start_stream(ids, opts, E.StreamOptions(text_lookahead_tokens=min_start)))
    np.testing.assert_array_equal(fin.codes, ref)
    assert fin.ended_by_eos == eos
    print(f"incremental text stream: {fin.frames} frames identical after {waits} waits")


def test_voice_clone_text_stream(tiny_text):
    model, oracle, eng, _ = tiny_text
    emb = (np.random.default_rng(3).standard_normal(model.spec.talker.hidden) * 0.5).astype(np.float32)
    prompt = VoiceClonePrompt(emb, x_vector_only_mode=True)
    tso = TS.TextStreamOptions(min_start_tokens=5)
    opts = E.GenerateOptions.greedy(16)
    print("[gpu] voice clone text stream", flush=True)
    ts = eng.start_voice_clone_text_stream_polling(prompt, opts, tso)
    for w in TEXT.split(" ")[:6]:
        ts.push_text(w + " ")
        ts.next_codes_chunk(4)
    ts.finish_text()
    ts.close()  # dropped mid-way: frees the slot
    ts = eng.start_voice_clone_text_stream_polling(prompt, opts, tso)
    ts.push_text(TEXT)
    ts.finish_text()
    got = drain_text_stream(ts, 6)
    ids = queue_of(eng, [TEXT], tso)
    ref, _ = drain_stream(eng.start_voice_clone_stream(ids, prompt, opts, E.StreamOptions(text_lookahead_tokens=5)))
    np.testing.assert_array_equal(got.codes, ref)
    bad = VoiceClonePrompt(emb, x_vector_only_mode=False)
    ts = eng.start_voice_clone_text_stream_polling(bad, opts, tso)
    ts.push_text(TEXT)
    with pytest.raises(ValueError, match="only x-vector-only"):
        ts.next_codes_chunk(2)


def test_blocking_text_stream_audio(tiny_text):
    """HipTextStream: a producer thread pushes words while the consumer pulls audio; each chunk
    is the decode of its frames with up to left_context_frames earlier frames."""
    model, oracle, eng, _ = tiny_text
    tso = TS.TextStreamOptions(min_start_tokens=4, left_context_frames=3)
    opts = E.GenerateOptions.greedy(14)
    pieces = [w + " " for w in TEXT.split(" ")[:8]]
    print("[gpu] blocking text stream with audio", flush=True)
    inp, st = eng.start_text_stream(opts, tso)

    def produce():
        for p in pieces:
            inp.push_text(p)
            time.sleep(0.01)
        inp.finish()

    th = threading.Thread(target=produce)
    th.start()
    chunks = []
    while (c := st.next_audio_chunk(4)) is not None:
        chunks.append(c)
    th.join()
    fin = st.finished_codes()
    st.close()
    assert fin is not None and sum(c.frames for c in chunks) == fin.frames
    spf = eng.info["samples_per_frame"]
    for c in chunks:
        start = c.total_frames - c.frames
        ctx = min(3, start)
        ref = eng.decode_codes(fin.codes[start - ctx:c.total_frames])[ctx * spf:]
        assert c.samples.shape == (c.frames * spf,)
        np.testing.assert_allclose(c.samples, ref, rtol=0, atol=1e-6)
    ids = queue_of(eng, pieces, tso)
    ref, _ = drain_stream(eng.start_stream(ids, opts, E.StreamOptions(text_lookahead_tokens=4)))
    np.testing.assert_array_equal(fin.codes, ref)


def test_rows_past_max_frames_and_raw_abi(tiny_text):
    """Through the C ABI directly: ids pushed beyond what max_frames frames read are dropped,
    frames stop at the pushed rows while the text is open, and push after finish fails."""
    model, oracle, eng, _ = tiny_text
    lib = E.load_library()
    opts = E.GenerateOptions.greedy(5)
    o = opts._c()
    pre = np.array(eng.content_ids("hello world"), np.int32)
    h = ctypes.c_void_p()
    print("[gpu] raw text stream ABI", flush=True)
    E._check(lib.q3t_text_stream_start(eng._h, E._iptr(pre), int(pre.size), None, 0, ctypes.byref(o),
                                       ctypes.byref(h)))
    buf = np.zeros((8, 16), np.int32)
    info = E._ChunkInfo()
    E._check(lib.q3t_stream_next_codes(h, 8, E._iptr(buf), ctypes.byref(info)))
    assert (info.frames, info.total_frames, info.ended_by_eos) == (0, 0, 0)  # waits for row 0
    more = np.array(eng.content_ids(" the quick brown fox jumps over the lazy dog"), np.int32)
    assert more.size > 6
    E._check(lib.q3t_text_stream_push(h, E._iptr(more[:2]), 2))
    E._check(lib.q3t_stream_next_codes(h, 8, E._iptr(buf), ctypes.byref(info)))
    assert info.frames == 2 or info.ended_by_eos  # frames 0 and 1 read rows 0 and 1; frame 2 waits
    first = buf[:info.frames].copy()
    E._check(lib.q3t_text_stream_push(h, E._iptr(more[2:]), int(more.size - 2)))  # past max_frames: dropped
    E._check(lib.q3t_text_stream_finish(h))
    E._check(lib.q3t_text_stream_finish(h))  # a second finish does nothing
    with pytest.raises(E.InvalidInputError, match="cannot push text after finish_text"):
        E._check(lib.q3t_text_stream_push(h, E._iptr(more[:1]), 1))
    E._check(lib.q3t_stream_next_codes(h, 8, E._iptr(buf), ctypes.byref(info)))
    assert info.total_frames == 5 or info.ended_by_eos
    codes = np.concatenate([first, buf[:info.frames]])
    E._check(lib.q3t_stream_destroy(h))
    ids = list(pre) + list(more)
    ref, _ = drain_stream(eng.start_stream(ids, opts, E.StreamOptions(text_lookahead_tokens=int(pre.size))))
    np.testing.assert_array_equal(codes, ref)


def test_text_stream_errors(tiny_text):
    model, oracle, eng, d = tiny_text
    with pytest.raises(E.CapacityError):
        ts = eng.start_text_stream_polling(E.GenerateOptions.greedy(250), TS.TextStreamOptions(min_start_tokens=8))
        ts.push_text(TEXT)
        ts.next_codes_chunk(1)
    ts = eng.start_text_stream_polling(E.GenerateOptions.greedy(4))
    ts.finish_text()
    r = ts.next_codes_chunk(3)
    assert r.kind == TS.FINISHED and r.codes.frames == 0
    with pytest.raises(E.InvalidInputError, match="cannot push text after finish_text"):
        ts.push_text("more")
    lib = E.load_library()
    o = E.GenerateOptions.greedy(4)._c()
    h = ctypes.c_void_p()
    empty = np.zeros(1, np.int32)
    with pytest.raises(E.InvalidInputError, match="at least one content token"):
        E._check(lib.q3t_text_stream_start(eng._h, E._iptr(empty), 0, None, 0, ctypes.byref(o), ctypes.byref(h)))
    with E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=128, max_streams=2)) as e2:
        ts = e2.start_text_stream_polling(E.GenerateOptions.greedy(4), TS.TextStreamOptions(min_start_tokens=1))
        ts.push_text("hello ")
        for _ in range(4):
            r = ts.next_codes_chunk(1)
            if r.kind != TS.CHUNK:
                break
        assert r.kind == TS.NEED_MORE_TEXT and ts._stream is not None
        st = e2.start_stream([1, 2, 3], E.GenerateOptions.greedy(4))
        with pytest.raises(E.InvalidInputError, match="open text input"):
            e2.next_codes_chunks([st, ts._stream], 2)
        st.close()
        ts.close()
