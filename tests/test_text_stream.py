"""Host side of text streams (q3t.text_stream) on the CPU.

* stable_prefix_len against the oracle's byte-offset restatement (generation.rs:1439-1451);
* TextStreamOptions validation and the TextStreamInput channel, as the reference's own unit
  tests of generation.rs:1459-1490 check it;
* the queue / flush / start / resume / end logic of PollingTextStream against the token-level
  oracle (oracle/text_stream.py) over random push / pull schedules.  A stand-in for libq3t
  models the device side of an open text stream (rows pushed, the end of the text, frames
  capped at the pushed rows) and records which trailing row each frame reads; the GPU tests
  check the real library.
"""
import ctypes
import random

import numpy as np
import pytest

from oracle.text_stream import EOS, PAD, TextStreamOracle, stable_prefix_len_bytes
from q3t import engine as E
from q3t import text_stream as TS

WORDS = ["hello", "world", "the", "a", "quick", "brown", "fox", "jumps", "héllo", "中文", "naïve", "ok", "x"]
SEPS = [" ", ", ", ". ", "! ", "? ", "; ", ": ", "\n", "", "\u00a0", "\u3000", "\u2003", "\u001c"]


def toy_tokenize(text):
    """A deterministic stand-in for content_ids_for_text: one id per character."""
    return [ord(c) % 997 + 1 for c in text]


@pytest.mark.parametrize("flush", [True, False])
def test_stable_prefix_len_matches_byte_restatement(flush):
    rng = random.Random(5)
    cases = ["", "abc", "abc ", "a b c", "a.b", "end.", "x\n", "\u4e2d\u6587 \u5b57", "h\u00e9llo, w\u00f6rld",
             "a\u2003b", "a\u200bb", "\u001cab", "a\u0085b", "tab\tx", "no-split-here"]
    for _ in range(300):
        cases.append("".join(rng.choice(WORDS) + rng.choice(SEPS) for _ in range(rng.randint(0, 4))))
    for text in cases:
        got = TS.stable_prefix_len(text, flush)
        ref = stable_prefix_len_bytes(text, flush)
        if ref is None:
            assert got is None, text
        else:
            assert len(text[:got].encode("utf-8")) == ref, (text, got, ref)


def test_text_stream_options_validation():
    TS.TextStreamOptions().validate()
    o = TS.TextStreamOptions()
    assert (o.min_start_tokens, o.min_resume_tokens, o.flush_on_punctuation, o.left_context_frames) == (8, 1, True, 25)
    with pytest.raises(E.InvalidInputError, match="min_start_tokens must be non-zero"):
        TS.TextStreamOptions(min_start_tokens=0).validate()
    with pytest.raises(E.InvalidInputError, match="min_resume_tokens must be non-zero"):
        TS.TextStreamOptions(min_resume_tokens=0).validate()


def test_text_stream_input_sends_text_then_finish():
    """generation.rs:1459-1476 (text_stream_input_sends_text_then_finish)."""
    ch = TS._Channel()
    inp = TS.TextStreamInput(ch)
    inp.push_text("hello")
    assert ch.queue.get_nowait() == ("text", "hello")
    inp.push_text("")  # empty text is not sent
    assert ch.queue.empty()
    inp.finish()
    assert ch.queue.get_nowait() == ("finish", None)
    with pytest.raises(E.InvalidInputError, match="cannot push text after finish"):
        inp.push_text("again")
    inp.finish()  # a second finish sends nothing
    assert ch.queue.empty()


def test_dropping_text_stream_input_finishes_input():
    """generation.rs:1478-1490 (dropping_text_stream_input_finishes_input)."""
    ch = TS._Channel()
    inp = TS.TextStreamInput(ch)
    del inp
    assert ch.queue.get_nowait() == ("finish", None)


def test_input_after_receiver_closed():
    ch = TS._Channel()
    inp = TS.TextStreamInput(ch)
    ch.receiving = False
    with pytest.raises(E.InvalidInputError, match="no longer receiving input"):
        inp.push_text("x")


class FakeDevice:
    """The device side of libq3t's open text streams: q3t_text_stream_start / _push / _finish,
    q3t_stream_next_codes capped at the pushed rows while the text is open, and the frame
    loop's row reads (trailing row f for frame f + 1 < max_frames; after the end of the text,
    tts_eos after the last pushed row and tts_pad later).  The semantic token of frame
    eos_frame is codec EOS."""

    def __init__(self, eos_frame, groups=16):
        self.eos_frame, self.groups = eos_frame, groups
        self.streams, self.next_id = {}, 1

    def q3t_last_error(self):
        return b"fake"

    def q3t_text_stream_start(self, eng, ids, n, emb, emb_len, opts, out):
        o = opts._obj
        h = self.next_id
        self.next_id += 1
        self.streams[h] = dict(prefill=[int(v) for v in np.ctypeslib.as_array(ids, (n,))], rows=[], closed=False,
                               frame=0, max_frames=o.max_frames, done=1 if self.eos_frame == 0 else 0, reads=[])
        out._obj.value = h
        return 0

    def q3t_text_stream_push(self, h, ids, n):
        s = self.streams[h.value]
        assert not s["closed"]
        s["rows"].extend(int(v) for v in np.ctypeslib.as_array(ids, (n,)))
        return 0

    def q3t_text_stream_finish(self, h):
        self.streams[h.value]["closed"] = True
        return 0

    def q3t_stream_next_codes(self, h, max_chunk, buf, info):
        s = self.streams[h.value]
        i = info._obj
        i.frames, i.total_frames, i.ended_by_eos = 0, s["frame"], int(s["done"] == 1)
        M = s["max_frames"]
        if s["done"] or s["frame"] >= M:
            return 0
        n = min(max_chunk, M - s["frame"])
        R = len(s["rows"])
        if not s["closed"] and R < M - 1:
            n = min(n, max(0, R - s["frame"]))
        out = np.ctypeslib.as_array(buf, (max_chunk * self.groups,))
        produced = 0
        for _ in range(n):
            if s["done"]:
                break
            f = s["frame"]
            out[produced * self.groups:(produced + 1) * self.groups] = f
            if f + 1 < M:
                assert f < R or s["closed"], "frame ran without its trailing row"
                s["reads"].append(s["rows"][f] if f < R else (EOS if f == R else PAD))
                if f + 1 == self.eos_frame:
                    s["done"] = 1
            s["frame"] += 1
            produced += 1
        if s["frame"] >= M and not s["done"]:
            s["done"] = 2
        i.frames, i.total_frames, i.ended_by_eos = produced, s["frame"], int(s["done"] == 1)
        return 0

    def q3t_stream_destroy(self, h):
        return 0


class FakeEngine:
    _h = None
    code_groups = 16
    info = {"samples_per_frame": 1920}

    def content_ids(self, text):
        return toy_tokenize(text)


def _schedule(rng):
    ops = []
    for _ in range(rng.randint(0, 14)):
        r = rng.random()
        if r < 0.55:
            ops.append(("push", rng.choice(WORDS) + rng.choice(SEPS)))
        else:
            ops.append(("pull", rng.randint(1, 7)))
    ops.append(("finish", None))
    ops += [("pull", rng.randint(1, 9)) for _ in range(12)]
    return ops


@pytest.mark.parametrize("seed", range(60))
def test_polling_text_stream_matches_oracle(seed, monkeypatch):
    rng = random.Random(seed)
    min_start = rng.choice([1, 2, 3, 8])
    min_resume = rng.choice([1, 1, 2, 4])
    flush = rng.random() < 0.7
    max_frames = rng.choice([1, 2, 5, 13, 40])
    eos_frame = rng.choice([None, None, 0, 1, 3, 9])
    dev = FakeDevice(eos_frame)
    monkeypatch.setattr(E, "_lib", dev)
    opts = E.GenerateOptions.greedy(max_frames)
    monkeypatch.setattr(E.GenerateOptions, "validate", lambda self: None)
    st = TS.PollingTextStream(FakeEngine(), opts, TS.TextStreamOptions(min_start, min_resume, flush))
    ref = TextStreamOracle(toy_tokenize, max_frames, min_start, min_resume, flush, eos_frame)
    frames = 0
    for op, arg in _schedule(rng):
        if op == "push":
            st.push_text(arg)
            ref.push_text(arg)
        elif op == "finish":
            st.finish_text()
            ref.finish_text()
        else:
            r = st.next_codes_chunk(arg)
            kind, n = ref.next_codes(arg)
            got_n = r.chunk.frames if r.kind == TS.CHUNK else (r.codes.frames if r.kind == TS.FINISHED else 0)
            assert (r.kind, got_n) == (kind, n), (seed, op, arg)
            if r.kind == TS.CHUNK:
                np.testing.assert_array_equal(r.chunk.codes[:, 0], np.arange(frames, frames + n))
                frames += n
    if not (ref.ended_by_eos or ref.frame >= max_frames):
        # (a stream that ended inside a chunk may have popped ids for frames that never ran)
        assert list(st.queued_tokens) == list(ref.queue)
    if ref.started:
        s = dev.streams[1]
        assert s["prefill"] == ref.prefill_tokens
        assert st.prefill_steps == 9 + len(ref.prefill_tokens)
        assert s["reads"] == ref.trailing
    if ref.finished is not None:
        assert st.finished_codes.frames == ref.finished
        assert st.finished_codes.ended_by_eos == ref.ended_by_eos


def test_push_after_finish_text(monkeypatch):
    monkeypatch.setattr(E, "_lib", FakeDevice(None))
    monkeypatch.setattr(E.GenerateOptions, "validate", lambda self: None)
    st = TS.PollingTextStream(FakeEngine(), E.GenerateOptions.greedy(4), TS.TextStreamOptions())
    st.finish_text()
    with pytest.raises(E.InvalidInputError, match="cannot push text after finish_text"):
        st.push_text("x")
    r = st.next_codes_chunk(2)
    assert r.kind == TS.FINISHED and r.codes.frames == 0
    with pytest.raises(E.InvalidInputError, match="max_chunk_frames must be non-zero"):
        st.next_codes_chunk(0)
