"""Text streams: text pushed while audio is produced.

Mirror of ``TextStreamOptions``, ``IncrementalAudio``, ``PollingTextStream``,
``HipTextStream`` and ``TextStreamInput`` (src/generation.rs:165-235, 1004-1451).  The host
keeps the reference's text state: the pending text, the flush rule that cuts it at a stable
boundary, the queue of content ids and the start / resume thresholds.  The device holds the
prompt rows and the trailing text rows, and its frame loop runs a frame only once that
frame's trailing row has been pushed (``q3t_text_stream_start`` / ``q3t_text_stream_push`` /
``q3t_text_stream_finish``).

A text stream that receives all of its text before the first pull produces the same codes as
``start_stream`` with ``text_lookahead_tokens = min_start_tokens`` over the same content ids:
stalls only delay frames, they change no state the frames read.
"""
from __future__ import annotations

import collections
import ctypes
import dataclasses
import queue
import threading
from typing import Optional, Tuple

import numpy as np

from . import engine as E
from .voice_clone import VoiceClonePrompt

# char::is_whitespace (the Unicode White_Space property), which stable_prefix_len splits on.
WHITE_SPACE = frozenset(chr(c) for c in (*range(0x09, 0x0E), 0x20, 0x85, 0xA0, 0x1680, *range(0x2000, 0x200B),
                                         0x2028, 0x2029, 0x202F, 0x205F, 0x3000))
SENTENCE_BOUNDARIES = frozenset(".,;:!?\n")  # is_sentence_boundary (generation.rs:1449-1451)


def stable_prefix_len(text: str, flush_on_punctuation: bool) -> Optional[int]:
    """``stable_prefix_len`` (generation.rs:1439-1447): the length of the longest prefix of
    ``text`` that ends in whitespace (or, with ``flush_on_punctuation``, a sentence boundary),
    or None.  Counted in characters; the reference counts UTF-8 bytes of the same prefix."""
    split = None
    for i, ch in enumerate(text):
        if ch in WHITE_SPACE or (flush_on_punctuation and ch in SENTENCE_BOUNDARIES):
            split = i + 1
    return split


@dataclasses.dataclass
class TextStreamOptions:
    """``TextStreamOptions`` (generation.rs:212-228)."""
    min_start_tokens: int = E.DEFAULT_TEXT_LOOKAHEAD_TOKENS
    min_resume_tokens: int = 1
    flush_on_punctuation: bool = True
    left_context_frames: int = E.DEFAULT_STREAM_LEFT_CONTEXT_FRAMES

    def validate(self) -> None:
        """``validate_text_stream_options`` (generation.rs:594-606)."""
        if self.min_start_tokens <= 0:
            raise E.InvalidInputError(E.Q3T_ERR_INVALID, "min_start_tokens must be non-zero")
        if self.min_resume_tokens <= 0:
            raise E.InvalidInputError(E.Q3T_ERR_INVALID, "min_resume_tokens must be non-zero")


CHUNK, NEED_MORE_TEXT, FINISHED = "chunk", "need_more_text", "finished"


@dataclasses.dataclass
class IncrementalAudio:
    """``IncrementalAudio`` (generation.rs:230-235): ``kind`` is CHUNK (``chunk`` set),
    NEED_MORE_TEXT, or FINISHED (``codes`` = every code of the stream)."""
    kind: str
    chunk: Optional[E.GeneratedAudioChunk] = None
    codes: Optional[E.GeneratedCodes] = None


@dataclasses.dataclass
class IncrementalCodes:
    """As :class:`IncrementalAudio` for a pull of codes without decoding (the reference's
    private ``next_codes_chunk`` with its ``NeedMoreText`` / ``Finished`` outcomes)."""
    kind: str
    chunk: Optional[E.GeneratedCodesChunk] = None
    codes: Optional[E.GeneratedCodes] = None


class PollingTextStream:
    """``PollingTextStream`` (generation.rs:176-211, 1093-1437).  Must not outlive its engine."""

    def __init__(self, engine: "E.HipTtsEngine", options: E.GenerateOptions, stream_options: TextStreamOptions,
                 voice_clone_prompt: Optional[VoiceClonePrompt] = None):
        options.validate()
        stream_options.validate()
        self.engine = engine
        self.options = options
        self.stream_options = stream_options
        self.voice_clone_prompt = voice_clone_prompt
        self.pending_text = ""
        self.queued_tokens: collections.deque = collections.deque()
        self.text_finished = False
        self.eos_pending = False
        self.eos_consumed = False
        self._stream: Optional[E.HipTtsStream] = None
        self._rows = 0               # trailing rows pushed to the device
        self._device_closed = False  # q3t_text_stream_finish done
        self.finished_codes: Optional[E.GeneratedCodes] = None

    # -- text input ----------------------------------------------------------------------
    def push_text(self, text: str) -> None:
        """``push_text`` (generation.rs:1108-1116)."""
        if self.text_finished:
            raise E.InvalidInputError(E.Q3T_ERR_INVALID, "cannot push text after finish_text")
        self.pending_text += text
        self._flush_stable_text()

    def finish_text(self) -> None:
        """``finish_text`` (generation.rs:1118-1129)."""
        if self.text_finished:
            return
        if self.pending_text:
            text, self.pending_text = self.pending_text, ""
            self._enqueue_text_tokens(text)
        self.text_finished = True
        self.eos_pending = True

    def _flush_stable_text(self) -> None:
        # flush_stable_text (generation.rs:1390-1403)
        split = stable_prefix_len(self.pending_text, self.stream_options.flush_on_punctuation)
        if not split:
            return
        prefix, self.pending_text = self.pending_text[:split], self.pending_text[split:]
        self._enqueue_text_tokens(prefix)

    def _enqueue_text_tokens(self, text: str) -> None:
        # enqueue_text_tokens (generation.rs:1405-1412): content_ids_for_text of the piece
        if text:
            self.queued_tokens.extend(self.engine.content_ids(text))

    # -- generation ----------------------------------------------------------------------
    def _try_start_generation(self) -> bool:
        # try_start_generation (generation.rs:1280-1358)
        if self._stream is not None:
            return True
        if len(self.queued_tokens) < self.stream_options.min_start_tokens and not self.text_finished:
            return False
        if not self.queued_tokens:
            return False
        look = max(1, min(self.stream_options.min_start_tokens, len(self.queued_tokens)))
        ids = np.array([self.queued_tokens.popleft() for _ in range(look)], dtype=np.int32)
        emb, emb_len = None, 0
        if self.voice_clone_prompt is not None:
            self.voice_clone_prompt.check_x_vector_only()
            emb_arr = np.ascontiguousarray(np.asarray(self.voice_clone_prompt.speaker_embedding,
                                                      dtype=np.float32).reshape(-1))
            emb, emb_len = E._fptr(emb_arr), int(emb_arr.size)
        o = self.options._c()
        handle = ctypes.c_void_p()
        E._check(E._lib.q3t_text_stream_start(self.engine._h, E._iptr(ids), int(ids.size), emb, emb_len,
                                              ctypes.byref(o), ctypes.byref(handle)))
        self._stream = E.HipTtsStream(
            self.engine, None, self.options,
            E.StreamOptions(left_context_frames=self.stream_options.left_context_frames),
            handle=handle, prefill_steps=9 + look)
        return True

    def _feed(self, max_chunk_frames: int) -> int:
        """Pops the content ids the next ``max_chunk_frames`` frames read as the reference's
        ``next_trailing_buffer`` would (generation.rs:1360-1388), pushes them to the device
        (and the end of the text, once reached), and returns the number of frames that may run."""
        F, M = self._stream.frame, self.options.max_frames
        push, close, n = [], False, 0
        while n < max_chunk_frames and F + n < M:
            f = F + n
            if f + 1 < M and not (self._device_closed or close) and f >= self._rows + len(push):
                if not self.text_finished and len(self.queued_tokens) < self.stream_options.min_resume_tokens:
                    break
                if self.queued_tokens:
                    push.append(self.queued_tokens.popleft())
                else:  # the text is finished: tts_eos, then tts_pad for every later frame
                    if self.eos_pending:
                        self.eos_pending = False
                        self.eos_consumed = True
                    close = True
            n += 1
        if push:
            ids = np.array(push, dtype=np.int32)
            E._check(E._lib.q3t_text_stream_push(self._stream._h, E._iptr(ids), int(ids.size)))
            self._rows += len(push)
        if close:
            E._check(E._lib.q3t_text_stream_finish(self._stream._h))
            self._device_closed = True
        return n

    def _generation_finished(self) -> bool:
        s = self._stream
        return s is not None and (s.ended_by_eos or s.frame >= self.options.max_frames)

    def _finish_codes(self) -> E.GeneratedCodes:
        s = self._stream
        if s is None:
            codes = E.GeneratedCodes(np.zeros((0, self.engine.code_groups), np.int32), 0, False)
        else:
            c = (np.concatenate(s._codes) if s._codes else np.zeros((0, self.engine.code_groups), np.int32))
            codes = E.GeneratedCodes(c, int(c.shape[0]), s.ended_by_eos)
            s.close()  # the codes are on the host: free the slot
        self.finished_codes = codes
        return codes

    def _pull(self, max_chunk_frames: int, audio: bool):
        if max_chunk_frames <= 0:
            raise E.InvalidInputError(E.Q3T_ERR_INVALID, "max_chunk_frames must be non-zero")
        if self.finished_codes is not None:
            return FINISHED, None, self.finished_codes
        if self._stream is None and not self._try_start_generation():
            if self.text_finished and not self.queued_tokens and self.eos_pending:
                return FINISHED, None, self._finish_codes()
            return NEED_MORE_TEXT, None, None
        n = self._feed(max_chunk_frames)
        # With n = 0 the device runs nothing (no trailing row for the next frame) and reports
        # whether the stream has ended.
        pull = self._stream.next_audio_chunk if audio else self._stream.next_codes_chunk
        chunk = pull(max(n, 1))
        if chunk is None:
            if self._generation_finished():
                return FINISHED, None, self._finish_codes()
            return NEED_MORE_TEXT, None, None
        return CHUNK, chunk, None

    def next_audio_chunk(self, max_chunk_frames: int) -> IncrementalAudio:
        """``next_audio_chunk`` (generation.rs:1132-1180)."""
        return IncrementalAudio(*self._pull(max_chunk_frames, True))

    def next_codes_chunk(self, max_chunk_frames: int) -> IncrementalCodes:
        """The codes of ``next_audio_chunk`` without decoding them."""
        return IncrementalCodes(*self._pull(max_chunk_frames, False))

    @property
    def prefill_steps(self) -> Optional[int]:
        return None if self._stream is None else self._stream.prefill_steps

    def close(self) -> None:
        if self._stream is not None:
            self._stream.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class _Channel:
    def __init__(self):
        self.queue: "queue.Queue[Tuple[str, Optional[str]]]" = queue.Queue()
        self.receiving = True
        self.lock = threading.Lock()

    def send(self, msg: Tuple[str, Optional[str]]) -> None:
        with self.lock:
            if not self.receiving:
                raise E.InvalidInputError(E.Q3T_ERR_INVALID, "text stream is no longer receiving input")
            self.queue.put(msg)


class TextStreamInput:
    """``TextStreamInput`` (generation.rs:171-174, 1004-1044): the sending end of a
    :class:`HipTextStream`.  Dropping it finishes the text."""

    def __init__(self, channel: _Channel):
        self._channel = channel
        self.finished = False

    def push_text(self, text: str) -> None:
        if self.finished:
            raise E.InvalidInputError(E.Q3T_ERR_INVALID, "cannot push text after finish")
        if text:
            self._channel.send(("text", text))

    def finish(self) -> None:
        if self.finished:
            return
        self.finished = True
        self._channel.send(("finish", None))

    def __del__(self):
        if not getattr(self, "finished", True):
            try:
                self._channel.send(("finish", None))
            except Exception:
                pass


class HipTextStream:
    """``HipTextStream`` (generation.rs:165-169, 1046-1091): a polling text stream that waits
    on its :class:`TextStreamInput` whenever the next frame needs more text."""

    def __init__(self, stream: PollingTextStream):
        self._channel = _Channel()
        self.stream = stream
        self._finished_codes: Optional[E.GeneratedCodes] = None

    def _input(self) -> TextStreamInput:
        return TextStreamInput(self._channel)

    def next_audio_chunk(self, max_chunk_frames: int) -> Optional[E.GeneratedAudioChunk]:
        if self._finished_codes is not None:
            return None
        while True:
            r = self.stream.next_audio_chunk(max_chunk_frames)
            if r.kind == CHUNK:
                return r.chunk
            if r.kind == FINISHED:
                self._finished_codes = r.codes
                return None
            if self.stream.text_finished:  # finished text never waits; do not block on the channel
                raise E.Q3tError(E.Q3T_ERR_INVALID, "text stream waits for text after finish_text")
            kind, text = self._channel.queue.get()
            if kind == "text":
                self.stream.push_text(text)
            else:
                self.stream.finish_text()

    def finished_codes(self) -> Optional[E.GeneratedCodes]:
        return self._finished_codes

    def close(self) -> None:
        with self._channel.lock:
            self._channel.receiving = False
        self.stream.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
