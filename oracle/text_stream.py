"""CPU restatement of the text handling of a text stream, at the token level.

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this module; it is the checker the
host side of q3t.text_stream (its queue, flush, start and resume rules, and which trailing row
each frame reads) is compared against.

Sources restated (reference = /root/reference of piedshag/qwen3-tts-hip):

* stable_prefix_len / is_sentence_boundary:        src/generation.rs:1439-1451
* push_text / finish_text / flush / enqueue:       src/generation.rs:1108-1129, 1390-1412
* next_audio_chunk's start / finish decisions:     src/generation.rs:1132-1160
* next_codes_chunk's frame loop (EOS check first,  src/generation.rs:1183-1270
  then the trailing row when frame + 1 < max_frames)
* try_start_generation:                            src/generation.rs:1280-1358
* next_trailing_buffer:                            src/generation.rs:1360-1388

The Talker and CodePredictor are not modelled: a frame's semantic token is EOS exactly at
frame ``eos_frame`` (None: never), which is all the loop's control flow reads from them.
``stable_prefix_len`` works on UTF-8 bytes, as the reference does.
"""
from __future__ import annotations

from collections import deque
from typing import Callable, List, Optional, Sequence, Tuple

_WHITE_SPACE = {0x09, 0x0A, 0x0B, 0x0C, 0x0D, 0x20, 0x85, 0xA0, 0x1680, *range(0x2000, 0x200B), 0x2028, 0x2029,
                0x202F, 0x205F, 0x3000}


def stable_prefix_len_bytes(text: str, flush_on_punctuation: bool) -> Optional[int]:
    """generation.rs:1439-1447: byte offset just past the last whitespace / boundary char."""
    split, offset = None, 0
    for ch in text:
        n = len(ch.encode("utf-8"))
        if ord(ch) in _WHITE_SPACE or (flush_on_punctuation and ch in ".,;:!?\n"):
            split = offset + n
        offset += n
    return split


EOS, PAD = "tts_eos", "tts_pad"


class TextStreamOracle:
    def __init__(self, tokenize: Callable[[str], Sequence[int]], max_frames: int, min_start_tokens: int = 8,
                 min_resume_tokens: int = 1, flush_on_punctuation: bool = True, eos_frame: Optional[int] = None):
        self.tokenize = tokenize
        self.max_frames = max_frames
        self.min_start, self.min_resume = min_start_tokens, min_resume_tokens
        self.flush_on_punctuation = flush_on_punctuation
        self.eos_frame = eos_frame
        self.pending = b""
        self.queue: deque = deque()
        self.text_finished = self.eos_pending = self.eos_consumed = False
        self.started = False
        self.prefill_tokens: List[int] = []
        self.frame = 0
        self.ended_by_eos = False
        self.finished: Optional[int] = None
        self.trailing: List[object] = []  # what the Talker step after frame f read: token id, EOS or PAD

    def push_text(self, text: str) -> None:
        if self.text_finished:
            raise ValueError("cannot push text after finish_text")
        self.pending += text.encode("utf-8")
        split = stable_prefix_len_bytes(self.pending.decode("utf-8"), self.flush_on_punctuation)
        if split:
            prefix, self.pending = self.pending[:split], self.pending[split:]
            self.queue.extend(self.tokenize(prefix.decode("utf-8")))

    def finish_text(self) -> None:
        if self.text_finished:
            return
        if self.pending:
            self.queue.extend(self.tokenize(self.pending.decode("utf-8")))
            self.pending = b""
        self.text_finished = True
        self.eos_pending = True

    def _try_start(self) -> bool:
        if self.started:
            return True
        if len(self.queue) < self.min_start and not self.text_finished:
            return False
        if not self.queue:
            return False
        look = max(1, min(self.min_start, len(self.queue)))
        self.prefill_tokens = [self.queue.popleft() for _ in range(look)]
        self.started = True
        return True

    def _next_trailing(self):
        if not self.text_finished and len(self.queue) < self.min_resume:
            return None
        if self.queue:
            return self.queue.popleft()
        if self.eos_pending:
            self.eos_pending = False
            self.eos_consumed = True
            return EOS
        if self.text_finished or self.eos_consumed:
            return PAD
        return None

    def _generation_finished(self) -> bool:
        return self.started and (self.ended_by_eos or self.frame >= self.max_frames)

    def next_codes(self, max_chunk: int) -> Tuple[str, int]:
        """("chunk", frames) | ("need_more_text", 0) | ("finished", total frames)."""
        if self.finished is not None:
            return "finished", self.finished
        if not self.started and not self._try_start():
            if self.text_finished and not self.queue and self.eos_pending:
                self.finished = 0
                return "finished", 0
            return "need_more_text", 0
        produced = 0
        if not (self.ended_by_eos or self.frame >= self.max_frames):
            while produced < max_chunk and self.frame < self.max_frames:
                if self.frame == self.eos_frame:
                    self.ended_by_eos = True
                    break
                trailing = None
                if self.frame + 1 < self.max_frames:
                    trailing = self._next_trailing()
                    if trailing is None:
                        break
                    self.trailing.append(trailing)
                produced += 1
                self.frame += 1
            if self.frame < self.max_frames and self.frame == self.eos_frame:
                self.ended_by_eos = True
        if produced == 0:
            if self._generation_finished():
                self.finished = self.frame
                return "finished", self.frame
            return "need_more_text", 0
        return "chunk", produced
