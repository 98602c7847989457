"""Host-side prompt preparation: token ids -> the [P, H] prefill, trailing text rows and tts_pad row.

This runs on the CPU before the token loop, as it does in the reference
(src/model/text.rs:340-382, :516-603); HipTtsEngine.prepare_text does the same on the GPU.
Callers pass content token ids (the ids between the chat-template prefix and suffix,
text.rs:361), which q3t.tokenizer produces from text.  Layout of the prefill (text.rs:516-573):

    3 rows   text_proj([im_start, assistant, "\\n"])
    6 rows   text_proj([pad, pad, pad, pad, pad, bos])[i] + codec_emb([think, think_bos,
             language, think_eos, <speaker>, pad])[i]
    L rows   text_proj(content[i]) + codec_emb(pad)   (codec_emb(bos) on the last row)

so P = 9 + L.  ``text_proj`` is the two-layer SiLU MLP of text.rs:575-603 applied to
rows of the text-embedding table.
"""
from __future__ import annotations

import dataclasses
from typing import Sequence

import numpy as np

from . import synth

NEWLINE = 198


@dataclasses.dataclass
class PreparedInputs:
    """Mirror of the reference's ``TtsPreparedInputs`` (text.rs:17-26)."""
    content_ids: np.ndarray
    prefill: np.ndarray          # [P, H] float32
    trailing_text: np.ndarray    # [T, H] float32
    tts_pad_embed: np.ndarray    # [H] float32

    @property
    def prefill_steps(self) -> int:
        return int(self.prefill.shape[0])

    @property
    def trailing_steps(self) -> int:
        return int(self.trailing_text.shape[0])


class TextPrep:
    def __init__(self, model: "synth.SyntheticModel"):
        self.model = model
        self.spec = model.spec
        cfg = model.config()
        self.tokens = dict(synth.TOKENS)
        self.language_ids = cfg["talker_config"]["codec_language_id"]
        self.speaker_ids = cfg["talker_config"]["spk_id"]
        f64 = lambda n: model.f32(n).astype(np.float64)
        self.fc1_w = f64("talker.text_projection.linear_fc1.weight")
        self.fc1_b = f64("talker.text_projection.linear_fc1.bias")
        self.fc2_w = f64("talker.text_projection.linear_fc2.weight")
        self.fc2_b = f64("talker.text_projection.linear_fc2.bias")
        self.codec_emb = model.f32("talker.model.codec_embedding.weight")

    def projected_text_embeddings(self, tokens: Sequence[int]) -> np.ndarray:
        rows = synth.text_embedding_rows(self.model.seed, np.asarray(tokens), self.spec.text_hidden)
        h = rows.astype(np.float64) @ self.fc1_w.T + self.fc1_b
        h = h / (1.0 + np.exp(-h))
        return (h @ self.fc2_w.T + self.fc2_b).astype(np.float32)

    def codec_embeddings(self, tokens: Sequence[int]) -> np.ndarray:
        tokens = list(tokens)
        for t in tokens:
            if not 0 <= t < self.codec_emb.shape[0]:
                raise ValueError(f"codec token {t} is out of range for vocab {self.codec_emb.shape[0]}")
        return self.codec_emb[tokens].astype(np.float32)

    def build_prefill(self, text_tokens: Sequence[int], speaker: str, language: str) -> np.ndarray:
        t = self.tokens
        speaker_id = self.speaker_ids[speaker.lower()]
        language_id = self.language_ids[language.lower()]
        role = self.projected_text_embeddings([t["im_start_token_id"], t["assistant_token_id"], NEWLINE])
        codec = self.codec_embeddings([t["codec_think_id"], t["codec_think_bos_id"], language_id,
                                       t["codec_think_eos_id"], speaker_id, t["codec_pad_id"],
                                       t["codec_bos_id"]])
        pad, bos = t["tts_pad_token_id"], t["tts_bos_token_id"]
        tts = self.projected_text_embeddings([pad, pad, pad, pad, pad, bos])
        rows = [role, tts + codec[:6]]
        if len(text_tokens):
            text = self.projected_text_embeddings(text_tokens)
            codec_rows = np.repeat(codec[5:6], len(text_tokens), axis=0)
            codec_rows[-1] = codec[6]
            rows.append(text + codec_rows)
        return np.concatenate(rows, axis=0).astype(np.float32)

    def prepare(self, content_ids: Sequence[int], speaker: str = "ryan", language: str = "english",
                text_lookahead_tokens: int = 1 << 30) -> PreparedInputs:
        """``prepare_custom_voice_with_lookahead`` (text.rs:340-382)."""
        if text_lookahead_tokens <= 0:
            raise ValueError("text_lookahead_tokens must be non-zero")
        content = [int(c) for c in content_ids]
        lookahead = 0 if not content else max(1, min(text_lookahead_tokens, len(content)))
        prefill = self.build_prefill(content[:lookahead], speaker, language)
        trailing = content[lookahead:] + [self.tokens["tts_eos_token_id"]]
        return PreparedInputs(
            content_ids=np.asarray(content, dtype=np.int64),
            prefill=prefill,
            trailing_text=self.projected_text_embeddings(trailing),
            tts_pad_embed=self.projected_text_embeddings([self.tokens["tts_pad_token_id"]])[0],
        )


def random_prompt(n_tokens: int, seed: int) -> np.ndarray:
    """Content ids uniform in [0, 151643) (32 ids, seed 1)."""
    return np.random.default_rng(seed).integers(0, 151643, n_tokens)
