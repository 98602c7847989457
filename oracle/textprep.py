"""CPU restatement of the prompt preparation that feeds the token loop.

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this module; it is the checker
that the device text preparation (q3t_prepare_text / q3t_stream_start_text) is compared
against.

Sources restated (reference = /root/reference of piedshag/qwen3-tts-hip):

* content ids, lookahead, trailing text, tts_pad row:   src/model/text.rs:340-382
* prefill layout (role, think/language/speaker rows,    src/model/text.rs:516-573
  content rows over codec pad / bos)
* text projection: fc1 + bias, SiLU, fc2 + bias          src/model/text.rs:575-603, 687-707
* codec / text embedding rows and their range checks    src/model/text.rs:605-640
* speaker / language ids from config.json                src/model/text.rs:492-505, 642-653;
                                                        src/model/config.rs:47-80
* voice clone (x-vector): the speaker row replaced by    src/model/text.rs:432-490, 507-514;
  the prompt's speaker embedding                        src/model/voice_clone.rs

Arithmetic is float64 (the reference's is float32 with a sequential fused multiply-add per
output, bias first); the weights are the bf16 values of the checkpoint.  The text-embedding
rows come from a caller-supplied function, because a synthetic checkpoint generates them
on demand instead of storing the 151,936-row table.
"""
from __future__ import annotations

import dataclasses
from typing import Callable, Dict, Sequence

import numpy as np

NEWLINE = 198  # text.rs:15


def _bf16(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


@dataclasses.dataclass
class Prepared:
    """``TtsPreparedInputs`` (text.rs:17-26) without the tokenizer's ids."""
    prefill: np.ndarray        # [9 + lookahead, H]
    trailing_text: np.ndarray  # [content - lookahead + 1, H]
    tts_pad_embed: np.ndarray  # [H]


class TextPrepOracle:
    def __init__(self, tensors: Dict[str, np.ndarray], config: dict,
                 text_rows: Callable[[np.ndarray], np.ndarray], text_vocab: int):
        self.fc1_w = _bf16(tensors["talker.text_projection.linear_fc1.weight"])
        self.fc1_b = _bf16(tensors["talker.text_projection.linear_fc1.bias"])
        self.fc2_w = _bf16(tensors["talker.text_projection.linear_fc2.weight"])
        self.fc2_b = _bf16(tensors["talker.text_projection.linear_fc2.bias"])
        self.codec_emb = _bf16(tensors["talker.model.codec_embedding.weight"])
        self.text_rows = text_rows
        self.text_vocab = text_vocab
        tc = config["talker_config"]
        self.tok = dict(
            im_start=config["im_start_token_id"], assistant=config["assistant_token_id"],
            tts_pad=config["tts_pad_token_id"], tts_bos=config["tts_bos_token_id"],
            tts_eos=config["tts_eos_token_id"], codec_pad=tc["codec_pad_id"], codec_bos=tc["codec_bos_id"],
            codec_think=tc["codec_think_id"], codec_think_bos=tc["codec_think_bos_id"],
            codec_think_eos=tc["codec_think_eos_id"])
        self.speaker_ids = tc["spk_id"]
        self.language_ids = tc["codec_language_id"]

    # text.rs:575-603: per token, fc1 (+ bias) -> SiLU -> fc2 (+ bias)
    def projected(self, tokens: Sequence[int]) -> np.ndarray:
        ids = np.asarray(list(tokens), dtype=np.int64)
        for t in ids:
            if not 0 <= t < self.text_vocab:  # text.rs:622-630
                raise ValueError(f"text token {t} is out of range for vocab {self.text_vocab}")
        x = self.text_rows(ids).astype(np.float64)
        h = x @ self.fc1_w.T + self.fc1_b
        h = h / (1.0 + np.exp(-h))
        return h @ self.fc2_w.T + self.fc2_b

    # text.rs:605-620
    def codec(self, tokens: Sequence[int]) -> np.ndarray:
        for t in tokens:
            if not 0 <= t < self.codec_emb.shape[0]:
                raise ValueError(f"codec token {t} is out of range for vocab {self.codec_emb.shape[0]}")
        return self.codec_emb[list(tokens)]

    # text.rs:516-573 (speaker: a config key, or an x-vector row of width H)
    def prefill(self, text_tokens: Sequence[int], speaker, language: str) -> np.ndarray:
        t = self.tok
        if isinstance(speaker, str) and speaker not in self.speaker_ids:
            raise ValueError(f"missing speaker token id for {speaker}")
        if language not in self.language_ids:
            raise ValueError(f"missing language token id for {language}")
        role = self.projected([t["im_start"], t["assistant"], NEWLINE])
        spk_id = self.speaker_ids[speaker] if isinstance(speaker, str) else t["codec_pad"]
        codec = self.codec([t["codec_think"], t["codec_think_bos"], self.language_ids[language],
                            t["codec_think_eos"], spk_id, t["codec_pad"], t["codec_bos"]])
        if not isinstance(speaker, str):
            xvec = np.asarray(speaker, dtype=np.float64)
            if xvec.shape != (codec.shape[1],):  # text.rs:445-451, 521-527
                raise ValueError(f"speaker embedding length {xvec.size} does not match hidden {codec.shape[1]}")
            codec = codec.copy()
            codec[4] = xvec
        tts = self.projected([t["tts_pad"]] * 5 + [t["tts_bos"]])
        rows = [role] + [tts[i] + codec[i] for i in range(6)]
        text = self.projected(text_tokens) if len(text_tokens) else np.zeros((0, codec.shape[1]))
        for i in range(len(text_tokens)):
            rows.append(text[i] + codec[6 if i + 1 == len(text_tokens) else 5])
        return np.vstack([np.atleast_2d(r) for r in rows])

    # text.rs:340-382; text.rs:432-490 with an x-vector as `speaker`
    def prepare(self, content_ids: Sequence[int], speaker="ryan", language: str = "english",
                text_lookahead_tokens: int = 1) -> Prepared:
        if text_lookahead_tokens == 0:
            raise ValueError("text_lookahead_tokens must be non-zero")
        content = [int(c) for c in content_ids]
        look = 0 if not content else max(1, min(text_lookahead_tokens, len(content)))
        prefill = self.prefill(content[:look], speaker, language)
        trailing = content[look:] + [self.tok["tts_eos"]]
        return Prepared(prefill=prefill, trailing_text=self.projected(trailing),
                        tts_pad_embed=self.projected([self.tok["tts_pad"]])[0])
