"""Voice-clone prompts: ``VoiceClonePrompt`` of src/model/voice_clone.rs.

A prompt file is JSON with a ``speaker_embedding`` array (one float per Talker hidden unit,
the x-vector a speaker encoder produced from reference audio) and the optional fields
``x_vector_only_mode``, ``icl_mode``, ``ref_text`` and ``ref_codes`` (voice_clone.rs:17-28).
Only x-vector prompts drive generation: the speaker embedding takes the place of the
speaker's codec-embedding row in the prefill (text.rs:432-514); ICL prompts are rejected as
the reference rejects them (text.rs:439-443).
"""
from __future__ import annotations

import dataclasses
import json
import os
from typing import List, Optional, Union

import numpy as np


class VoiceClonePromptError(ValueError):
    """``Error::InvalidInput`` raised while reading or applying a voice-clone prompt."""


@dataclasses.dataclass
class VoiceClonePrompt:
    speaker_embedding: np.ndarray
    x_vector_only_mode: bool = False
    icl_mode: bool = False
    ref_text: Optional[str] = None
    ref_codes: Optional[List[int]] = None

    @classmethod
    def from_json(cls, path: Union[str, os.PathLike]) -> "VoiceClonePrompt":
        """``VoiceClonePrompt::from_json`` (voice_clone.rs:30-45)."""
        try:
            with open(path, "rb") as f:
                data = f.read()
        except OSError as err:
            raise VoiceClonePromptError(f"failed to read {path}: {err}") from None
        try:
            raw = json.loads(data)
            if not isinstance(raw, dict):
                raise ValueError("expected a JSON object")
            if "speaker_embedding" not in raw:
                raise ValueError("missing field `speaker_embedding`")
            emb = raw["speaker_embedding"]
            if not isinstance(emb, list) or not all(isinstance(v, (int, float)) and not isinstance(v, bool)
                                                    for v in emb):
                raise ValueError("`speaker_embedding` must be an array of numbers")
            ref_codes = raw.get("ref_codes")
            if ref_codes is not None and (not isinstance(ref_codes, list)
                                          or not all(isinstance(v, int) and not isinstance(v, bool)
                                                     and -2**31 <= v < 2**31 for v in ref_codes)):
                raise ValueError("`ref_codes` must be an array of 32-bit integers")
            ref_text = raw.get("ref_text")
            if ref_text is not None and not isinstance(ref_text, str):
                raise ValueError("`ref_text` must be a string")
            flags = {k: raw.get(k, False) for k in ("x_vector_only_mode", "icl_mode")}
            for k, v in flags.items():
                if not isinstance(v, bool):
                    raise ValueError(f"`{k}` must be a boolean")
        except ValueError as err:
            raise VoiceClonePromptError(f"failed to parse {path}: {err}") from None
        return cls(speaker_embedding=np.asarray(emb, dtype=np.float32), ref_text=ref_text, ref_codes=ref_codes,
                   **flags)

    def check_x_vector_only(self) -> None:
        """The prompt kinds ``prepare_voice_clone_xvector_with_lookahead`` accepts (text.rs:439-443)."""
        if not self.x_vector_only_mode or self.icl_mode or self.ref_codes is not None:
            raise VoiceClonePromptError("only x-vector-only voice clone prompts are supported for now")

    def to_json(self, path: Union[str, os.PathLike]) -> None:
        doc = {"speaker_embedding": [float(v) for v in np.asarray(self.speaker_embedding, np.float32)],
               "x_vector_only_mode": bool(self.x_vector_only_mode), "icl_mode": bool(self.icl_mode)}
        if self.ref_text is not None:
            doc["ref_text"] = self.ref_text
        if self.ref_codes is not None:
            doc["ref_codes"] = [int(c) for c in self.ref_codes]
        with open(path, "w") as f:
            json.dump(doc, f)
