"""Host-side text tokenizer: ``TextTokenizer`` (reference src/model/text.rs:156-247).

The reference builds its tokenizer with the Rust ``tokenizers`` crate 0.22.2
(Cargo.lock); the Python ``tokenizers`` package wraps the same library, and this module
loads the model directory's files the same way:

* ``tokenizer.json`` when present (``Tokenizer::from_file``);
* else ``vocab.json`` + ``merges.txt``: a byte-level BPE with a ByteLevel pre-tokenizer
  (no prefix space), decoder and post-processor (trim_offsets false), plus the added tokens
  of ``tokenizer_config.json``'s ``added_tokens_decoder`` in id order (text.rs:195-237).

``encode`` adds no special tokens (text.rs:240-247).  ``content_ids`` wraps the text in the
chat template and keeps the ids between its 3-token prefix and 5-token suffix
(text.rs:384-395).
"""
from __future__ import annotations

import json
import os
from typing import List


class TokenizerError(ValueError):
    pass


CHAT_TEMPLATE = "<|im_start|>assistant\n{text}<|im_end|>\n<|im_start|>assistant\n"


class TextTokenizer:
    def __init__(self, tokenizer):
        self._tok = tokenizer

    @classmethod
    def from_pretrained(cls, path: str) -> "TextTokenizer":
        from tokenizers import Tokenizer

        if os.path.isdir(path):
            tj = os.path.join(path, "tokenizer.json")
            if os.path.exists(tj):
                return cls._from_file(tj)
            vocab, merges = os.path.join(path, "vocab.json"), os.path.join(path, "merges.txt")
            if os.path.exists(vocab) and os.path.exists(merges):
                return cls._from_bpe_files(path, vocab, merges)
            raise TokenizerError(f"tokenizer files not found under {path}; expected tokenizer.json or "
                                 "vocab.json + merges.txt")
        return cls._from_file(path)

    @classmethod
    def _from_file(cls, path: str) -> "TextTokenizer":
        from tokenizers import Tokenizer

        try:
            return cls(Tokenizer.from_file(path))
        except Exception as err:  # the library raises its own exception type
            raise TokenizerError(f"failed to load tokenizer from {path}: {err}") from err

    @classmethod
    def _from_bpe_files(cls, root: str, vocab: str, merges: str) -> "TextTokenizer":
        from tokenizers import AddedToken, Tokenizer, decoders, models, pre_tokenizers, processors

        try:
            bpe = models.BPE.from_file(vocab, merges)
        except Exception as err:
            raise TokenizerError(f"failed to load BPE tokenizer: {err}") from err
        tok = Tokenizer(bpe)
        tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
        tok.decoder = decoders.ByteLevel()
        tok.post_processor = processors.ByteLevel(trim_offsets=False)
        cfg_path = os.path.join(root, "tokenizer_config.json")
        if os.path.exists(cfg_path):
            with open(cfg_path) as f:
                cfg = json.load(f)
            entries = []
            for key, t in cfg.get("added_tokens_decoder", {}).items():
                try:
                    entries.append((int(key), t))
                except ValueError as err:
                    raise TokenizerError(f"invalid added token id: {err}") from err
            entries.sort(key=lambda e: e[0])
            tok.add_tokens([AddedToken(t["content"], special=t.get("special", False),
                                       single_word=t.get("single_word", False), lstrip=t.get("lstrip", False),
                                       rstrip=t.get("rstrip", False), normalized=t.get("normalized", False))
                            for _, t in entries])
        return cls(tok)

    def encode(self, text: str) -> List[int]:
        try:
            return list(self._tok.encode(text, add_special_tokens=False).ids)
        except Exception as err:
            raise TokenizerError(f"failed to encode text: {err}") from err

    def content_ids(self, text: str) -> List[int]:
        """``content_ids_for_text`` (text.rs:384-395)."""
        ids = self.encode(CHAT_TEMPLATE.format(text=text))
        if len(ids) < 8:
            raise TokenizerError(f"formatted prompt is too short: {len(ids)} tokens")
        return ids[3:len(ids) - 5]
