"""Host tokenizer (q3t/tokenizer.py, text.rs:156-247 and 384-395) on the synthetic byte-level
BPE files: known answers for the chat-template encoding and the content-id slice, byte
fallback for text the merges do not cover, both file forms (vocab.json + merges.txt with
tokenizer_config.json's added tokens, and tokenizer.json) and the missing-files error.  The
real Qwen vocabulary does not ship offline, so its ids are parity unpinned; the library is
the one the reference links (tokenizers 0.22.2)."""
import os

import pytest

from q3t import synth
from q3t.tokenizer import TextTokenizer, TokenizerError


@pytest.fixture(scope="module")
def tok_dir(tmp_path_factory):
    d = str(tmp_path_factory.mktemp("tok"))
    synth.write_tokenizer(d)
    return d


def byte_ids(text: str):
    alphabet = synth.byte_level_alphabet()
    bs = list(range(ord("!"), ord("~") + 1)) + list(range(0xA1, 0xAD)) + list(range(0xAE, 0x100))
    order = bs + [b for b in range(256) if b not in bs]
    assert len(order) == len(alphabet) == 256
    return [order.index(b) for b in text.encode()]


def test_chat_template_known_answer(tok_dir):
    t = TextTokenizer.from_pretrained(tok_dir)
    ids = t.encode("<|im_start|>assistant\nhello world<|im_end|>\n<|im_start|>assistant\n")
    assert ids == [151644, 77091, 198, 9707, 1879, 151645, 198, 151644, 77091, 198]
    assert t.content_ids("hello world") == [9707, 1879]


def test_byte_fallback(tok_dir):
    t = TextTokenizer.from_pretrained(tok_dir)
    assert byte_ids("\n") == [198]
    assert t.content_ids("héllo!\n") == byte_ids("héllo!\n")


def test_tokenizer_json_form_agrees(tok_dir, tmp_path):
    t = TextTokenizer.from_pretrained(tok_dir)
    t._tok.save(str(tmp_path / "tokenizer.json"))
    t2 = TextTokenizer.from_pretrained(str(tmp_path))
    text = "hello world, helloé world!"
    assert t2.content_ids(text) == t.content_ids(text)


def test_missing_files(tmp_path):
    with pytest.raises(TokenizerError, match="tokenizer files not found"):
        TextTokenizer.from_pretrained(str(tmp_path))
