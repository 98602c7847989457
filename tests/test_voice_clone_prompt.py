"""VoiceClonePrompt::from_json (src/model/voice_clone.rs:30-45) and the prompt-kind check of
prepare_voice_clone_xvector_with_lookahead (src/model/text.rs:439-443), on the CPU."""
import json

import numpy as np
import pytest

from q3t.voice_clone import VoiceClonePrompt, VoiceClonePromptError


def _write(tmp_path, doc, name="prompt.json"):
    p = tmp_path / name
    p.write_text(doc if isinstance(doc, str) else json.dumps(doc))
    return p


def test_defaults_and_fields(tmp_path):
    p = VoiceClonePrompt.from_json(_write(tmp_path, {"speaker_embedding": [0.5, -1, 2.25]}))
    np.testing.assert_array_equal(p.speaker_embedding, np.array([0.5, -1.0, 2.25], np.float32))
    assert p.speaker_embedding.dtype == np.float32
    assert (p.x_vector_only_mode, p.icl_mode, p.ref_text, p.ref_codes) == (False, False, None, None)
    q = VoiceClonePrompt.from_json(_write(tmp_path, {
        "speaker_embedding": [1.0], "x_vector_only_mode": True, "icl_mode": False, "ref_text": "hi",
        "ref_codes": [1, -2], "unknown_field": 3}))
    assert (q.x_vector_only_mode, q.icl_mode, q.ref_text, q.ref_codes) == (True, False, "hi", [1, -2])
    r = VoiceClonePrompt.from_json(_write(tmp_path, {"speaker_embedding": [], "ref_text": None,
                                                     "ref_codes": None}))
    assert r.speaker_embedding.size == 0 and r.ref_text is None and r.ref_codes is None


def test_round_trip(tmp_path):
    emb = np.random.default_rng(0).standard_normal(64).astype(np.float32)
    p = VoiceClonePrompt(emb, x_vector_only_mode=True)
    p.to_json(tmp_path / "p.json")
    q = VoiceClonePrompt.from_json(tmp_path / "p.json")
    np.testing.assert_array_equal(q.speaker_embedding, emb)
    assert q.x_vector_only_mode and not q.icl_mode


@pytest.mark.parametrize("doc,match", [
    ("{", "failed to parse"),
    ("[1, 2]", "failed to parse"),
    ({"x_vector_only_mode": True}, "failed to parse"),
    ({"speaker_embedding": "abc"}, "failed to parse"),
    ({"speaker_embedding": [1, "a"]}, "failed to parse"),
    ({"speaker_embedding": [1.0], "icl_mode": 1}, "failed to parse"),
    ({"speaker_embedding": [1.0], "ref_codes": [2 ** 31]}, "failed to parse"),
    ({"speaker_embedding": [1.0], "ref_text": 5}, "failed to parse"),
])
def test_parse_errors(tmp_path, doc, match):
    with pytest.raises(VoiceClonePromptError, match=match):
        VoiceClonePrompt.from_json(_write(tmp_path, doc))


def test_read_error(tmp_path):
    with pytest.raises(VoiceClonePromptError, match="failed to read"):
        VoiceClonePrompt.from_json(tmp_path / "missing.json")


@pytest.mark.parametrize("xonly,icl,codes,ok", [
    (True, False, None, True), (False, False, None, False), (True, True, None, False),
    (True, False, [1, 2], False)])
def test_x_vector_only_check(xonly, icl, codes, ok):
    p = VoiceClonePrompt(np.zeros(4, np.float32), x_vector_only_mode=xonly, icl_mode=icl, ref_codes=codes)
    if ok:
        p.check_x_vector_only()
    else:
        with pytest.raises(VoiceClonePromptError, match="only x-vector-only voice clone prompts"):
            p.check_x_vector_only()
