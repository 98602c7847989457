"""The prompt-preparation oracle (oracle/textprep.py), pinned without the reference's code:

* the text projection against torch's Linear + SiLU in float64 on the same weights (a
  transposed weight, a dropped bias or a wrong activation fails it);
* the prefill layout of text.rs:516-573 row by row, built here from the projection and the
  codec table directly (role rows alone, think / language / speaker rows, pad over every
  content row but the last, bos on the last);
* the lookahead split of text.rs:340-382, the empty-content case and the range errors;
* agreement with the package's host preparation (q3t/textprep.py), written separately.
"""
import numpy as np
import pytest
import torch

from oracle.textprep import NEWLINE, TextPrepOracle
from q3t import synth, textprep


@pytest.fixture(scope="module")
def tiny():
    model = synth.SyntheticModel.build("tiny", 0)
    rows = lambda ids: synth.text_embedding_rows(model.seed, ids, model.spec.text_hidden)
    return model, TextPrepOracle(model.tensors, model.config(), rows, synth.TEXT_VOCAB)


def test_projection_is_torch_linear_silu_linear(tiny):
    model, o = tiny
    ids = np.array([0, 17, 151643, 151671, synth.TEXT_VOCAB - 1])
    x = torch.from_numpy(synth.text_embedding_rows(0, ids, model.spec.text_hidden).astype(np.float64))
    f = lambda n: torch.from_numpy(model.f32(n).astype(np.float64))
    h = torch.nn.functional.silu(torch.nn.functional.linear(
        x, f("talker.text_projection.linear_fc1.weight"), f("talker.text_projection.linear_fc1.bias")))
    y = torch.nn.functional.linear(h, f("talker.text_projection.linear_fc2.weight"),
                                   f("talker.text_projection.linear_fc2.bias"))
    np.testing.assert_allclose(o.projected(ids), y.numpy(), rtol=1e-12, atol=1e-14)


def test_prefill_layout_row_by_row(tiny):
    model, o = tiny
    cfg = model.config()
    t, tc = synth.TOKENS, cfg["talker_config"]
    content = [5, 99, 1234, 151000]
    got = o.prepare(content, "vivian", "german", text_lookahead_tokens=3)
    codec = model.f32("talker.model.codec_embedding.weight").astype(np.float64)
    proj = o.projected
    expect = [proj([t["im_start_token_id"]])[0], proj([t["assistant_token_id"]])[0], proj([NEWLINE])[0]]
    codec6 = [t["codec_think_id"], t["codec_think_bos_id"], tc["codec_language_id"]["german"],
              t["codec_think_eos_id"], tc["spk_id"]["vivian"], t["codec_pad_id"]]
    for i in range(6):
        tok = t["tts_bos_token_id"] if i == 5 else t["tts_pad_token_id"]
        expect.append(proj([tok])[0] + codec[codec6[i]])
    for i in range(3):
        expect.append(proj([content[i]])[0] + codec[t["codec_bos_id"] if i == 2 else t["codec_pad_id"]])
    # batched and one-row products differ only in float64 summation order
    close = lambda a, b: np.testing.assert_allclose(a, b, rtol=0, atol=1e-14)
    close(got.prefill, np.vstack(expect))
    close(got.trailing_text, proj([content[3], t["tts_eos_token_id"]]))
    close(got.tts_pad_embed, proj([t["tts_pad_token_id"]])[0])


def test_lookahead_and_empty_content(tiny):
    _, o = tiny
    content = list(range(10, 30))
    for look, p, tr in [(1, 10, 20), (8, 17, 13), (20, 29, 1), (1 << 30, 29, 1)]:
        got = o.prepare(content, text_lookahead_tokens=look)
        assert got.prefill.shape[0] == p and got.trailing_text.shape[0] == tr
    empty = o.prepare([], text_lookahead_tokens=5)
    assert empty.prefill.shape[0] == 9 and empty.trailing_text.shape[0] == 1
    with pytest.raises(ValueError):
        o.prepare(content, text_lookahead_tokens=0)
    with pytest.raises(ValueError):
        o.prepare([synth.TEXT_VOCAB])
    with pytest.raises(ValueError):
        o.prepare(content, speaker="nobody")


def test_agrees_with_host_preparation(tiny):
    model, o = tiny
    content = textprep.random_prompt(40, 3)
    host = textprep.TextPrep(model).prepare(content, "ryan", "english", text_lookahead_tokens=8)
    ref = o.prepare(content, "ryan", "english", text_lookahead_tokens=8)
    np.testing.assert_allclose(host.prefill, ref.prefill, rtol=0, atol=1e-6)
    np.testing.assert_allclose(host.trailing_text, ref.trailing_text, rtol=0, atol=1e-6)
    np.testing.assert_allclose(host.tts_pad_embed, ref.tts_pad_embed, rtol=0, atol=1e-6)


def test_voice_clone_replaces_the_speaker_row(tiny):
    """prepare_voice_clone_xvector_with_lookahead (text.rs:432-490): the custom-voice layout with
    the speaker's codec row (prefill row 7) replaced by the prompt's x-vector."""
    model, o = tiny
    content = [5, 99, 1234]
    H = model.spec.talker.hidden
    xvec = np.random.default_rng(4).standard_normal(H) * 0.05
    vc = o.prepare(content, xvec, "english", text_lookahead_tokens=8)
    cv = o.prepare(content, "ryan", "english", text_lookahead_tokens=8)
    spk = model.config()["talker_config"]["spk_id"]["ryan"]
    codec = model.f32("talker.model.codec_embedding.weight").astype(np.float64)
    diff = vc.prefill - cv.prefill
    np.testing.assert_allclose(diff[7], xvec - codec[spk], rtol=0, atol=1e-14)
    np.testing.assert_array_equal(np.delete(diff, 7, axis=0), 0)
    np.testing.assert_array_equal(vc.trailing_text, cv.trailing_text)
    with pytest.raises(ValueError, match="speaker embedding length"):
        o.prepare(content, xvec[:-1], "english")
