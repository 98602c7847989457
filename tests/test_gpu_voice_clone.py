"""Voice clone with an x-vector prompt on the device (q3t_prepare_text_voice_clone /
q3t_stream_start_voice_clone) against the CPU oracle of text.rs:432-514 (the custom-voice
layout with the speaker's codec row replaced by the prompt's speaker embedding) and the
token-loop oracle, on the tiny model written with its text-embedding table."""
import numpy as np
import pytest

from oracle.model import GenerateOptions as OracleOptions
from oracle.model import Oracle
from oracle.textprep import TextPrepOracle
from q3t import engine as E
from q3t import synth, textprep
from q3t.voice_clone import VoiceClonePrompt, VoiceClonePromptError

from parity import check_codes

pytestmark = pytest.mark.gpu

TOL = 2e-5  # as the custom-voice preparation: fp32 projection vs the float64 oracle


@pytest.fixture(scope="module")
def tiny_text(models):
    model, d = models.get_with_text("tiny")
    rows = lambda ids: synth.text_embedding_rows(model.seed, ids, model.spec.text_hidden)
    oracle = TextPrepOracle(model.tensors, model.config(), rows, synth.TEXT_VOCAB)
    eng = E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=256))
    yield model, oracle, eng
    eng.close()


def _prompt(model, seed, scale=0.05):
    emb = np.random.default_rng(seed).standard_normal(model.spec.talker.hidden) * scale
    return VoiceClonePrompt(emb.astype(np.float32), x_vector_only_mode=True)


@pytest.mark.parametrize("n,look,language", [(40, 1 << 30, "english"), (40, 8, "german"), (3, 1, "korean"),
                                             (150, 20, "chinese"), (0, 2, "english")])
def test_prepare_matches_oracle(tiny_text, n, look, language):
    model, oracle, eng = tiny_text
    ids = textprep.random_prompt(n, 31 + n)
    prompt = _prompt(model, n)
    print(f"[gpu] prepare_voice_clone_text n={n} lookahead={look} {language}", flush=True)
    got = eng.prepare_voice_clone_text(ids, prompt, language, look)
    ref = oracle.prepare(ids, prompt.speaker_embedding.astype(np.float64), language, look)
    assert got.prefill.shape == ref.prefill.shape and got.trailing_text.shape == ref.trailing_text.shape
    err = max(float(np.abs(got.prefill - ref.prefill).max()),
              float(np.abs(got.trailing_text - ref.trailing_text).max()),
              float(np.abs(got.tts_pad_embed - ref.tts_pad_embed).max()))
    print(f"voice clone prepare n={n}: max err {err:.2e}")
    assert err <= TOL
    # the custom-voice rows differ from these in the speaker row only (prefill row 7)
    cv = eng.prepare_text(ids, "ryan", language, look)
    d = np.abs(cv.prefill - got.prefill).max(axis=1)
    assert d[7] > 1e-3 and np.all(np.delete(d, 7) == 0)


def test_stream_matches_oracle(tiny_text, tmp_path):
    model, oracle, eng = tiny_text
    ids = textprep.random_prompt(28, 5)
    _prompt(model, 77, scale=0.5).to_json(tmp_path / "prompt.json")
    prompt = VoiceClonePrompt.from_json(tmp_path / "prompt.json")
    opts = E.GenerateOptions.greedy(16)
    print("[gpu] voice clone stream n=28 lookahead=5", flush=True)
    with eng.start_voice_clone_stream(ids, prompt, opts, E.StreamOptions(text_lookahead_tokens=5)) as st:
        assert st.prefill_steps == 14
        chunks = []
        while (c := st.next_codes_chunk(6)) is not None:
            chunks.append(c.codes)
        eos = st.ended_by_eos
    codes = np.concatenate(chunks)
    ref_in = oracle.prepare(ids, prompt.speaker_embedding.astype(np.float64), "english", 5)
    o = Oracle(model.tensors, model.config(), max_cache_steps=256)
    oo = OracleOptions(**{k: getattr(opts, k) for k in OracleOptions.__dataclass_fields__})
    tr = o.rollout(ref_in.prefill, ref_in.trailing_text, ref_in.tts_pad_embed, oo)
    fx = dict(codes=tr.codes, talker_logits=tr.talker_logits, talker_margins=tr.talker_margins,
              cp_margins=tr.cp_margins, meta=dict(ended_by_eos=tr.ended_by_eos))
    same = check_codes(codes, eos, fx)
    print(f"voice clone stream: {same} frames identical")


def test_generate_codes_matches_host_prepared(tiny_text):
    """generate_voice_clone_codes (generation.rs:373-393) = the rows it prepares, started
    through q3t_stream_start with every content id in the prefill."""
    model, oracle, eng = tiny_text
    ids = textprep.random_prompt(20, 9)
    prompt = _prompt(model, 3, scale=0.5)
    opts = E.GenerateOptions.greedy(12)
    print("[gpu] generate_voice_clone_codes n=20", flush=True)
    a = eng.generate_voice_clone_codes(ids, prompt, opts)
    b = eng.start_stream(eng.prepare_voice_clone_text(ids, prompt), opts)
    cb = b.next_codes_chunk(12)
    b.close()
    np.testing.assert_array_equal(a.codes, cb.codes)
    assert a.frames == cb.frames


def test_voice_clone_errors(tiny_text):
    model, oracle, eng = tiny_text
    H = model.spec.talker.hidden
    ok = VoiceClonePrompt(np.zeros(H, np.float32), x_vector_only_mode=True)
    with pytest.raises(E.InvalidInputError, match="speaker embedding length"):
        eng.prepare_voice_clone_text([1, 2], VoiceClonePrompt(np.zeros(H - 1, np.float32), x_vector_only_mode=True))
    with pytest.raises(VoiceClonePromptError, match="only x-vector-only"):
        eng.prepare_voice_clone_text([1, 2], VoiceClonePrompt(np.zeros(H, np.float32), x_vector_only_mode=False))
    with pytest.raises(E.InvalidInputError, match="text_lookahead_tokens"):
        eng.prepare_voice_clone_text([1, 2], ok, text_lookahead_tokens=0)
    with pytest.raises(E.InvalidInputError):
        eng.prepare_voice_clone_text([synth.TEXT_VOCAB], ok)
    with pytest.raises(E.CapacityError):
        eng.start_voice_clone_stream(list(range(300)), ok, E.GenerateOptions.greedy(8),
                                     E.StreamOptions(text_lookahead_tokens=1 << 30))
    # the slot is free again after the failed start
    with eng.start_voice_clone_stream([1, 2, 3], ok, E.GenerateOptions.greedy(2)) as st:
        assert st.next_codes_chunk(2) is not None
