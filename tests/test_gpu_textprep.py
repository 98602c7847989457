"""Device prompt preparation (q3t_prepare_text / q3t_stream_start_text) against the CPU
oracle of text.rs:340-382 / 516-603 (oracle/textprep.py), on the tiny model written with its
full text-embedding table.  Prompts of 4..150 content ids cover both GEMM paths of the text
projection (fewer and more than 128 rows)."""
import numpy as np
import pytest

from oracle.model import GenerateOptions as OracleOptions
from oracle.model import Oracle
from oracle.textprep import TextPrepOracle
from q3t import engine as E
from q3t import synth, textprep

from parity import check_codes, check_talker_logits

pytestmark = pytest.mark.gpu

TOL = 2e-5  # fp32 projection (exact bf16 x fp32 products) vs the float64 oracle; rows are ~0.05


@pytest.fixture(scope="module")
def tiny_text(models):
    model, d = models.get_with_text("tiny")
    rows = lambda ids: synth.text_embedding_rows(model.seed, ids, model.spec.text_hidden)
    oracle = TextPrepOracle(model.tensors, model.config(), rows, synth.TEXT_VOCAB)
    eng = E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=256))
    yield model, oracle, eng
    eng.close()


@pytest.mark.parametrize("n,look,speaker,language", [
    (40, 1 << 30, "ryan", "english"), (40, 8, "vivian", "german"), (4, 1, "ono_anna", "japanese"),
    (150, 20, "dylan", "chinese"), (0, 3, "ryan", "english")])
def test_prepare_text_matches_oracle(tiny_text, n, look, speaker, language):
    model, oracle, eng = tiny_text
    assert eng.has_device_text_prep
    ids = textprep.random_prompt(n, 11 + n)
    print(f"[gpu] prepare_text n={n} lookahead={look} {speaker}/{language}", flush=True)
    got = eng.prepare_text(ids, speaker, language, look)
    ref = oracle.prepare(ids, speaker, language, look)
    assert got.prefill.shape == ref.prefill.shape and got.trailing_text.shape == ref.trailing_text.shape
    err = max(float(np.abs(got.prefill - ref.prefill).max()),
              float(np.abs(got.trailing_text - ref.trailing_text).max()),
              float(np.abs(got.tts_pad_embed - ref.tts_pad_embed).max()))
    print(f"prepare_text n={n}: max err {err:.2e}")
    assert err <= TOL


@pytest.mark.parametrize("n,steps", [(32, 15), (0, 9)])
def test_stream_from_ids_matches_oracle(tiny_text, n, steps):
    """A stream started from content ids (lookahead 6), including empty content: the 9-row
    role prefix alone, then tts_eos as the only trailing text row."""
    model, oracle, eng = tiny_text
    ids = textprep.random_prompt(n, 1)
    opts = E.GenerateOptions.greedy(16)
    print(f"[gpu] stream from {n} content ids", flush=True)
    st = eng.start_stream_text(ids, opts, E.StreamOptions(text_lookahead_tokens=6))
    assert st.prefill_steps == steps
    chunks = []
    while (c := st.next_codes_chunk(5)) is not None:
        chunks.append(c.codes)
    eos = st.ended_by_eos
    st.close()
    codes = np.concatenate(chunks)
    ref_in = oracle.prepare(ids, "ryan", "english", 6)
    o = Oracle(model.tensors, model.config(), max_cache_steps=256)
    oo = OracleOptions(**{k: getattr(opts, k) for k in OracleOptions.__dataclass_fields__})
    tr = o.rollout(ref_in.prefill, ref_in.trailing_text, ref_in.tts_pad_embed, oo)
    fx = dict(codes=tr.codes, talker_logits=tr.talker_logits, talker_margins=tr.talker_margins,
              cp_margins=tr.cp_margins, meta=dict(ended_by_eos=tr.ended_by_eos))
    same = check_codes(codes, eos, fx)
    print(f"stream from content ids: {same} frames identical")


def test_device_and_host_prepared_streams_agree(tiny_text):
    model, oracle, eng = tiny_text
    ids = textprep.random_prompt(24, 2)
    opts = E.GenerateOptions.greedy(12)
    a = eng.start_stream_text(ids, opts, E.StreamOptions(text_lookahead_tokens=1 << 30))
    ca = a.next_codes_chunk(12).codes
    a.close()
    b = eng.start_stream(eng.prepare_text(ids), opts)
    cb = b.next_codes_chunk(12).codes
    b.close()
    np.testing.assert_array_equal(ca, cb)


def test_text_prep_errors(tiny_text, models):
    model, oracle, eng = tiny_text
    with pytest.raises(E.InvalidInputError):
        eng.prepare_text([1, 2, 3], text_lookahead_tokens=0)
    with pytest.raises(E.InvalidInputError):
        eng.prepare_text([synth.TEXT_VOCAB])
    with pytest.raises(E.InvalidInputError):
        eng.prepare_text([1, 2, 3], speaker="nobody")
    with pytest.raises(E.CapacityError):
        eng.start_stream_text(list(range(300)), E.GenerateOptions.greedy(8),
                              E.StreamOptions(text_lookahead_tokens=1 << 30))
    _, plain = models.get("tiny")
    with E.HipTtsEngine(plain, E.EngineOptions(max_cache_steps=64)) as e2:
        assert not e2.has_device_text_prep
        with pytest.raises(E.NotFoundError):
            e2.prepare_text([1, 2, 3])


def test_generate_codes_from_text(tiny_text, models):
    """Text in, codes out: the directory's tokenizer, the chat-template slice, device
    preparation with every content id in the prefill (generate_codes, generation.rs:356-371)."""
    model, oracle, eng = tiny_text
    assert eng.tokenizer is not None
    text = "hello world, hello world!"
    ids = eng.content_ids(text)
    assert ids[:2] == [9707, 1879]
    opts = E.GenerateOptions.greedy(10)
    a = eng.generate_codes(text, opts)
    b = eng.generate_codes(ids, opts)            # ids prepared on the device (no host TextPrep given)
    np.testing.assert_array_equal(a.codes, b.codes)
    ref_in = oracle.prepare(ids, "ryan", "english", 1 << 30)
    o = Oracle(model.tensors, model.config(), max_cache_steps=256)
    oo = OracleOptions(**{k: getattr(opts, k) for k in OracleOptions.__dataclass_fields__})
    tr = o.rollout(ref_in.prefill, ref_in.trailing_text, ref_in.tts_pad_embed, oo)
    fx = dict(codes=tr.codes, talker_logits=tr.talker_logits, talker_margins=tr.talker_margins,
              cp_margins=tr.cp_margins, meta=dict(ended_by_eos=tr.ended_by_eos))
    same = check_codes(a.codes, a.ended_by_eos, fx)
    print(f"generate_codes from text: {same} frames identical")
    with eng.start_stream(text, opts, E.StreamOptions(text_lookahead_tokens=2)) as st:
        assert st.prefill_steps == 11
        assert st.next_codes_chunk(4).frames == 4
