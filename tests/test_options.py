"""Speaker / Language names as the reference parses them (Speaker::from_str, Language::from_str,
src/model/text.rs:75-93, 137-153) and their q3t_generate_options ordinals (the enums' order,
text.rs:28-40, 95-106)."""
import pytest

from q3t import engine as E


@pytest.mark.parametrize("name,idx", [("Ryan", 3), ("ryan", 3), ("RYAN", 3), ("serena", 0), ("Vivian", 1),
                                      ("uncle_fu", 2), ("UncleFu", 2), ("aiden", 4), ("Ono_Anna", 5),
                                      ("onoanna", 5), ("sohee", 6), ("eric", 7), ("Dylan", 8)])
def test_speakers(name, idx):
    assert E.parse_speaker(name) == idx
    assert E.GenerateOptions(speaker=name)._c().speaker == idx


@pytest.mark.parametrize("name,idx", [("English", 1), ("en", 1), ("EN", 1), ("chinese", 0), ("zh", 0),
                                      ("Japanese", 2), ("ja", 2), ("korean", 3), ("ko", 3), ("German", 4),
                                      ("de", 4), ("french", 5), ("fr", 5), ("russian", 6), ("ru", 6),
                                      ("Portuguese", 7), ("pt", 7), ("spanish", 8), ("es", 8), ("italian", 9),
                                      ("it", 9)])
def test_languages(name, idx):
    assert E.parse_language(name) == idx
    assert E.GenerateOptions(language=name)._c().language == idx


def test_unknown_names():
    with pytest.raises(E.InvalidInputError, match="unknown speaker Bob"):
        E.parse_speaker("Bob")
    with pytest.raises(E.InvalidInputError, match="unknown language klingon"):
        E.parse_language("klingon")
    with pytest.raises(E.InvalidInputError, match="unknown speaker uncle fu"):
        E.GenerateOptions(speaker="uncle fu")._c()


def test_option_defaults_match_the_reference():
    """GenerateOptions / StreamOptions defaults (generation.rs:40-92)."""
    o = E.GenerateOptions()
    assert (o.speaker.lower(), o.language.lower(), o.max_frames, o.decode_audio, o.do_sample, o.top_k, o.top_p,
            o.temperature, o.repetition_penalty, o.subtalker_dosample, o.subtalker_top_k, o.subtalker_top_p,
            o.subtalker_temperature, o.seed) == ("ryan", "english", 240, True, True, 50, 1.0, 0.9, 1.05, True, 50,
                                                 1.0, 0.9, 0)
    assert o.repetition_penalty_per_occurrence is False and o._c().repetition_penalty_per_occurrence == 0
    s = E.StreamOptions()
    assert (s.text_lookahead_tokens, s.left_context_frames) == (8, 25)
    assert (E.DEFAULT_MAX_CACHE_STEPS, E.DEFAULT_PREFILL_HEADROOM, E.SAMPLE_RATE) == (512, 256, 24000)
