"""Frame-loop semantics of the oracle's rollout, with the model replaced by a script, checked
against the reference's rules (src/generation.rs:657-749, 876-963):

* EOS is checked before a frame runs: the EOS frame emits no codes;
* the Talker decodes frame f at position P + f; the last frame has no Talker step;
* trailing text row f feeds the step after frame f, tts_pad once the rows run out;
* the repetition-penalty history is every semantic token emitted so far;
* capacity: P + max_frames <= max_cache_steps.
"""
import numpy as np
import pytest

from oracle.model import GenerateOptions, Oracle
from oracle.sampling import GREEDY

V, H, G = 3072, 4, 16
EOS = 2150


class ScriptedOracle(Oracle):
    def __init__(self, semantics, cap=64):
        self.semantics = list(semantics)
        self.codec_eos = EOS
        self.num_code_groups = G
        self.max_cache_steps = cap
        self.dtype = np.float64
        self.codec_emb = np.arange(V * H, dtype=np.float64).reshape(V, H) * 0.0
        self.calls = []
        self.hidden = np.zeros(H)

        class _T:
            def reset(self_inner):
                pass

        self.talker = _T()

    def _logits(self, i):
        l = np.zeros(V)
        l[self.semantics[i]] = 10.0
        return l

    def prefill(self, prefill):
        self.calls.append(("prefill", prefill.shape[0]))
        self.n = 0
        return self._logits(0)

    def decode(self, step, offset):
        self.n += 1
        self.calls.append(("decode", offset, step.copy()))
        return self._logits(self.n)

    def code_predictor(self, prefix, cfg=GREEDY, seed=0, frame=0, forced=None):
        tokens = np.full(G - 1, frame, dtype=np.int32)
        return tokens, np.zeros(H), np.zeros((G - 1, 2048)), np.ones(G - 1)


def _inputs(P=5, T=2):
    prefill = np.zeros((P, H))
    trailing = np.stack([np.full(H, 100.0 + i) for i in range(T)])
    pad = np.full(H, -7.0)
    return prefill, trailing, pad


def test_eos_frame_emits_no_codes():
    o = ScriptedOracle([11, 12, EOS, 13])
    tr = o.rollout(*_inputs(), GenerateOptions.greedy(10))
    assert tr.ended_by_eos
    assert tr.codes[:, 0].tolist() == [11, 12]
    assert tr.frames == 2


def test_positions_and_last_frame_without_talker_step():
    o = ScriptedOracle([1, 2, 3, 4, 5])
    P = 5
    tr = o.rollout(*_inputs(P), GenerateOptions.greedy(3))
    assert not tr.ended_by_eos and tr.frames == 3
    decodes = [c for c in o.calls if c[0] == "decode"]
    assert [c[1] for c in decodes] == [P + 0, P + 1]      # frame 2 (last) decodes nothing
    assert len(tr.talker_logits) == 3


def test_trailing_rows_then_tts_pad():
    o = ScriptedOracle([1, 2, 3, 4, 5, 6])
    o.rollout(*_inputs(T=2), GenerateOptions.greedy(5))
    steps = [c[2] for c in o.calls if c[0] == "decode"]
    # step input = codec_emb[sem] (zeros here) + acoustic sum (zeros) + trailing row
    assert [s[0] for s in steps] == [100.0, 101.0, -7.0, -7.0]


def test_codes_are_frame_major_semantic_first():
    o = ScriptedOracle([7, 8, 9])
    tr = o.rollout(*_inputs(), GenerateOptions.greedy(3))
    assert tr.codes.shape == (3, G)
    assert tr.codes[1].tolist() == [8] + [1] * (G - 1)


def test_repetition_history_is_all_emitted_semantics():
    """With penalty p the scripted winner is divided by p once per distinct token seen."""
    seen = []

    class Spy(ScriptedOracle):
        def talker_select(self, logits, history, penalty, cfg, u, per_occurrence=False):
            seen.append(None if history is None else list(history))
            return super().talker_select(logits, history, penalty, cfg, u, per_occurrence)

    o = Spy([3, 4, 3, 5])
    opts = GenerateOptions(max_frames=4, do_sample=False, repetition_penalty=1.2, subtalker_dosample=False)
    o.rollout(*_inputs(), opts)
    assert seen == [None, [3], [3, 4], [3, 4, 3]]


def test_capacity_check():
    o = ScriptedOracle([1] * 10, cap=10)
    with pytest.raises(ValueError, match="cache steps"):
        o.rollout(*_inputs(P=5), GenerateOptions.greedy(6))
    o.rollout(*_inputs(P=5), GenerateOptions.greedy(5))


def test_option_validation():
    with pytest.raises(ValueError):
        GenerateOptions(max_frames=0).validate()
    with pytest.raises(ValueError):
        GenerateOptions(repetition_penalty=0.0).validate()
    with pytest.raises(ValueError):
        GenerateOptions(top_p=0.0).validate()
    with pytest.raises(ValueError):
        GenerateOptions(subtalker_temperature=0.0).validate()


def test_hook_fixture_inputs_follow_the_reference_formula():
    """deterministic_hidden (qwen3_tts_reference.py:620-626): ((i % m) - c) / m, and the hook
    fixtures carry the reference's array names."""
    import os
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
    from make_golden import deterministic_hidden

    from parity import fixture_exists, load_fixture
    v = deterministic_hidden(40, 17.0, 15.0)
    assert v[0] == np.float32(-15 / 17) and v[15] == 0.0 and v[16] == np.float32(1 / 17) and v[17] == v[0]
    w = deterministic_hidden(30, 23.0, 11.0)
    assert w[11] == 0.0 and w[22] == np.float32(11 / 23) and w[23] == np.float32(-11 / 23)
    for spec in ("tiny", "0.6b"):
        if not fixture_exists(f"hooks_{spec}"):
            continue
        fx = load_fixture(f"hooks_{spec}")
        for name in ("prefill", "last_hidden", "logits", "first_semantic", "first_step_input",
                     "forward_next_logits", "next_semantic", "talker_hidden", "semantic_embed",
                     "acoustic_tokens", "embedding_sum"):
            assert name in fx, name
        H = fx["talker_hidden"].shape[0]
        np.testing.assert_array_equal(fx["talker_hidden"], deterministic_hidden(H, 17.0, 15.0))
        np.testing.assert_array_equal(fx["semantic_embed"], deterministic_hidden(H, 23.0, 11.0))
