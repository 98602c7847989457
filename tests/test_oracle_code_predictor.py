"""Pins the oracle's CodePredictor loop, projection and Talker step input independently.

The reference defines the token loop as two causal sequences evaluated by HF models
(python-reference/qwen3_tts_reference.py:339-483, 629-676; src/model/code_predictor.rs:366-471;
src/model/talker.rs:296-356; src/generation.rs:657-749):

* the Talker runs over ``prefill rows, step_input_0, step_input_1, ...`` at positions
  0, 1, 2, ...; frame f's logits come from row P - 1 + f through the final norm and
  ``codec_head``, where ``step_input_f = codec_emb[semantic_f] + sum_i cp_emb[i][a_{f,i}]
  + (trailing[f] if f < T else tts_pad)`` (qwen3_tts_reference.py:420-440, 462-476);
* per frame, the CodePredictor runs over ``project([hidden_f, codec_emb[semantic_f],
  cp_emb[0][a_0], ..., cp_emb[13][a_13]])`` at positions 0..15, and group g's logits are
  ``lm_head[g](h[g + 1])`` (HF ``generate`` over inputs_embeds; code_predictor.rs:366-471);
  ``project`` is ``small_to_mtp_projection`` (weight and bias) or the identity.

Here both sequences are built from those definitions with torch's Embedding / linear and
evaluated by transformers' Qwen3Model over the whole sequence in one pass (no KV cache,
no oracle code), and compared with a teacher-forced oracle rollout.  Planted mistakes in
the oracle (a CodePredictor position off by one, the embedding table of the wrong group,
a dropped projection bias, a dropped term of the step input, a Talker position off by one)
must each fail the same comparison.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import hf_ref
from oracle.model import GenerateOptions, Oracle
from q3t import synth, textprep

TOL = 1e-10         # float64 oracle vs float64 library forward (measured ~5e-15)
MUTANT_MIN = 1e-4   # every planted mistake moves some logit by more than this


def _inputs(model):
    # 6 content ids with lookahead 2: 5 trailing rows (4 ids + tts_eos), then tts_pad rows
    return textprep.TextPrep(model).prepare(textprep.random_prompt(6, 4), text_lookahead_tokens=2)


def reference_logits(model, inputs, codes):
    """Talker logits [F, V], CodePredictor logits [F, 15, Vc], normed Talker hidden [F, H] and
    step inputs [F - 1, H] of a teacher-forced rollout with the given codes, from the
    definitions above."""
    t, cfg = model.tensors, model.config()["talker_config"]
    cc = cfg["code_predictor_config"]
    n_ac = cfg["num_code_groups"] - 1
    talker = hf_ref.stack_from_config(t, cfg, "talker.model")
    cp = hf_ref.stack_from_config(t, cc, "talker.code_predictor.model")
    emb = lambda name: torch.nn.Embedding.from_pretrained(hf_ref.bf64(t[name]))
    codec_emb = emb("talker.model.codec_embedding.weight")
    cp_emb = [emb(f"talker.code_predictor.model.codec_embedding.{i}.weight") for i in range(n_ac)]
    lm_head = [hf_ref.bf64(t[f"talker.code_predictor.lm_head.{g}.weight"]) for g in range(n_ac)]
    codec_head = hf_ref.bf64(t["talker.codec_head.weight"])
    if model.spec.has_projection:
        pw = hf_ref.bf64(t["talker.code_predictor.small_to_mtp_projection.weight"])
        pb = hf_ref.bf64(t["talker.code_predictor.small_to_mtp_projection.bias"])
        project = lambda x: F.linear(x, pw, pb)
    else:
        project = lambda x: x
    c = torch.from_numpy(np.asarray(codes, dtype=np.int64))
    frames = len(codes)
    trailing = torch.from_numpy(inputs.trailing_text.astype(np.float64))
    pad = torch.from_numpy(inputs.tts_pad_embed.astype(np.float64))
    steps = []
    for f in range(frames - 1):
        hid = torch.cat([codec_emb(c[f, 0:1])] + [cp_emb[i](c[f, i + 1:i + 2]) for i in range(n_ac)])
        steps.append(hid.sum(0) + (trailing[f] if f < len(trailing) else pad))
    steps = torch.stack(steps) if steps else torch.zeros(0, pad.shape[0], dtype=torch.float64)
    P = inputs.prefill_steps
    seq = torch.cat([torch.from_numpy(inputs.prefill.astype(np.float64)), steps])
    h = torch.from_numpy(hf_ref.forward(talker, seq.numpy()))
    hidden = h[P - 1:P - 1 + frames]
    t_logits = hidden @ codec_head.T
    cp_logits = []
    for f in range(frames):
        rows = [hidden[f], codec_emb(c[f, 0])] + [cp_emb[g - 1](c[f, g]) for g in range(1, n_ac)]
        hc = torch.from_numpy(hf_ref.forward(cp, project(torch.stack(rows)).numpy()))
        cp_logits.append(torch.stack([lm_head[g] @ hc[g + 1] for g in range(n_ac)]))
    return t_logits.numpy(), torch.stack(cp_logits).numpy(), hidden.numpy(), steps.numpy()


def oracle_rollout(oracle, inputs, frames, forced=None):
    """Teacher-forced (or free) greedy rollout; also records every Talker decode's input and
    position."""
    seen = []
    decode = oracle.decode

    def record(step, offset):
        seen.append((np.array(step, copy=True), offset))
        return decode(step, offset)

    oracle.decode = record
    tr = oracle.rollout(inputs.prefill, inputs.trailing_text, inputs.tts_pad_embed,
                        GenerateOptions.greedy(frames), keep_cp_logits=frames, forced_codes=forced)
    oracle.decode = decode
    return tr, seen


def compare(model, inputs, tr, seen):
    """Largest deviation of a rollout trace from the library-built reference."""
    t_ref, cp_ref, hid_ref, steps_ref = reference_logits(model, inputs, tr.codes)
    P = inputs.prefill_steps
    err = dict(
        talker=float(np.abs(tr.talker_logits[:len(t_ref)] - t_ref).max()),
        cp=float(np.abs(np.asarray(tr.cp_logits) - cp_ref).max()),
        hidden=float(np.abs(tr.talker_hidden[:len(hid_ref)] - hid_ref).max()),
        step=max([float(np.abs(s - r).max()) for (s, _), r in zip(seen, steps_ref)], default=0.0),
    )
    err["offsets_ok"] = [off for _, off in seen] == [P + f for f in range(len(seen))]
    return err


FRAMES = 8


@pytest.fixture(scope="module", params=["tiny", "tiny-proj"])
def case(request):
    model = synth.SyntheticModel.build(request.param, 0)
    inputs = _inputs(model)
    assert inputs.trailing_steps < FRAMES - 1          # the rollout reaches the tts_pad rows
    oracle = Oracle(model.tensors, model.config(), max_cache_steps=64)
    tr, seen = oracle_rollout(oracle, inputs, FRAMES)
    assert tr.frames == FRAMES and len(seen) == FRAMES - 1
    return model, inputs, tr


def test_rollout_matches_library_forward(case):
    model, inputs, tr = case
    oracle = Oracle(model.tensors, model.config(), max_cache_steps=64)
    tr2, seen = oracle_rollout(oracle, inputs, FRAMES, forced=tr.codes)
    np.testing.assert_array_equal(tr2.codes, tr.codes)
    err = compare(model, inputs, tr2, seen)
    print(model.spec.name, err)
    assert err["offsets_ok"]
    assert err["talker"] <= TOL and err["cp"] <= TOL and err["hidden"] <= TOL
    assert err["step"] <= 1e-12


def test_code_predictor_hook_inputs_match_library_forward(case):
    """The reference's CodePredictor fixture inputs (deterministic_hidden(H, 17, 15) and
    (H, 23, 11), qwen3_tts_reference.py:620-676): greedy tokens and every group's logits."""
    model, _, _ = case
    oracle = Oracle(model.tensors, model.config(), max_cache_steps=64)
    H = model.spec.talker_hidden
    dh = lambda n, m, c: np.array([((i % int(m)) - c) / m for i in range(n)], dtype=np.float32)
    prefix = np.stack([dh(H, 17.0, 15.0), dh(H, 23.0, 11.0)]).astype(np.float64)
    tokens, emb_sum, logits, _ = oracle.code_predictor(prefix)
    assert np.array_equal(tokens, logits.argmax(1))
    # library sequence: prefix then cp_emb[g - 1][token g - 1], projected
    t = model.tensors
    cc = model.config()["talker_config"]["code_predictor_config"]
    cp = hf_ref.stack_from_config(t, cc, "talker.code_predictor.model")
    rows = [torch.from_numpy(prefix[0]), torch.from_numpy(prefix[1])]
    rows += [hf_ref.bf64(t[f"talker.code_predictor.model.codec_embedding.{g - 1}.weight"])[int(tokens[g - 1])]
             for g in range(1, 15)]
    x = torch.stack(rows)
    if model.spec.has_projection:
        x = F.linear(x, hf_ref.bf64(t["talker.code_predictor.small_to_mtp_projection.weight"]),
                     hf_ref.bf64(t["talker.code_predictor.small_to_mtp_projection.bias"]))
    hc = hf_ref.forward(cp, x.numpy())
    ref = np.stack([synth.bf16_bits_to_f32(t[f"talker.code_predictor.lm_head.{g}.weight"]).astype(np.float64)
                    @ hc[g + 1] for g in range(15)])
    assert float(np.abs(logits - ref).max()) <= TOL
    ref_sum = sum(hf_ref.bf64(t[f"talker.code_predictor.model.codec_embedding.{g}.weight"])[int(tokens[g])]
                  for g in range(15)).numpy()
    np.testing.assert_allclose(emb_sum, ref_sum, rtol=0, atol=1e-12)


def test_project_is_linear_with_bias():
    model = synth.SyntheticModel.build("tiny-proj", 0)
    oracle = Oracle(model.tensors, model.config(), max_cache_steps=16)
    x = np.random.default_rng(0).standard_normal((3, model.spec.talker_hidden))
    t = model.tensors
    ref = F.linear(torch.from_numpy(x), hf_ref.bf64(t["talker.code_predictor.small_to_mtp_projection.weight"]),
                   hf_ref.bf64(t["talker.code_predictor.small_to_mtp_projection.bias"])).numpy()
    np.testing.assert_allclose(oracle.project(x), ref, rtol=0, atol=1e-12)
    tiny = synth.SyntheticModel.build("tiny", 0)          # equal widths: the identity
    y = np.random.default_rng(1).standard_normal((2, tiny.spec.talker_hidden))
    np.testing.assert_array_equal(Oracle(tiny.tensors, tiny.config(), max_cache_steps=16).project(y), y)


# -- planted mistakes (in the oracle, on the CPU): each must fail the comparison ---------------

def _cp_position_g(o):
    step = o.cp.decode_step
    o.cp.decode_step = lambda x, offset: step(x, offset - 1)      # group g at position g


def _cp_table_of_next_group(o):
    o.cp_emb = o.cp_emb[1:] + o.cp_emb[:1]       # group g's input from cp_emb[g] instead of [g - 1]


def _projection_without_bias(o):
    if o.proj_b is None:
        pytest.skip("no projection in this shape")
    o.proj_b = np.zeros_like(o.proj_b)


def _step_input_without_acoustic_sum(o):
    o.build_step_input = lambda semantic, acoustic_sum, row: o.codec_emb[semantic] + row


def _step_input_without_semantic(o):
    o.build_step_input = lambda semantic, acoustic_sum, row: acoustic_sum + row


def _talker_position_plus_one(o):
    step = o.talker.decode_step
    o.talker.decode_step = lambda x, offset: step(x, offset + 1)


def _cp_prefix_swapped(o):
    prefix = o.prepare_code_predictor_prefix
    o.prepare_code_predictor_prefix = lambda semantic: prefix(semantic)[::-1].copy()


@pytest.mark.parametrize("mutate", [_cp_position_g, _cp_table_of_next_group, _projection_without_bias,
                                    _step_input_without_acoustic_sum, _step_input_without_semantic,
                                    _talker_position_plus_one, _cp_prefix_swapped])
def test_planted_mistakes_fail(case, mutate):
    model, inputs, tr = case
    oracle = Oracle(model.tensors, model.config(), max_cache_steps=64)
    mutate(oracle)
    tr2, seen = oracle_rollout(oracle, inputs, FRAMES, forced=tr.codes)
    err = compare(model, inputs, tr2, seen)
    worst = max(err["talker"], err["cp"], err["hidden"])
    assert worst > MUTANT_MIN, (mutate.__name__, err)
