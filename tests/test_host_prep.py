"""Host-side inputs: synthetic checkpoint writer/reader, bf16 rounding, prompt layout."""
import json
import os

import numpy as np
import pytest
import torch

from q3t import synth, textprep
from q3t.workloads import WORKLOADS


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 0.02,
                        # exact ties: halfway between two bf16 values, both parities
                        np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8)], dtype=np.float32)])
    ours = synth.f32_to_bf16_bits(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)
    np.testing.assert_array_equal(synth.bf16_bits_to_f32(ours),
                                  torch.from_numpy(x).to(torch.bfloat16).float().numpy())


def test_generation_is_deterministic_and_per_tensor():
    a = synth.generate_tensor(0, "talker.codec_head.weight", (8, 16), "mat")
    b = synth.generate_tensor(0, "talker.codec_head.weight", (8, 16), "mat")
    c = synth.generate_tensor(1, "talker.codec_head.weight", (8, 16), "mat")
    np.testing.assert_array_equal(a, b)
    assert not np.array_equal(a, c)
    g = synth.bf16_bits_to_f32(synth.generate_tensor(0, "x.norm.weight", (4096,), "gain"))
    assert abs(g.mean() - 1.0) < 0.01 and 0.01 < g.std() < 0.03
    m = synth.bf16_bits_to_f32(synth.generate_tensor(0, "x.w", (512, 512), "mat"))
    assert abs(m.std() - 0.02) < 0.001


def test_tiny_checksum_matches_fixture():
    meta = json.loads(str(np.load(os.path.join(os.path.dirname(__file__), "golden", "tiny_greedy.npz"))["meta"]))
    assert synth.SyntheticModel.build("tiny", 0).checksum() == meta["checksum"]


def test_safetensors_round_trip(tmp_path):
    m = synth.SyntheticModel.build("tiny", 0)
    m.write(str(tmp_path))
    back = synth.read_safetensors_bf16(str(tmp_path / "model.safetensors"))
    assert set(back) == set(m.tensors)
    for k in ("talker.codec_head.weight", "talker.model.layers.1.mlp.down_proj.weight"):
        np.testing.assert_array_equal(np.asarray(back[k]), m.tensors[k])
    cfg = json.load(open(tmp_path / "config.json"))
    tc = cfg["talker_config"]
    assert tc["codec_eos_token_id"] == 2150 and tc["code_predictor_config"]["num_hidden_layers"] == 2
    # the file is also readable by the safetensors package (header + offsets well formed)
    from safetensors import safe_open
    with safe_open(str(tmp_path / "model.safetensors"), framework="pt") as f:
        t = f.get_tensor("talker.codec_head.weight")
    np.testing.assert_array_equal(t.view(torch.int16).numpy().view(np.uint16), m.tensors["talker.codec_head.weight"])


def test_inventory_sizes_match_the_0_6b_stacks():
    """0.6B Talker stack 440,466,432 params; CP stack 78,654,720 (+ 2 x 1024 norms): 28 and 5
    layers of hidden 1024, 16 q / 8 kv heads of 128, intermediate 3072, with q/k norms."""
    inv = {n: int(np.prod(s)) for n, s, _ in synth.tensor_inventory(synth.SPECS["0.6b"])}
    talker = sum(v for k, v in inv.items() if k.startswith("talker.model.layers."))
    cp = sum(v for k, v in inv.items() if k.startswith("talker.code_predictor.model.layers."))
    assert talker == 440466432
    assert cp == 78654720


@pytest.fixture(scope="module")
def prep():
    return textprep.TextPrep(synth.SyntheticModel.build("tiny", 0))


def test_prefill_layout(prep):
    ids = [5, 6, 7, 8]
    inp = prep.prepare(ids)
    H = prep.spec.talker.hidden
    assert inp.prefill.shape == (9 + 4, H)
    t = prep.tokens
    role = prep.projected_text_embeddings([t["im_start_token_id"], t["assistant_token_id"], 198])
    np.testing.assert_allclose(inp.prefill[:3], role)
    pad = prep.projected_text_embeddings([t["tts_pad_token_id"]])[0]
    bos = prep.projected_text_embeddings([t["tts_bos_token_id"]])[0]
    emb = prep.codec_emb
    np.testing.assert_allclose(inp.prefill[3], pad + emb[t["codec_think_id"]], rtol=1e-6)
    np.testing.assert_allclose(inp.prefill[5], pad + emb[2050], rtol=1e-6)          # english
    np.testing.assert_allclose(inp.prefill[7], pad + emb[3061], rtol=1e-6)          # ryan
    np.testing.assert_allclose(inp.prefill[8], bos + emb[t["codec_pad_id"]], rtol=1e-6)
    txt = prep.projected_text_embeddings(ids)
    np.testing.assert_allclose(inp.prefill[9], txt[0] + emb[t["codec_pad_id"]], rtol=1e-6)
    np.testing.assert_allclose(inp.prefill[12], txt[3] + emb[t["codec_bos_id"]], rtol=1e-6)
    eos = prep.projected_text_embeddings([t["tts_eos_token_id"]])
    np.testing.assert_allclose(inp.trailing_text, eos)          # all text in the prefill
    np.testing.assert_allclose(inp.tts_pad_embed, pad)


def test_lookahead_splits_prompt(prep):
    ids = list(range(100, 110))
    inp = prep.prepare(ids, text_lookahead_tokens=3)
    assert inp.prefill_steps == 12 and inp.trailing_steps == 8   # 7 remaining + tts_eos
    np.testing.assert_allclose(inp.trailing_text[0], prep.projected_text_embeddings([103])[0])
    with pytest.raises(ValueError):
        prep.prepare(ids, text_lookahead_tokens=0)


def test_text_projection_is_silu_mlp(prep):
    row = synth.text_embedding_rows(0, [42], prep.spec.text_hidden).astype(np.float64)
    h = row @ prep.fc1_w.T + prep.fc1_b
    want = (h * (1 / (1 + np.exp(-h)))) @ prep.fc2_w.T + prep.fc2_b
    np.testing.assert_allclose(prep.projected_text_embeddings([42]), want.astype(np.float32), rtol=1e-6)


def test_workload_capacities_fit():
    m = synth.SyntheticModel.build("tiny", 0)
    for w in WORKLOADS.values():
        P = 9 + (w.prompt_tokens if w.lookahead is None else min(w.lookahead, w.prompt_tokens))
        assert P + w.frames <= w.max_cache_steps, w.name
    w = WORKLOADS["tiny_greedy"]
    assert w.inputs(m).prefill_steps == 9 + w.prompt_tokens
