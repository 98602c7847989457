"""The C-ABI library without a GPU: it loads, exports every symbol include/q3t.h declares,
and its host-side validation mirrors the reference (src/generation.rs:569-617,
src/model/sampling.rs:11-26).  No kernel is launched here."""
import ctypes
import json
import os
import re
import subprocess

import pytest

from q3t import engine as E

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "q3t.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(q3t_[a-z_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = E.load_library()
    names = declared_symbols()
    assert len(names) >= 12
    out = subprocess.run(["nm", "-D", "--defined-only", E.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (q3t_\w+)", out))
    for n in names:
        assert n in exported, n
        assert getattr(lib, n) is not None


def test_library_carries_gfx950_code_object():
    """The fat binary embedded in our own build names the gfx950 target."""
    data = open(E.LIB_PATH, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in data


def test_default_options_match_reference():
    E.load_library()
    o = E._GenerateOptions()
    E._lib.q3t_generate_options_default(ctypes.byref(o))
    ref = E.GenerateOptions()
    assert o.max_frames == ref.max_frames == 240
    assert o.do_sample == 1 and o.top_k == 50 and o.top_p == 1.0
    assert abs(o.temperature - 0.9) < 1e-7 and abs(o.repetition_penalty - 1.05) < 1e-7
    assert o.subtalker_dosample == 1 and o.subtalker_top_k == 50 and abs(o.subtalker_temperature - 0.9) < 1e-7
    assert o.seed == 0 and o.decode_audio == 1


@pytest.mark.parametrize("field,value,msg", [
    ("max_frames", 0, "max_frames must be non-zero"),
    ("repetition_penalty", 0.0, "repetition_penalty must be positive"),
    ("repetition_penalty", -1.0, "repetition_penalty must be positive"),
    ("top_p", 0.0, "talker.top_p"),
    ("top_p", 1.5, "talker.top_p"),
    ("temperature", 0.0, "talker.temperature"),
    ("subtalker_top_p", 0.0, "subtalker.top_p"),
    ("subtalker_temperature", -0.1, "subtalker.temperature"),
    ("top_k", -1, "talker.top_k"),
])
def test_option_validation(field, value, msg):
    opts = E.GenerateOptions(**{field: value})
    with pytest.raises(E.InvalidInputError, match=msg):
        opts.validate()


def test_valid_options_pass():
    E.GenerateOptions().validate()
    E.GenerateOptions.greedy(12).validate()
    E.GenerateOptions(top_p=0.5, top_k=0, temperature=1e-3).validate()


def test_stream_options_validation():
    with pytest.raises(E.InvalidInputError):
        E.StreamOptions(text_lookahead_tokens=0).validate()


def test_missing_model_dir_is_not_found(tmp_path):
    with pytest.raises(E.NotFoundError, match="config.json"):
        E.HipTtsEngine(str(tmp_path / "nope"))


def _config_dir(tmp_path, **talker_overrides):
    from q3t import synth
    cfg = synth.SPECS["tiny"].config_json()
    cfg["talker_config"].update(talker_overrides)
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    return str(tmp_path)


def test_unsupported_shapes_rejected_before_any_gpu_call(tmp_path):
    with pytest.raises(E.InvalidInputError, match="head_dim"):
        E.HipTtsEngine(_config_dir(tmp_path, head_dim=64))
    with pytest.raises(E.InvalidInputError, match="q_heads"):
        E.HipTtsEngine(_config_dir(tmp_path, head_dim=128, num_attention_heads=6, num_key_value_heads=2))


def test_missing_weights_file(tmp_path):
    with pytest.raises(E.NotFoundError, match="model.safetensors"):
        E.HipTtsEngine(_config_dir(tmp_path))


def test_cache_limit_rejected(tmp_path):
    with pytest.raises(E.InvalidInputError, match="max_cache_steps"):
        E.HipTtsEngine(_config_dir(tmp_path), E.EngineOptions(max_cache_steps=1 << 20))


def test_null_arguments():
    lib = E.load_library()
    assert lib.q3t_engine_create(None, None) == E.Q3T_ERR_INVALID
    assert lib.q3t_stream_next_codes(None, 6, None, None) == E.Q3T_ERR_INVALID
    assert lib.q3t_generate_options_validate(None) == E.Q3T_ERR_INVALID
    assert lib.q3t_engine_destroy(None) == E.Q3T_OK
    assert lib.q3t_stream_destroy(None) == E.Q3T_OK


def _weights_file(tmp_path, header, data=b"\0" * 64, hlen=None):
    import struct
    h = json.dumps(header).encode()
    (tmp_path / "model.safetensors").write_bytes(struct.pack("<Q", len(h) if hlen is None else hlen) + h + data)


@pytest.mark.parametrize("header,hlen,match", [
    ({"a": {"dtype": "BF16", "shape": [4], "data_offsets": [-8, 0]}}, None, "data offsets"),
    ({"a": {"dtype": "BF16", "shape": [4], "data_offsets": [8, 0]}}, None, "data offsets"),
    ({"a": {"dtype": "BF16", "shape": [40], "data_offsets": [0, 80]}}, None, "data offsets"),
    ({"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 8]}}, None, "data offsets"),
    ({"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16.5]}}, None, "integer"),
    ({"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 1e30]}}, None, "integer"),
    ({"a": {"dtype": "F32", "shape": [-4], "data_offsets": [0, 16]}}, None, "shape"),
    ({"a": {"dtype": "F32", "shape": [4], "data_offsets": [0]}}, None, "data_offsets"),
    ({"a": {"dtype": "Q4", "shape": [4], "data_offsets": [0, 16]}}, None, "dtype"),
    ({}, (1 << 64) - 1, "header length"),
    ({}, 1 << 20, "header length"),
])
def test_malformed_weights_header_rejected_before_any_gpu_call(tmp_path, header, hlen, match):
    """Every tensor entry of model.safetensors must describe a byte range inside the data
    section that holds exactly its shape; the whole header is checked when the file is
    opened, before any device call."""
    d = _config_dir(tmp_path)
    _weights_file(tmp_path, {"__metadata__": {"format": "pt"}, **header}, hlen=hlen)
    with pytest.raises(E.InvalidInputError, match=match):
        E.HipTtsEngine(d)


def _raw_weights_file(tmp_path, text: bytes):
    import struct
    (tmp_path / "model.safetensors").write_bytes(struct.pack("<Q", len(text)) + text + b"\0" * 64)


@pytest.mark.parametrize("text,match", [
    (b'{"a": ' + b"[" * 100000 + b"]" * 100000 + b"}", "nesting too deep"),
    (b'{"a": ' + b'{"b": ' * 65 + b"1" + b"}" * 65 + b"}", "nesting too deep"),
    (b'{"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16', "unexpected end|expected"),
    (b'{"a": {"dtype": "F32", "shape": [4], "data_off', "unterminated string"),
], ids=["arrays-100000-deep", "objects-66-deep", "truncated-number", "truncated-key"])
def test_deep_or_truncated_weights_header_rejected(tmp_path, text, match):
    """A safetensors header nested past the parser's depth limit, or cut off mid-value, is
    an InvalidInputError from q3t_engine_create (not a host stack overflow), before any
    device call."""
    d = _config_dir(tmp_path)
    _raw_weights_file(tmp_path, text)
    with pytest.raises(E.InvalidInputError, match=match):
        E.HipTtsEngine(d)


def test_header_nesting_at_the_limit_parses(tmp_path):
    """64 levels of nesting are accepted (the limit is not off by one): the file then fails
    later, on its missing tensors, not in the parser."""
    d = _config_dir(tmp_path)
    _raw_weights_file(tmp_path, b'{"__metadata__": ' + b"[" * 63 + b"]" * 63 + b"}")
    with pytest.raises(E.Q3tError) as ei:
        E.HipTtsEngine(d)
    assert "nesting" not in str(ei.value)


def test_deeply_nested_config_json_rejected(tmp_path):
    """config.json goes through the same parser: deep nesting is an InvalidInputError."""
    (tmp_path / "config.json").write_text('{"x": ' + "[" * 50000 + "]" * 50000 + "}")
    with pytest.raises(E.InvalidInputError, match="nesting too deep"):
        E.HipTtsEngine(str(tmp_path))
