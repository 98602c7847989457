"""Synthetic Qwen3-TTS checkpoints: config.json + model.safetensors in the reference schema.

The reference loads a model directory holding ``config.json`` (schema: reference
src/model/config.rs:105-150) and ``model.safetensors`` whose tensors carry the names
listed in src/model/decode.rs:2097-2123, src/model/talker.rs:95-101 and
src/model/code_predictor.rs:175-233.  No real checkpoint is available offline, so
this module writes a random-init model of the same shape.

Value rules (fixed here so that every consumer sees the same bits):

* every matrix and embedding table: N(0, 0.02) drawn in float32, rounded to
  bfloat16 (round-to-nearest-even);
* RMSNorm gains: 1 + N(0, 0.02), rounded to bfloat16 (HF initialises them to 1;
  the small perturbation makes a dropped gain observable in parity tests);
* biases: N(0, 0.02), rounded to bfloat16.

Each tensor comes from its own Philox stream keyed by (seed, crc32(name)), so a
tensor's values do not depend on which other tensors exist.  The text-embedding
table (151,936 x 2048) is row-addressable instead: row r is keyed by
(seed, crc32(name), r + 1) and only the rows a prompt needs are ever generated.
"""
from __future__ import annotations

import dataclasses
import json
import os
import struct
import zlib
from typing import Dict, Iterator, List, Optional, Tuple

import numpy as np

TEXT_VOCAB = 151936
TEXT_HIDDEN = 2048

# Special ids.  codec_eos (2150), English (2050), Ryan (3061) and the newline id
# (198) are the values the reference hard-codes (tools/experiments/bin/hip-e2e-bench.rs:12,
# src/model/text.rs:46, :113, :15).  The remaining ids are synthetic choices that
# sit in the same ranges (codec specials inside [2048, 3072), text specials above
# the BPE vocabulary).
LANGUAGE_IDS = {
    "chinese": 2055, "english": 2050, "japanese": 2058, "korean": 2064,
    "german": 2053, "french": 2061, "russian": 2069, "portuguese": 2071,
    "spanish": 2054, "italian": 2070,
}
SPEAKER_IDS = {
    "serena": 3066, "vivian": 3065, "uncle_fu": 3010, "ryan": 3061, "aiden": 2861,
    "ono_anna": 2873, "sohee": 2864, "eric": 2875, "dylan": 2878,
}
TOKENS = dict(
    codec_pad_id=2148, codec_bos_id=2149, codec_eos_token_id=2150,
    codec_think_id=2154, codec_think_bos_id=2156, codec_think_eos_id=2157,
    tts_pad_token_id=151671, tts_bos_token_id=151672, tts_eos_token_id=151673,
    im_start_token_id=151644, assistant_token_id=77091,
)


@dataclasses.dataclass(frozen=True)
class StackShape:
    hidden: int
    intermediate: int
    layers: int
    q_heads: int
    kv_heads: int
    head_dim: int
    vocab: int
    rms_eps: float = 1e-6
    rope_theta: float = 1e6


@dataclasses.dataclass(frozen=True)
class ModelSpec:
    name: str
    talker: StackShape
    code_predictor: StackShape
    num_code_groups: int = 16
    text_hidden: int = TEXT_HIDDEN
    text_proj_intermediate: int = TEXT_HIDDEN

    @property
    def talker_hidden(self) -> int:
        return self.talker.hidden

    @property
    def has_projection(self) -> bool:
        return self.talker.hidden != self.code_predictor.hidden

    def config_json(self) -> dict:
        t, c = self.talker, self.code_predictor
        cp = dict(
            head_dim=c.head_dim, hidden_size=c.hidden, intermediate_size=c.intermediate,
            num_attention_heads=c.q_heads, num_code_groups=self.num_code_groups,
            num_hidden_layers=c.layers, num_key_value_heads=c.kv_heads,
            rms_norm_eps=c.rms_eps, rope_theta=c.rope_theta, vocab_size=c.vocab,
        )
        talker = dict(
            code_predictor_config=cp,
            codec_bos_id=TOKENS["codec_bos_id"], codec_eos_token_id=TOKENS["codec_eos_token_id"],
            codec_language_id=dict(LANGUAGE_IDS), codec_pad_id=TOKENS["codec_pad_id"],
            codec_think_id=TOKENS["codec_think_id"], codec_think_bos_id=TOKENS["codec_think_bos_id"],
            codec_think_eos_id=TOKENS["codec_think_eos_id"], spk_id=dict(SPEAKER_IDS),
            head_dim=t.head_dim, hidden_size=t.hidden, intermediate_size=t.intermediate,
            num_attention_heads=t.q_heads, num_code_groups=self.num_code_groups,
            num_hidden_layers=t.layers, num_key_value_heads=t.kv_heads,
            rms_norm_eps=t.rms_eps, rope_theta=t.rope_theta, vocab_size=t.vocab,
            text_hidden_size=self.text_hidden, text_vocab_size=TEXT_VOCAB,
        )
        return dict(
            assistant_token_id=TOKENS["assistant_token_id"], im_start_token_id=TOKENS["im_start_token_id"],
            tts_bos_token_id=TOKENS["tts_bos_token_id"], tts_eos_token_id=TOKENS["tts_eos_token_id"],
            tts_pad_token_id=TOKENS["tts_pad_token_id"], talker_config=talker,
            q3t_synthetic=dict(spec=self.name),
        )


def _cp_shape(hidden: int = 1024) -> StackShape:
    return StackShape(hidden=hidden, intermediate=3072, layers=5, q_heads=16, kv_heads=8,
                      head_dim=128, vocab=2048)


SPECS: Dict[str, ModelSpec] = {
    # BASELINE configs 1-3 and 5.
    "0.6b": ModelSpec("0.6b",
                      StackShape(1024, 3072, 28, 16, 8, 128, 3072),
                      _cp_shape()),
    # BASELINE config 4 (CodePredictor identical, plus the 2048 -> 1024 projection).
    "1.7b": ModelSpec("1.7b",
                      StackShape(2048, 6144, 28, 16, 8, 128, 3072),
                      _cp_shape()),
    # Small shapes for quick CPU/GPU parity runs.  head_dim stays 128 and the codec
    # vocabularies stay 3072/2048 so the special-token ranges are the real ones.
    "tiny": ModelSpec("tiny",
                      StackShape(512, 1024, 2, 4, 2, 128, 3072),
                      StackShape(512, 1024, 2, 4, 2, 128, 2048),
                      text_proj_intermediate=512),
    "tiny-proj": ModelSpec("tiny-proj",
                           StackShape(1024, 1536, 2, 8, 4, 128, 3072),
                           StackShape(512, 1024, 2, 4, 2, 128, 2048),
                           text_proj_intermediate=512),
    # One query head per KV head in both stacks, and a 512 -> 1024 projection into the
    # CodePredictor (the real models have two query heads per KV head).
    "tiny-g1": ModelSpec("tiny-g1",
                         StackShape(512, 1024, 2, 4, 4, 128, 3072),
                         StackShape(1024, 1024, 2, 8, 8, 128, 2048),
                         text_proj_intermediate=512),
}


# ----------------------------------------------------------------------------------------
# bf16 helpers
# ----------------------------------------------------------------------------------------

def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 (nearest, ties to even); returns uint16 bit patterns."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounded = u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))
    return (rounded >> np.uint32(16)).astype(np.uint16)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


# ----------------------------------------------------------------------------------------
# tensor inventory
# ----------------------------------------------------------------------------------------

def _stack_tensors(prefix: str, s: StackShape) -> List[Tuple[str, Tuple[int, ...], str]]:
    q_out, kv_out = s.q_heads * s.head_dim, s.kv_heads * s.head_dim
    out = []
    for i in range(s.layers):
        p = f"{prefix}.layers.{i}"
        out += [
            (f"{p}.input_layernorm.weight", (s.hidden,), "gain"),
            (f"{p}.post_attention_layernorm.weight", (s.hidden,), "gain"),
            (f"{p}.self_attn.q_proj.weight", (q_out, s.hidden), "mat"),
            (f"{p}.self_attn.k_proj.weight", (kv_out, s.hidden), "mat"),
            (f"{p}.self_attn.v_proj.weight", (kv_out, s.hidden), "mat"),
            (f"{p}.self_attn.o_proj.weight", (s.hidden, q_out), "mat"),
            (f"{p}.self_attn.q_norm.weight", (s.head_dim,), "gain"),
            (f"{p}.self_attn.k_norm.weight", (s.head_dim,), "gain"),
            (f"{p}.mlp.gate_proj.weight", (s.intermediate, s.hidden), "mat"),
            (f"{p}.mlp.up_proj.weight", (s.intermediate, s.hidden), "mat"),
            (f"{p}.mlp.down_proj.weight", (s.hidden, s.intermediate), "mat"),
        ]
    out.append((f"{prefix}.norm.weight", (s.hidden,), "gain"))
    return out


def tensor_inventory(spec: ModelSpec) -> List[Tuple[str, Tuple[int, ...], str]]:
    """(name, shape, kind) for every tensor the path reads, in file order."""
    t, c = spec.talker, spec.code_predictor
    inv = _stack_tensors("talker.model", t)
    inv += [
        ("talker.codec_head.weight", (t.vocab, t.hidden), "mat"),
        ("talker.model.codec_embedding.weight", (t.vocab, t.hidden), "mat"),
        ("talker.text_projection.linear_fc1.weight", (spec.text_proj_intermediate, spec.text_hidden), "mat"),
        ("talker.text_projection.linear_fc1.bias", (spec.text_proj_intermediate,), "bias"),
        ("talker.text_projection.linear_fc2.weight", (t.hidden, spec.text_proj_intermediate), "mat"),
        ("talker.text_projection.linear_fc2.bias", (t.hidden,), "bias"),
    ]
    inv += _stack_tensors("talker.code_predictor.model", c)
    for g in range(spec.num_code_groups - 1):
        inv.append((f"talker.code_predictor.lm_head.{g}.weight", (c.vocab, c.hidden), "mat"))
    for g in range(spec.num_code_groups - 1):
        inv.append((f"talker.code_predictor.model.codec_embedding.{g}.weight", (c.vocab, t.hidden), "mat"))
    if spec.has_projection:
        inv += [
            ("talker.code_predictor.small_to_mtp_projection.weight", (c.hidden, t.hidden), "mat"),
            ("talker.code_predictor.small_to_mtp_projection.bias", (c.hidden,), "bias"),
        ]
    return inv


TEXT_EMBEDDING_NAME = "talker.model.text_embedding.weight"


def _philox(seed: int, name: str, row: int = 0) -> np.random.Generator:
    key = ((seed & 0xFFFFFFFF) << 96) | (zlib.crc32(name.encode()) << 64) | (row & 0xFFFFFFFFFFFFFFFF)
    return np.random.Generator(np.random.Philox(key=key))


def generate_tensor(seed: int, name: str, shape: Tuple[int, ...], kind: str) -> np.ndarray:
    """bf16 bit patterns (uint16) of one synthetic tensor."""
    n = int(np.prod(shape))
    z = _philox(seed, name).standard_normal(n, dtype=np.float32)
    z *= np.float32(0.02)
    if kind == "gain":
        z += np.float32(1.0)
    return f32_to_bf16_bits(z).reshape(shape)


def text_embedding_rows(seed: int, rows: np.ndarray, text_hidden: int = TEXT_HIDDEN) -> np.ndarray:
    """float32 rows of the (never materialised) 151,936 x text_hidden text-embedding table."""
    rows = np.asarray(rows, dtype=np.int64).reshape(-1)
    out = np.empty((rows.size, text_hidden), dtype=np.float32)
    for i, r in enumerate(rows):
        if not 0 <= r < TEXT_VOCAB:
            raise ValueError(f"text token {r} is out of range for vocab {TEXT_VOCAB}")
        z = _philox(seed, TEXT_EMBEDDING_NAME, int(r) + 1).standard_normal(text_hidden, dtype=np.float32)
        out[i] = bf16_bits_to_f32(f32_to_bf16_bits(z * np.float32(0.02)))
    return out


def text_embedding_block(seed: int, r0: int, r1: int, text_hidden: int = TEXT_HIDDEN) -> np.ndarray:
    """bf16 bit patterns of table rows r0 .. r1-1 (the values text_embedding_rows returns)."""
    out = np.empty((r1 - r0, text_hidden), dtype=np.uint16)
    for r in range(r0, r1):
        z = _philox(seed, TEXT_EMBEDDING_NAME, r + 1).standard_normal(text_hidden, dtype=np.float32)
        out[r - r0] = f32_to_bf16_bits(z * np.float32(0.02))
    return out


class SyntheticModel:
    """All path tensors of one synthetic model, as bf16 bit patterns held in memory."""

    def __init__(self, spec: ModelSpec, seed: int = 0, tensors: Optional[Dict[str, np.ndarray]] = None):
        self.spec = spec
        self.seed = seed
        if tensors is None:
            inv = tensor_inventory(spec)
            # Each tensor has its own Philox stream, so generation order does not matter.
            from concurrent.futures import ThreadPoolExecutor
            workers = min(8, os.cpu_count() or 1)
            with ThreadPoolExecutor(workers) as pool:
                arrays = list(pool.map(lambda t: generate_tensor(seed, *t), inv))
            tensors = {name: arr for (name, _, _), arr in zip(inv, arrays)}
        self.tensors = tensors

    @classmethod
    def build(cls, spec_name: str, seed: int = 0) -> "SyntheticModel":
        return cls(SPECS[spec_name], seed)

    def f32(self, name: str) -> np.ndarray:
        return bf16_bits_to_f32(self.tensors[name])

    def config(self) -> dict:
        return self.spec.config_json()

    def checksum(self) -> str:
        h = 0
        for name, _, _ in tensor_inventory(self.spec):
            h = zlib.crc32(self.tensors[name].tobytes(), h)
        return f"{h:08x}"

    def write(self, model_dir: str, text_embedding: bool = False) -> None:
        """Write config.json + model.safetensors (BF16, [out, in] row-major).

        text_embedding=True also writes the full 151,936-row text-embedding table (the rows
        ``text_embedding_rows`` generates; ~0.6 GB at text_hidden 2048, ~11 s), which device
        text preparation reads.  It is streamed to the file in row blocks."""
        os.makedirs(model_dir, exist_ok=True)
        with open(os.path.join(model_dir, "config.json"), "w") as f:
            json.dump(self.config(), f, indent=1)
        inv = tensor_inventory(self.spec)
        header: Dict[str, dict] = {"__metadata__": {"format": "pt", "q3t_seed": str(self.seed),
                                                    "q3t_spec": self.spec.name}}
        offset = 0
        for name, shape, _ in inv:
            nbytes = int(np.prod(shape)) * 2
            header[name] = {"dtype": "BF16", "shape": list(shape), "data_offsets": [offset, offset + nbytes]}
            offset += nbytes
        th = self.spec.text_hidden
        if text_embedding:
            nbytes = TEXT_VOCAB * th * 2
            header[TEXT_EMBEDDING_NAME] = {"dtype": "BF16", "shape": [TEXT_VOCAB, th],
                                           "data_offsets": [offset, offset + nbytes]}
            offset += nbytes
        blob = json.dumps(header, separators=(",", ":")).encode()
        blob += b" " * ((8 - len(blob) % 8) % 8)
        path = os.path.join(model_dir, "model.safetensors")
        with open(path + ".tmp", "wb") as f:
            f.write(struct.pack("<Q", len(blob)))
            f.write(blob)
            for name, _, _ in inv:
                f.write(np.ascontiguousarray(self.tensors[name]).tobytes())
            if text_embedding:
                for r0 in range(0, TEXT_VOCAB, 8192):
                    f.write(text_embedding_block(self.seed, r0, min(TEXT_VOCAB, r0 + 8192), th).tobytes())
        os.replace(path + ".tmp", path)


# ----------------------------------------------------------------------------------------
# synthetic speech-tokenizer (codec) checkpoint: speech_tokenizer/model.safetensors
# ----------------------------------------------------------------------------------------
# Shapes of the reference's codec decoder (src/audio/codec_hip.rs:18-45, 214-336).
CODEC = dict(groups=16, codebook=2048, codebook_dim=256, projected=512, pre_conv=1024, hidden=512,
             layers=8, heads=16, head_dim=64, intermediate=1024, upsample=1024, convnext=4096,
             decoder_init=1536, blocks=((1536, 768, 8), (768, 384, 5), (384, 192, 4), (192, 96, 3)),
             final=96)


def codec_inventory(c: dict = CODEC) -> List[Tuple[str, Tuple[int, ...], str]]:
    """(name, shape, kind) of every codec-decoder tensor.  Kinds: fan:N[:g] = N(0, g^2/N) weights
    (so activations stay O(1) through the ~40 layers; g = 0.25 on the residual units' last
    convolutions, whose outputs add up over 12 units), bias, gain (1 + N(0, 0.02)), code (codebook
    sums, N(0, 1)), usage (cluster usage, e^N(0, 0.3)), scale (0.1 + N(0, 0.02): layer scales,
    ConvNeXt gamma), snake (log alpha / log beta, N(0, 0.1))."""
    inv = []
    q = "decoder.quantizer"
    for name, n in (("rvq_first", 1), ("rvq_rest", c["groups"] - 1)):
        for i in range(n):
            p = f"{q}.{name}.vq.layers.{i}._codebook"
            inv += [(f"{p}.embedding_sum", (c["codebook"], c["codebook_dim"]), "code"),
                    (f"{p}.cluster_usage", (c["codebook"],), "usage")]
        inv.append((f"{q}.{name}.output_proj.weight", (c["projected"], c["codebook_dim"], 1),
                    f"fan:{2 * c['codebook_dim']}"))
    inv += [("decoder.pre_conv.conv.weight", (c["pre_conv"], c["projected"], 3), f"fan:{3 * c['projected']}"),
            ("decoder.pre_conv.conv.bias", (c["pre_conv"],), "bias")]
    t, H, Q, I = "decoder.pre_transformer", c["hidden"], c["heads"] * c["head_dim"], c["intermediate"]
    inv += [(f"{t}.input_proj.weight", (H, c["pre_conv"]), f"fan:{c['pre_conv']}"),
            (f"{t}.input_proj.bias", (H,), "bias")]
    for i in range(c["layers"]):
        p = f"{t}.layers.{i}"
        inv += [(f"{p}.input_layernorm.weight", (H,), "gain"),
                (f"{p}.self_attn.q_proj.weight", (Q, H), f"fan:{H}"),
                (f"{p}.self_attn.k_proj.weight", (Q, H), f"fan:{H}"),
                (f"{p}.self_attn.v_proj.weight", (Q, H), f"fan:{H}"),
                (f"{p}.self_attn.o_proj.weight", (H, Q), f"fan:{Q}"),
                (f"{p}.self_attn_layer_scale.scale", (H,), "scale"),
                (f"{p}.post_attention_layernorm.weight", (H,), "gain"),
                (f"{p}.mlp.gate_proj.weight", (I, H), f"fan:{H}"),
                (f"{p}.mlp.up_proj.weight", (I, H), f"fan:{H}"),
                (f"{p}.mlp.down_proj.weight", (H, I), f"fan:{I}"),
                (f"{p}.mlp_layer_scale.scale", (H,), "scale")]
    inv += [(f"{t}.norm.weight", (H,), "gain"),
            (f"{t}.output_proj.weight", (c["pre_conv"], H), f"fan:{H}"),
            (f"{t}.output_proj.bias", (c["pre_conv"],), "bias")]
    U, X = c["upsample"], c["convnext"]
    for i in range(2):
        p = f"decoder.upsample.{i}"
        inv += [(f"{p}.0.conv.weight", (U, U, 2), f"fan:{U}"), (f"{p}.0.conv.bias", (U,), "bias"),
                (f"{p}.1.dwconv.conv.weight", (U, 1, 7), "fan:7"), (f"{p}.1.dwconv.conv.bias", (U,), "bias"),
                (f"{p}.1.norm.weight", (U,), "gain"), (f"{p}.1.norm.bias", (U,), "bias"),
                (f"{p}.1.pwconv1.weight", (X, U), f"fan:{U}"), (f"{p}.1.pwconv1.bias", (X,), "bias"),
                (f"{p}.1.pwconv2.weight", (U, X), f"fan:{X}"), (f"{p}.1.pwconv2.bias", (U,), "bias"),
                (f"{p}.1.gamma", (U,), "scale")]
    inv += [("decoder.decoder.0.conv.weight", (c["decoder_init"], c["pre_conv"], 7), f"fan:{7 * c['pre_conv']}"),
            ("decoder.decoder.0.conv.bias", (c["decoder_init"],), "bias")]
    for b, (ci, co, stride) in enumerate(c["blocks"]):
        p = f"decoder.decoder.{b + 1}.block"
        inv += [(f"{p}.0.alpha", (ci,), "snake"), (f"{p}.0.beta", (ci,), "snake"),
                (f"{p}.1.conv.weight", (ci, co, 2 * stride), f"fan:{2 * ci}"), (f"{p}.1.conv.bias", (co,), "bias")]
        for u in range(3):
            r = f"{p}.{u + 2}"
            inv += [(f"{r}.act1.alpha", (co,), "snake"), (f"{r}.act1.beta", (co,), "snake"),
                    (f"{r}.conv1.conv.weight", (co, co, 7), f"fan:{7 * co}"), (f"{r}.conv1.conv.bias", (co,), "bias"),
                    (f"{r}.act2.alpha", (co,), "snake"), (f"{r}.act2.beta", (co,), "snake"),
                    (f"{r}.conv2.conv.weight", (co, co, 1), f"fan:{co}:0.25"), (f"{r}.conv2.conv.bias", (co,), "bias")]
    inv += [("decoder.decoder.5.alpha", (c["final"],), "snake"), ("decoder.decoder.5.beta", (c["final"],), "snake"),
            ("decoder.decoder.6.conv.weight", (1, c["final"], 7), f"fan:{7 * c['final']}:0.2"),
            ("decoder.decoder.6.conv.bias", (1,), "bias")]
    return inv


def generate_codec_tensor(seed: int, name: str, shape: Tuple[int, ...], kind: str) -> np.ndarray:
    """bf16 bit patterns of one synthetic codec tensor (its own Philox stream, as the model's)."""
    n = int(np.prod(shape))
    z = _philox(seed, "codec:" + name).standard_normal(n, dtype=np.float32)
    if kind.startswith("fan:"):
        parts = kind.split(":")
        gain = float(parts[2]) if len(parts) > 2 else 1.0
        z *= np.float32(gain / np.sqrt(float(parts[1])))
    elif kind == "bias":
        z *= np.float32(0.02)
    elif kind == "gain":
        z = np.float32(1.0) + z * np.float32(0.02)
    elif kind == "usage":
        z = np.exp(z * np.float32(0.3)).astype(np.float32)
    elif kind == "scale":
        z = np.float32(0.1) + z * np.float32(0.02)
    elif kind == "snake":
        z *= np.float32(0.1)
    elif kind != "code":
        raise ValueError(f"unknown codec tensor kind {kind}")
    return f32_to_bf16_bits(z).reshape(shape)


def codec_tensors(seed: int = 0) -> Dict[str, np.ndarray]:
    return {name: generate_codec_tensor(seed, name, shape, kind) for name, shape, kind in codec_inventory()}


def write_codec(model_dir: str, seed: int = 0, tensors: Optional[Dict[str, np.ndarray]] = None) -> None:
    """speech_tokenizer/model.safetensors (BF16) under model_dir, the file the reference's
    codec loader opens (codec_hip.rs:214-215)."""
    tensors = tensors if tensors is not None else codec_tensors(seed)
    d = os.path.join(model_dir, "speech_tokenizer")
    os.makedirs(d, exist_ok=True)
    header: Dict[str, dict] = {"__metadata__": {"format": "pt", "q3t_seed": str(seed)}}
    offset = 0
    names = [name for name, _, _ in codec_inventory()]
    for name in names:
        nbytes = tensors[name].size * 2
        header[name] = {"dtype": "BF16", "shape": list(tensors[name].shape),
                        "data_offsets": [offset, offset + nbytes]}
        offset += nbytes
    blob = json.dumps(header, separators=(",", ":")).encode()
    blob += b" " * ((8 - len(blob) % 8) % 8)
    path = os.path.join(d, "model.safetensors")
    with open(path + ".tmp", "wb") as f:
        f.write(struct.pack("<Q", len(blob)))
        f.write(blob)
        for name in names:
            f.write(np.ascontiguousarray(tensors[name]).tobytes())
    os.replace(path + ".tmp", path)


# ----------------------------------------------------------------------------------------
# synthetic tokenizer files
# ----------------------------------------------------------------------------------------
def byte_level_alphabet() -> List[str]:
    """The 256 byte-level symbols in the GPT-2 / Qwen2 vocabulary order: printable bytes
    first, then the rest mapped above U+0100 (so byte 10, the newline, is id 198)."""
    bs = list(range(ord("!"), ord("~") + 1)) + list(range(0xA1, 0xAC + 1)) + list(range(0xAE, 0xFF + 1))
    cs = list(bs)
    n = 0
    for b in range(256):
        if b not in bs:
            bs.append(b)
            cs.append(256 + n)
            n += 1
    return [chr(c) for c in cs]


# Merges of the synthetic BPE: "assistant" (77091, as the real vocabulary has it) and a few
# words, so that encoding exercises multi-step merges and the space marker.
SYNTH_WORDS = {"assistant": TOKENS["assistant_token_id"], "hello": 9707, "\u0120world": 1879,
               "the": 1782, "\u0120the": 279}
SPECIAL_TOKENS = {151643: "<|endoftext|>", 151644: "<|im_start|>", 151645: "<|im_end|>"}


def write_tokenizer(model_dir: str) -> None:
    """vocab.json + merges.txt + tokenizer_config.json of a small byte-level BPE with the real
    vocabulary size (151,643 ids, unused ids filled with unreachable tokens) and the chat
    specials as added tokens, the files TextTokenizer::from_bpe_files reads (text.rs:195-237)."""
    alphabet = byte_level_alphabet()
    vocab = {ch: i for i, ch in enumerate(alphabet)}
    merges = []
    next_id = 256
    for word, wid in SYNTH_WORDS.items():
        cur = word[0]
        for k in range(1, len(word)):
            merges.append(f"{cur} {word[k]}")
            cur += word[k]
            if cur not in vocab:
                if k == len(word) - 1:
                    vocab[cur] = wid
                else:
                    vocab[cur] = next_id
                    next_id += 1
    used = set(vocab.values())
    filler = (i for i in range(151643) if i not in used)
    for i in filler:
        vocab[f"<|q3t_unused_{i}|>"] = i
    os.makedirs(model_dir, exist_ok=True)
    with open(os.path.join(model_dir, "vocab.json"), "w") as f:
        json.dump(vocab, f, ensure_ascii=False)
    with open(os.path.join(model_dir, "merges.txt"), "w") as f:
        f.write("#version: 0.2\n" + "\n".join(merges) + "\n")
    added = {str(i): dict(content=c, lstrip=False, normalized=False, rstrip=False, single_word=False, special=True)
             for i, c in SPECIAL_TOKENS.items()}
    with open(os.path.join(model_dir, "tokenizer_config.json"), "w") as f:
        json.dump({"added_tokens_decoder": added}, f)


def read_safetensors_bf16(path: str) -> Dict[str, np.ndarray]:
    """Read a BF16 safetensors file into uint16 arrays (memory-mapped)."""
    with open(path, "rb") as f:
        (hlen,) = struct.unpack("<Q", f.read(8))
        header = json.loads(f.read(hlen))
    data = np.memmap(path, dtype=np.uint8, mode="r", offset=8 + hlen)
    out = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        if meta["dtype"] != "BF16":
            raise ValueError(f"{name}: dtype {meta['dtype']} is not BF16")
        b, e = meta["data_offsets"]
        out[name] = data[b:e].view(np.uint16).reshape(meta["shape"])
    return out


def iter_specs() -> Iterator[str]:
    return iter(SPECS)
