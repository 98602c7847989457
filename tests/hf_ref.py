"""transformers' Qwen3Model as an independent reference for the oracle's decoder stacks.

The library model (installed; not the reference) is loaded with a synthetic checkpoint's
stack weights and evaluated in float64.  Two of its float32 steps are replaced by the same
formulas in float64:

* the RoPE angles (HF computes ``position * inv_freq`` in float32; supplied here in float64,
  HF's layout: cos/sin of cat(freqs, freqs));
* Qwen3RMSNorm (casts its input to float32).

Attention runs through torch's scaled_dot_product_attention ("sdpa"), which stays in float64
on the CPU.  A comparison with the float64 oracle then agrees to ~1e-14; a wrong sign, index,
position or operand shows up as O(0.1).
"""
from __future__ import annotations

import numpy as np
import torch

from q3t import synth


def bf64(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(synth.bf16_bits_to_f32(bits).astype(np.float64))


def qwen3_model(tensors: dict, prefix: str, hidden: int, intermediate: int, layers: int, q_heads: int,
                kv_heads: int, head_dim: int, eps: float, theta: float):
    """A float64 transformers Qwen3Model holding the stack ``{prefix}.layers.*`` and
    ``{prefix}.norm.weight`` of ``tensors`` (bf16 bits).  Its output is the final-normed
    hidden state."""
    from transformers.models.qwen3 import modeling_qwen3 as mq

    cfg = mq.Qwen3Config(hidden_size=hidden, intermediate_size=intermediate, num_hidden_layers=layers,
                         num_attention_heads=q_heads, num_key_value_heads=kv_heads, head_dim=head_dim,
                         rms_norm_eps=eps, vocab_size=8, max_position_embeddings=8192,
                         rope_parameters={"rope_type": "default", "rope_theta": theta},
                         attention_bias=False, attn_implementation="sdpa")
    hf = mq.Qwen3Model(cfg).to(torch.float64).eval()
    pre = prefix + "."
    sd = {k[len(pre):]: bf64(v) for k, v in tensors.items()
          if k.startswith(pre) and (k[len(pre):].startswith("layers.") or k[len(pre):] == "norm.weight")}
    sd["embed_tokens.weight"] = torch.zeros(8, hidden, dtype=torch.float64)
    missing, unexpected = hf.load_state_dict(sd, strict=False)
    assert not unexpected, unexpected
    assert all("rotary" in m for m in missing), missing

    def rotary64(x, position_ids):
        inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float64) / head_dim))
        freqs = position_ids[..., None].to(torch.float64) * inv
        emb = torch.cat([freqs, freqs], dim=-1)
        return emb.cos(), emb.sin()

    hf.rotary_emb.forward = rotary64

    def norm64(self, h):
        return self.weight * (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + self.variance_epsilon))

    for mod in hf.modules():
        if isinstance(mod, mq.Qwen3RMSNorm):
            mod.forward = norm64.__get__(mod)
    return hf


def stack_from_config(tensors: dict, cfg: dict, prefix: str):
    """``qwen3_model`` with the shape read from a config.json section (talker_config or
    code_predictor_config)."""
    return qwen3_model(tensors, prefix, cfg["hidden_size"], cfg["intermediate_size"], cfg["num_hidden_layers"],
                       cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"],
                       cfg["rms_norm_eps"], cfg["rope_theta"])


def forward(hf, rows: np.ndarray) -> np.ndarray:
    """Final-normed hidden states of one causal sequence, positions 0 .. len(rows) - 1."""
    with torch.no_grad():
        x = torch.from_numpy(np.asarray(rows, dtype=np.float64))[None]
        return hf(inputs_embeds=x).last_hidden_state[0].numpy()
