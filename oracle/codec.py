"""CPU restatement of the codec decoder that turns codec frames into 24 kHz audio.

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this module; it is the checker the
device codec decoder (q3t_decode_codes) is compared against.

Sources restated (reference = /root/reference of piedshag/qwen3-tts-hip):

* shapes and the stage order:                    src/audio/codec_hip.rs:18-45, 214-336
* RVQ dequantisation + 1x1 output projections:   src/audio/codec_hip.rs:338-378, 2135-2170;
                                                 src/gpu/kernels.rs:454-495 (codec_rvq_project_f32)
* causal (dilated) convolution:                  kernels.rs:497-526, 742-770 (padding (k-1)*dilation,
                                                 codec_hip.rs:1370-1394)
* pre-transformer (RMSNorm eps 1e-5, RoPE theta  codec_hip.rs:380-654; kernels.rs:40-77 (rope_bhsd),
  1e4 over head_dim 64, causal attention, layer  980-1040 (attention_scores_causal / apply_value),
  scales, SwiGLU MLP)                            596-608 (scaled residual add)
* upsample stages: transposed conv k = stride = 2, codec_hip.rs:656-800; kernels.rs:614-640
  ConvNeXt block (depthwise causal k 7, LayerNorm (transconv1d), 642-690 (depthwise, convnext
  eps 1e-6, pointwise 4096 GELU(erf), gamma)     residual), 582-612 (layernorm), 572-580 (gelu)
* decoder: causal conv k 7, 4 blocks (Snake,     codec_hip.rs:802-1072, 1253-1368;
  transposed conv k = 2 stride right-trimmed,    kernels.rs:692-710 (snake_beta), 787-816
  residual units dilation 1 / 3 / 9), Snake,     (transconv1d_channels), 903-918 (clamp)
  conv k 7 to one channel, clamp to [-1, 1]
* chunked streaming with left context:           src/generation.rs:619-647, 965-989

Arithmetic is float64 on the checkpoint's bf16 values; activations are time-major [T, C]
(the reference keeps channel-major [C, T]; the layout does not change the arithmetic).
"""
from __future__ import annotations

from typing import Dict

import numpy as np

SAMPLES_PER_FRAME = 1920
BLOCKS = ((1536, 768, 8), (768, 384, 5), (384, 192, 4), (192, 96, 3))


def _f64(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def causal_conv(x: np.ndarray, w: np.ndarray, b: np.ndarray, dilation: int = 1) -> np.ndarray:
    """y[t, o] = b[o] + sum_{c, j} x[t + j*d - (k-1)*d, c] w[o, c, j] (zero outside [0, T))."""
    T = x.shape[0]
    out_c, in_c, k = w.shape
    pad = (k - 1) * dilation
    xp = np.concatenate([np.zeros((pad, in_c)), x], axis=0)
    y = np.tile(b, (T, 1)).astype(np.float64)
    for j in range(k):
        y += xp[j * dilation:j * dilation + T] @ np.ascontiguousarray(w[:, :, j].T)
    return y


def transposed_conv(x: np.ndarray, w: np.ndarray, b: np.ndarray, stride: int) -> np.ndarray:
    """y[t*s + j, o] += x[t, c] w[c, o, j] for j < k, outputs past T*s dropped, + b."""
    T = x.shape[0]
    in_c, out_c, k = w.shape
    y = np.zeros((T * stride + k, out_c))
    for j in range(k):
        y[j:j + T * stride:stride] += x @ np.ascontiguousarray(w[:, :, j])
    return y[:T * stride] + b


def snake(x: np.ndarray, log_alpha: np.ndarray, log_beta: np.ndarray) -> np.ndarray:
    """x + sin(x e^alpha)^2 / (e^beta + 1e-9), per channel."""
    return x + np.sin(x * np.exp(log_alpha)) ** 2 / (np.exp(log_beta) + 1e-9)


def rmsnorm(x: np.ndarray, g: np.ndarray, eps: float) -> np.ndarray:
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * g


def layernorm(x: np.ndarray, g: np.ndarray, b: np.ndarray, eps: float) -> np.ndarray:
    mu = x.mean(axis=-1, keepdims=True)
    var = np.maximum((x * x).mean(axis=-1, keepdims=True) - mu * mu, 0.0)
    return (x - mu) / np.sqrt(var + eps) * g + b


def gelu(x: np.ndarray) -> np.ndarray:
    from scipy.special import erf
    return 0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))


def rope(x: np.ndarray, theta: float) -> np.ndarray:
    """Rotate-half RoPE over [T, heads, d] at positions 0..T-1: pairs (i, i + d/2), angle
    t / theta^(2i/d)."""
    T, _, d = x.shape
    half = d // 2
    inv = theta ** (-(2.0 * np.arange(half)) / d)
    ang = np.arange(T)[:, None] * inv[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    a, b2 = x[..., :half], x[..., half:]
    return np.concatenate([a * c - b2 * s, b2 * c + a * s], axis=-1)


def causal_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray) -> np.ndarray:
    """[T, heads, d] each; softmax(q k^T / sqrt(d)) over keys <= query, applied to v."""
    T, h, d = q.shape
    s = np.einsum("thd,uhd->htu", q, k) / np.sqrt(d)
    s = np.where(np.tril(np.ones((T, T), dtype=bool))[None], s, -np.inf)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("htu,uhd->thd", p, v)


class CodecOracle:
    def __init__(self, tensors: Dict[str, np.ndarray]):
        self.t = {n: _f64(v) for n, v in tensors.items()}

    def _cb(self, prefix: str) -> np.ndarray:
        # load_normalized_codebook (codec_hip.rs:2135-2154)
        return self.t[f"{prefix}.embedding_sum"] / np.maximum(self.t[f"{prefix}.cluster_usage"], 1e-7)[:, None]

    def rvq(self, codes: np.ndarray) -> np.ndarray:
        t, q = self.t, "decoder.quantizer"
        codes = np.asarray(codes, dtype=np.int64) % 2048
        first = self._cb(f"{q}.rvq_first.vq.layers.0._codebook")[codes[:, 0]]
        rest = sum(self._cb(f"{q}.rvq_rest.vq.layers.{g - 1}._codebook")[codes[:, g]] for g in range(1, 16))
        return (first @ t[f"{q}.rvq_first.output_proj.weight"][:, :, 0].T
                + rest @ t[f"{q}.rvq_rest.output_proj.weight"][:, :, 0].T)

    def pre_transformer(self, x: np.ndarray) -> np.ndarray:
        t, p = self.t, "decoder.pre_transformer"
        h = x @ t[f"{p}.input_proj.weight"].T + t[f"{p}.input_proj.bias"]
        T = h.shape[0]
        for i in range(8):
            L = f"{p}.layers.{i}"
            n = rmsnorm(h, t[f"{L}.input_layernorm.weight"], 1e-5)
            q = rope((n @ t[f"{L}.self_attn.q_proj.weight"].T).reshape(T, 16, 64), 1e4)
            k = rope((n @ t[f"{L}.self_attn.k_proj.weight"].T).reshape(T, 16, 64), 1e4)
            v = (n @ t[f"{L}.self_attn.v_proj.weight"].T).reshape(T, 16, 64)
            o = causal_attention(q, k, v).reshape(T, 1024) @ t[f"{L}.self_attn.o_proj.weight"].T
            h = h + o * t[f"{L}.self_attn_layer_scale.scale"]
            n = rmsnorm(h, t[f"{L}.post_attention_layernorm.weight"], 1e-5)
            g = n @ t[f"{L}.mlp.gate_proj.weight"].T
            m = (g / (1.0 + np.exp(-g)) * (n @ t[f"{L}.mlp.up_proj.weight"].T)) @ t[f"{L}.mlp.down_proj.weight"].T
            h = h + m * t[f"{L}.mlp_layer_scale.scale"]
        n = rmsnorm(h, t[f"{p}.norm.weight"], 1e-5)
        return n @ t[f"{p}.output_proj.weight"].T + t[f"{p}.output_proj.bias"]

    def convnext(self, y: np.ndarray, i: int) -> np.ndarray:
        """The ConvNeXt block of upsample stage i on the transposed conv's output y
        (codec_hip.rs:700-800): depthwise causal conv k 7, LayerNorm eps 1e-6, pointwise 4C +
        GELU(erf), pointwise back to C, times gamma, plus y."""
        t, p = self.t, f"decoder.upsample.{i}.1"
        dw = y.shape[1]
        w = t[f"{p}.dwconv.conv.weight"][:, 0, :]               # [C, 7]
        yp = np.concatenate([np.zeros((6, dw)), y], axis=0)
        d = t[f"{p}.dwconv.conv.bias"] + sum(yp[j:j + y.shape[0]] * w[:, j] for j in range(7))
        n = layernorm(d, t[f"{p}.norm.weight"], t[f"{p}.norm.bias"], 1e-6)
        a = gelu(n @ t[f"{p}.pwconv1.weight"].T + t[f"{p}.pwconv1.bias"])
        u = a @ t[f"{p}.pwconv2.weight"].T + t[f"{p}.pwconv2.bias"]
        return y + u * t[f"{p}.gamma"]

    def upsample(self, x: np.ndarray, i: int) -> np.ndarray:
        """Upsample stage i (codec_hip.rs:656-800): transposed conv k = stride = 2, then the
        ConvNeXt block."""
        t, p = self.t, f"decoder.upsample.{i}"
        y = transposed_conv(x, t[f"{p}.0.conv.weight"], t[f"{p}.0.conv.bias"], 2)
        return self.convnext(y, i)

    def residual_unit(self, h: np.ndarray, b: int, u: int) -> np.ndarray:
        """Residual unit u (dilation 1, 3, 9) of decoder block b (codec_hip.rs:1253-1368):
        h + conv k 1(Snake(conv k 7, dilated(Snake(h))))."""
        t, r, dil = self.t, f"decoder.decoder.{b + 1}.block.{u + 2}", (1, 3, 9)[u]
        a = snake(h, t[f"{r}.act1.alpha"], t[f"{r}.act1.beta"])
        a = causal_conv(a, t[f"{r}.conv1.conv.weight"], t[f"{r}.conv1.conv.bias"], dil)
        a = snake(a, t[f"{r}.act2.alpha"], t[f"{r}.act2.beta"])
        return h + causal_conv(a, t[f"{r}.conv2.conv.weight"], t[f"{r}.conv2.conv.bias"])

    def decoder_block(self, h: np.ndarray, b: int) -> np.ndarray:
        """Decoder block b (codec_hip.rs:802-1072): Snake, the right-trimmed transposed conv
        (kernel 2 x stride), then the three residual units."""
        t, p = self.t, f"decoder.decoder.{b + 1}.block"
        h = snake(h, t[f"{p}.0.alpha"], t[f"{p}.0.beta"])
        h = transposed_conv(h, t[f"{p}.1.conv.weight"], t[f"{p}.1.conv.bias"], BLOCKS[b][2])
        for u in range(3):
            h = self.residual_unit(h, b, u)
        return h

    def decoder(self, x: np.ndarray) -> np.ndarray:
        t = self.t
        h = causal_conv(x, t["decoder.decoder.0.conv.weight"], t["decoder.decoder.0.conv.bias"])
        for b in range(len(BLOCKS)):
            h = self.decoder_block(h, b)
        h = snake(h, t["decoder.decoder.5.alpha"], t["decoder.decoder.5.beta"])
        return causal_conv(h, t["decoder.decoder.6.conv.weight"], t["decoder.decoder.6.conv.bias"])[:, 0]

    def decode(self, codes: np.ndarray, stages: bool = False):
        """``decode_codes`` (generation.rs:619-647): codes [F, 16] -> F * 1920 samples in [-1, 1]."""
        t = self.t
        q = self.rvq(codes)
        pc = causal_conv(q, t["decoder.pre_conv.conv.weight"], t["decoder.pre_conv.conv.bias"])
        tr = self.pre_transformer(pc)
        u0 = self.upsample(tr, 0)
        u1 = self.upsample(u0, 1)
        raw = self.decoder(u1)
        wav = np.clip(raw, -1.0, 1.0)
        if stages:
            return wav, dict(rvq=q, pre_conv=pc, pre_transformer=tr, upsample0=u0, upsample1=u1, raw=raw)
        return wav


def stream_chunk_samples(oracle: CodecOracle, codes: np.ndarray, start: int, end: int, left_context: int):
    """``next_audio_chunk`` (generation.rs:965-989): decode frames [start - context, end) and
    drop the context's samples."""
    ctx = min(left_context, start)
    wav = oracle.decode(codes[start - ctx:end])
    return wav[ctx * SAMPLES_PER_FRAME:]
