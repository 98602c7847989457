"""The codec-decoder oracle (oracle/codec.py), pinned without the reference's code:

* each primitive against the torch library routine in float64: causal (dilated) conv1d,
  right-trimmed conv_transpose1d, layer_norm, erf GELU, causal scaled-dot-product attention;
  RoPE against the same rotation written with complex numbers;
* Snake and the RVQ gather by closed form (a zero code row, the modulo of out-of-range codes);
* end to end on the synthetic codec: 1920 samples per frame in [-1, 1], and causality: the
  decode of a prefix of the frames is the prefix of the decode (what chunked streaming
  relies on), with the streaming chunk of generation.rs:965-989 equal to the full decode's
  slice when the left context covers the history.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import codec as C
from q3t import synth

rng = np.random.default_rng(0)


def test_causal_conv_is_torch_conv1d():
    for k, d in [(7, 1), (7, 3), (7, 9), (3, 1), (1, 1)]:
        x, w, b = rng.standard_normal((40, 5)), rng.standard_normal((6, 5, k)), rng.standard_normal(6)
        xt = F.pad(torch.from_numpy(x.T[None]), ((k - 1) * d, 0))
        ref = F.conv1d(xt, torch.from_numpy(w), torch.from_numpy(b), dilation=d)[0].numpy().T
        np.testing.assert_allclose(C.causal_conv(x, w, b, d), ref, rtol=1e-12, atol=1e-12)


def test_transposed_conv_is_torch_conv_transpose1d_right_trimmed():
    for s, k in [(2, 2), (8, 16), (5, 10), (3, 6)]:
        x, w, b = rng.standard_normal((9, 4)), rng.standard_normal((4, 3, k)), rng.standard_normal(3)
        ref = F.conv_transpose1d(torch.from_numpy(x.T[None]), torch.from_numpy(w), torch.from_numpy(b),
                                 stride=s)[0].numpy().T[:9 * s]
        np.testing.assert_allclose(C.transposed_conv(x, w, b, s), ref, rtol=1e-12, atol=1e-12)


def test_norms_gelu_attention_are_torch():
    x, g, b = rng.standard_normal((7, 32)), rng.standard_normal(32), rng.standard_normal(32)
    np.testing.assert_allclose(C.layernorm(x, g, b, 1e-6),
                               F.layer_norm(torch.from_numpy(x), (32,), torch.from_numpy(g), torch.from_numpy(b),
                                            1e-6).numpy(), rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(C.rmsnorm(x, g, 1e-5),
                               F.rms_norm(torch.from_numpy(x), (32,), torch.from_numpy(g), 1e-5).numpy(),
                               rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(C.gelu(x), F.gelu(torch.from_numpy(x)).numpy(), rtol=1e-12, atol=1e-12)
    q, k, v = (rng.standard_normal((11, 4, 8)) for _ in range(3))
    ref = F.scaled_dot_product_attention(*(torch.from_numpy(a.transpose(1, 0, 2)) for a in (q, k, v)),
                                         is_causal=True).numpy().transpose(1, 0, 2)
    np.testing.assert_allclose(C.causal_attention(q, k, v), ref, rtol=1e-10, atol=1e-12)


def test_rope_is_a_complex_rotation():
    x = rng.standard_normal((6, 3, 64))
    z = x[..., :32] + 1j * x[..., 32:]
    ang = np.arange(6)[:, None, None] * (1e4 ** (-np.arange(32) * 2 / 64))[None, None, :]
    rot = z * np.exp(1j * ang)
    np.testing.assert_allclose(C.rope(x, 1e4), np.concatenate([rot.real, rot.imag], -1), rtol=1e-12, atol=1e-12)


def test_snake_and_rvq_closed_forms():
    x = rng.standard_normal((4, 3))
    np.testing.assert_allclose(C.snake(x, np.zeros(3), np.zeros(3)), x + np.sin(x) ** 2 / (1 + 1e-9))
    o = C.CodecOracle(synth.codec_tensors(0))
    t = o.t
    codes = np.zeros((2, 16), np.int64)
    codes[1, 3] = 2048 + 7                                   # out of range: taken modulo 2048
    cb = lambda p, r: t[f"{p}.embedding_sum"][r] / max(t[f"{p}.cluster_usage"][r], 1e-7)
    q = "decoder.quantizer"
    first = cb(f"{q}.rvq_first.vq.layers.0._codebook", 0)
    rest = [sum(cb(f"{q}.rvq_rest.vq.layers.{g}._codebook", 7 if (f, g) == (1, 2) else 0) for g in range(15))
            for f in range(2)]
    for f in range(2):
        expect = t[f"{q}.rvq_first.output_proj.weight"][:, :, 0] @ first + \
            t[f"{q}.rvq_rest.output_proj.weight"][:, :, 0] @ rest[f]
        np.testing.assert_allclose(o.rvq(codes)[f], expect, rtol=1e-12, atol=1e-12)


@pytest.fixture(scope="module")
def oracle():
    return C.CodecOracle(synth.codec_tensors(0))


def test_decode_shape_range_and_causality(oracle):
    codes = np.random.default_rng(3).integers(0, 2048, (5, 16))
    full, st = oracle.decode(codes, stages=True)
    assert full.shape == (5 * C.SAMPLES_PER_FRAME,)
    assert np.abs(full).max() <= 1.0 and np.isfinite(st["raw"]).all()
    assert 0.01 < np.abs(st["raw"]).mean() < 1.0               # the synthetic scales keep the signal O(1)
    head = oracle.decode(codes[:3])
    np.testing.assert_allclose(head, full[:3 * C.SAMPLES_PER_FRAME], rtol=0, atol=1e-12)
    chunk = C.stream_chunk_samples(oracle, codes, 3, 5, left_context=25)
    np.testing.assert_allclose(chunk, full[3 * C.SAMPLES_PER_FRAME:], rtol=0, atol=1e-12)
