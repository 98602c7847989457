"""The codec oracle's stage wiring (oracle/codec.py), pinned against transformers' own
Qwen3-Omni code-to-wave modules on the synthetic codec checkpoint, in float64.

The primitives are pinned one by one in tests/test_oracle_codec.py; these tests pin how the
oracle chains them, which a wiring mistake made the same way in the oracle and in the device
decoder would otherwise pass:

* the ConvNeXt half of each upsample stage (depthwise conv, LayerNorm, pointwise, GELU,
  pointwise, gamma, residual) against ``Qwen3OmniMoeConvNeXtBlock``;
* each of the 12 residual units (Snake, dilated conv k 7, Snake, conv k 1, residual) against
  ``Qwen3OmniMoeCode2WavDecoderResidualUnit`` with the reference's dilations 1 / 3 / 9;
* each decoder block: its leading Snake against ``Qwen3OmniMoeSnakeBeta``, and its chain after
  the transposed conv against the library's three residual units in sequence (the library's
  ``Qwen3OmniMoeCausalTransConvNet`` trims the transposed conv's output on both sides, the
  reference only on the right (src/gpu/kernels.rs:652-685), so the transposed conv itself
  stays on its primitive test);
* the decoder's first conv (k 7) and its closing Snake + conv (k 7) against
  ``Qwen3OmniMoeCausalConvNet`` / ``Qwen3OmniMoeSnakeBeta``.

The parameter names of the library modules are the checkpoint's (the reference reads the
same names, src/audio/codec_hip.rs:656-1072), so each module loads the oracle's float64
tensors by name.  Planted mistakes in a copy of the oracle (act and conv swapped, gamma
dropped, a wrong dilation, the two Snakes' parameters swapped) must fail the same checks.
"""
import numpy as np
import pytest
import torch

from oracle import codec as C
from q3t import synth

M = pytest.importorskip("transformers.models.qwen3_omni_moe.modeling_qwen3_omni_moe")

TOL = 1e-10


@pytest.fixture(scope="module")
def oracle():
    return C.CodecOracle(synth.codec_tensors(0))


def _load(module: torch.nn.Module, t: dict, prefix: str) -> torch.nn.Module:
    module = module.double()
    state = {name: torch.from_numpy(np.ascontiguousarray(t[f"{prefix}.{name}"])) for name in module.state_dict()}
    module.load_state_dict(state, strict=True)
    return module.eval()


def _run(module: torch.nn.Module, x: np.ndarray) -> np.ndarray:
    """A library module on time-major x [T, C] (the library is channel-major [1, C, T])."""
    with torch.no_grad():
        return module(torch.from_numpy(np.ascontiguousarray(x.T))[None])[0].numpy().T


def _rel(a: np.ndarray, b: np.ndarray) -> float:
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def _input(T: int, ch: int, seed: int, scale: float = 1.0) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal((T, ch)) * scale


def _unit_module(o, b, u):
    dim = C.BLOCKS[b][1]
    return _load(M.Qwen3OmniMoeCode2WavDecoderResidualUnit(dim, (1, 3, 9)[u]), o.t, f"decoder.decoder.{b + 1}.block.{u + 2}")


# ----------------------------------------------------------------------------------------- pins
@pytest.mark.parametrize("i", [0, 1])
def test_convnext_half_of_upsample_is_the_library_block(oracle, i):
    y = _input(24, 1024, i, 2.0)
    lib = _load(M.Qwen3OmniMoeConvNeXtBlock(1024), oracle.t, f"decoder.upsample.{i}.1")
    assert _rel(oracle.convnext(y, i), _run(lib, y)) < TOL
    # and upsample = the right-trimmed transposed conv, then that block
    x = _input(12, 1024, 10 + i)
    t, p = oracle.t, f"decoder.upsample.{i}.0.conv"
    np.testing.assert_array_equal(oracle.upsample(x, i),
                                  oracle.convnext(C.transposed_conv(x, t[f"{p}.weight"], t[f"{p}.bias"], 2), i))


@pytest.mark.parametrize("b", range(4))
@pytest.mark.parametrize("u", range(3))
def test_residual_unit_is_the_library_unit(oracle, b, u):
    dim = C.BLOCKS[b][1]
    h = _input(40, dim, 100 * b + u, 0.5)
    assert _rel(oracle.residual_unit(h, b, u), _run(_unit_module(oracle, b, u), h)) < TOL


@pytest.mark.parametrize("b", range(4))
def test_decoder_block_chain_is_the_library_chain(oracle, b):
    in_dim, out_dim, stride = C.BLOCKS[b]
    t, p = oracle.t, f"decoder.decoder.{b + 1}.block"
    # the leading Snake
    x = _input(10, in_dim, 200 + b)
    snake = _load(M.Qwen3OmniMoeSnakeBeta(in_dim), t, f"{p}.0")
    np.testing.assert_allclose(C.snake(x, t[f"{p}.0.alpha"], t[f"{p}.0.beta"]), _run(snake, x), rtol=TOL, atol=TOL)
    # the block = Snake, transposed conv (right-trimmed, primitive-tested), then the library's
    # three residual units in order
    y = C.transposed_conv(_run(snake, x), t[f"{p}.1.conv.weight"], t[f"{p}.1.conv.bias"], stride)
    for u in range(3):
        y = _run(_unit_module(oracle, b, u), y)
    assert _rel(oracle.decoder_block(x, b), y) < TOL


def test_decoder_head_and_tail_are_library_convs(oracle):
    t = oracle.t
    x = _input(16, 1024, 300)
    head = _load(M.Qwen3OmniMoeCausalConvNet(1024, 1536, 7), t, "decoder.decoder.0")
    assert _rel(C.causal_conv(x, t["decoder.decoder.0.conv.weight"], t["decoder.decoder.0.conv.bias"]), _run(head, x)) < TOL
    h = _input(64, 96, 301)
    snake = _load(M.Qwen3OmniMoeSnakeBeta(96), t, "decoder.decoder.5")
    last = _load(M.Qwen3OmniMoeCausalConvNet(96, 1, 7), t, "decoder.decoder.6")
    ours = C.causal_conv(C.snake(h, t["decoder.decoder.5.alpha"], t["decoder.decoder.5.beta"]),
                         t["decoder.decoder.6.conv.weight"], t["decoder.decoder.6.conv.bias"])
    assert _rel(ours, _run(last, _run(snake, h))) < TOL


# ------------------------------------------------------------------------------ planted mistakes
class _SwappedActConv(C.CodecOracle):
    """Residual unit with the first Snake after its conv instead of before."""

    def residual_unit(self, h, b, u):
        t, r, dil = self.t, f"decoder.decoder.{b + 1}.block.{u + 2}", (1, 3, 9)[u]
        a = C.causal_conv(h, t[f"{r}.conv1.conv.weight"], t[f"{r}.conv1.conv.bias"], dil)
        a = C.snake(a, t[f"{r}.act1.alpha"], t[f"{r}.act1.beta"])
        a = C.snake(a, t[f"{r}.act2.alpha"], t[f"{r}.act2.beta"])
        return h + C.causal_conv(a, t[f"{r}.conv2.conv.weight"], t[f"{r}.conv2.conv.bias"])


class _WrongDilation(C.CodecOracle):
    """Residual units all at dilation 1."""

    def residual_unit(self, h, b, u):
        t, r = self.t, f"decoder.decoder.{b + 1}.block.{u + 2}"
        a = C.snake(h, t[f"{r}.act1.alpha"], t[f"{r}.act1.beta"])
        a = C.causal_conv(a, t[f"{r}.conv1.conv.weight"], t[f"{r}.conv1.conv.bias"], 1)
        a = C.snake(a, t[f"{r}.act2.alpha"], t[f"{r}.act2.beta"])
        return h + C.causal_conv(a, t[f"{r}.conv2.conv.weight"], t[f"{r}.conv2.conv.bias"])


class _SwappedSnakes(C.CodecOracle):
    """The unit's two Snakes with each other's parameters."""

    def residual_unit(self, h, b, u):
        t, r, dil = self.t, f"decoder.decoder.{b + 1}.block.{u + 2}", (1, 3, 9)[u]
        a = C.snake(h, t[f"{r}.act2.alpha"], t[f"{r}.act2.beta"])
        a = C.causal_conv(a, t[f"{r}.conv1.conv.weight"], t[f"{r}.conv1.conv.bias"], dil)
        a = C.snake(a, t[f"{r}.act1.alpha"], t[f"{r}.act1.beta"])
        return h + C.causal_conv(a, t[f"{r}.conv2.conv.weight"], t[f"{r}.conv2.conv.bias"])


class _NoGamma(C.CodecOracle):
    """ConvNeXt block without its gamma scale."""

    def convnext(self, y, i):
        t, p = self.t, f"decoder.upsample.{i}.1"
        w = t[f"{p}.dwconv.conv.weight"][:, 0, :]
        yp = np.concatenate([np.zeros((6, y.shape[1])), y], axis=0)
        d = t[f"{p}.dwconv.conv.bias"] + sum(yp[j:j + y.shape[0]] * w[:, j] for j in range(7))
        n = C.layernorm(d, t[f"{p}.norm.weight"], t[f"{p}.norm.bias"], 1e-6)
        a = C.gelu(n @ t[f"{p}.pwconv1.weight"].T + t[f"{p}.pwconv1.bias"])
        return y + a @ t[f"{p}.pwconv2.weight"].T + t[f"{p}.pwconv2.bias"]


@pytest.mark.parametrize("mutant", [_SwappedActConv, _WrongDilation, _SwappedSnakes])
def test_planted_unit_mistakes_fail_the_pin(oracle, mutant):
    bad = mutant.__new__(mutant)
    bad.t = oracle.t
    failed = []
    for b in range(4):
        for u in range(3):
            if _WrongDilation is mutant and u == 0:
                continue  # dilation 1 is right for the first unit
            h = _input(40, C.BLOCKS[b][1], 100 * b + u, 0.5)
            failed.append(_rel(bad.residual_unit(h, b, u), _run(_unit_module(oracle, b, u), h)) > 1e-6)
    assert all(failed), failed


@pytest.mark.parametrize("i", [0, 1])
def test_planted_gamma_drop_fails_the_pin(oracle, i):
    bad = _NoGamma.__new__(_NoGamma)
    bad.t = oracle.t
    y = _input(24, 1024, i, 2.0)
    lib = _load(M.Qwen3OmniMoeConvNeXtBlock(1024), oracle.t, f"decoder.upsample.{i}.1")
    assert _rel(bad.convnext(y, i), _run(lib, y)) > 1e-6
