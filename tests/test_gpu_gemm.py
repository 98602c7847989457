"""The matrix-core GEMM (bf16 weights, fp32 activations as three bf16 terms, fp32 accumulate)
against a float64 numpy product, through the C ABI test hook q3t_debug_gemm."""
import numpy as np
import pytest

from q3t import engine as E
from q3t import synth
from q3t.workloads import WORKLOADS

pytestmark = pytest.mark.gpu

# Activations enter as three bf16 terms (24 significant bits), so every product with a bf16
# weight is exact; what remains is fp32 accumulation (~1e-7 relative over these K).
REL_TOL = 2e-6


@pytest.fixture(scope="module")
def eng(models):
    w = WORKLOADS["tiny_greedy"]
    _, d = models.get(w.spec)
    e = E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=64))
    yield e
    e.close()


def _weights(rows, K, seed):
    return synth.f32_to_bf16_bits((np.random.default_rng(seed).standard_normal((rows, K)) * 0.02).astype(np.float32))


def _close(got, want):
    scale = np.abs(want).max()
    err = np.abs(got - want).max() / scale
    assert err < REL_TOL, f"max error {err:.3g} of scale {scale:.3g}"
    return err


@pytest.mark.parametrize("M,N,K", [(1, 64, 32), (16, 1024, 1024), (17, 300, 64), (73, 4096, 1024),
                                   (521, 1024, 3072), (5, 2048, 2048), (16, 1024, 3072), (1, 3072, 1024),
                                   (9, 100, 6144), (521, 96, 1024), (300, 192, 672), (130, 288, 384)])
def test_store(eng, M, N, K):
    print(f"[gpu] gemm store M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M * 7 + N)
    X = rng.standard_normal((M, K)).astype(np.float32)
    Wb = _weights(N, K, N + K)
    W = synth.bf16_bits_to_f32(Wb).astype(np.float64)
    got = eng.debug_gemm(0, X, Wb, N)
    _close(got, X.astype(np.float64) @ W.T)


def test_epilogues_and_norm(eng):
    M, N, K = 37, 384, 1024
    rng = np.random.default_rng(3)
    X = (rng.standard_normal((M, K)) * 3).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    Xn = X.astype(np.float64) / np.sqrt((X.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6) * g
    Wb = _weights(2 * N, K, 11)
    W = synth.bf16_bits_to_f32(Wb).astype(np.float64)
    res = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    # residual (+ RMSNorm prologue)
    _close(eng.debug_gemm(1, X, Wb[:N], N, gamma=g, res=res), res + Xn @ W[:N].T)
    # bias
    _close(eng.debug_gemm(3, X, Wb[:N], N, bias=bias), X.astype(np.float64) @ W[:N].T + bias)
    # SwiGLU over gate rows [0, N) and up rows [N, 2N)
    gate, up = Xn @ W[:N].T, Xn @ W[N:].T
    _close(eng.debug_gemm(2, X, Wb, N, gamma=g), gate / (1 + np.exp(-gate)) * up)


@pytest.mark.parametrize("N", [96, 192])
def test_epilogues_96_column_blocks(eng, N):
    """M >= 128 with N a multiple of 96 but not of 128 (the codec's 96- and 192-channel
    convolutions) runs the LDS-tiled kernel in 96-column blocks: bias, and residual with the
    RMSNorm prologue."""
    M, K = 200, 672
    print(f"[gpu] gemm 96-column blocks M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(N)
    X = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    Xn = X.astype(np.float64) / np.sqrt((X.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6) * g
    Wb = _weights(N, K, N + 1)
    W = synth.bf16_bits_to_f32(Wb).astype(np.float64)
    res = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    _close(eng.debug_gemm(3, X, Wb, N, bias=bias), X.astype(np.float64) @ W.T + bias)
    _close(eng.debug_gemm(1, X, Wb, N, gamma=g, res=res), res + Xn @ W.T)


@pytest.mark.parametrize("M", [16, 40])
def test_epilogues_skinny_and_tiled(eng, M):
    """M <= 16 runs the batched-decode kernel (fused RMSNorm), larger M the prefill kernel."""
    N, K = 208, 1024
    rng = np.random.default_rng(M)
    X = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    Xn = X.astype(np.float64) / np.sqrt((X.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6) * g
    Wb = _weights(2 * N, K, M + 5)
    W = synth.bf16_bits_to_f32(Wb).astype(np.float64)
    res = rng.standard_normal((M, N)).astype(np.float32)
    _close(eng.debug_gemm(0, X, Wb[:N], N, gamma=g), Xn @ W[:N].T)
    _close(eng.debug_gemm(1, X, Wb[:N], N, res=res), res + X.astype(np.float64) @ W[:N].T)
    gate, up = Xn @ W[:N].T, Xn @ W[N:].T
    _close(eng.debug_gemm(2, X, Wb, N, gamma=g), gate / (1 + np.exp(-gate)) * up)


@pytest.mark.parametrize("M,N,K", [(16, 1024, 2048), (16, 1024, 3072), (5, 256, 1024), (11, 64, 6144),
                                   (1, 2048, 4096)])
def test_residual_k_split(eng, M, N, K):
    """The batched frame's O / down form: K in two halves whose sums meet in fp32 atomic adds
    on a zeroed T16 output, the first half adding the residual and zeroing the next GEMM's
    accumulator (the hook fails if any of its M x N elements is left nonzero).  Two adds onto
    zero commute, so repeated calls agree bit for bit."""
    print(f"[gpu] gemm residual K split M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M * 13 + K)
    X = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    Wb = _weights(N, K, N * 3 + K)
    W = synth.bf16_bits_to_f32(Wb).astype(np.float64)
    res = rng.standard_normal((M, N)).astype(np.float32)
    got = eng.debug_gemm(4, X, Wb, N, res=res)
    _close(got, res + X.astype(np.float64) @ W.T)
    assert np.array_equal(got.view(np.uint32), eng.debug_gemm(4, X, Wb, N, res=res).view(np.uint32))
    # the same product through the single-pass kernel, to fp32 summation order
    np.testing.assert_allclose(got, eng.debug_gemm(1, X, Wb, N, res=res), rtol=0, atol=2e-6 * np.abs(got).max())


def test_rejects_bad_shapes(eng):
    with pytest.raises(E.InvalidInputError):
        eng.debug_gemm(0, np.zeros((4, 48), np.float32), np.zeros((8, 48), np.uint16), 8)
    with pytest.raises(E.InvalidInputError):  # the K split needs K = 1024 * c
        eng.debug_gemm(4, np.zeros((4, 512), np.float32), np.zeros((32, 512), np.uint16), 32,
                       res=np.zeros((4, 32), np.float32))


@pytest.mark.parametrize("M,K", [(128, 1024), (300, 2048), (521, 1024)])
def test_prefill_tiles_all_epilogues(eng, M, K):
    """M >= 128 with K % 64 == 0 runs the LDS-tiled prefill kernel: RMSNorm rows (1/rms and
    gain applied on the way into LDS), store / residual / SwiGLU / bias epilogues."""
    print(f"[gpu] gemm tiles M={M} K={K}", flush=True)
    N = 256
    rng = np.random.default_rng(M + K)
    X = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    Xn = X.astype(np.float64) / np.sqrt((X.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6) * g
    Wb = _weights(2 * N, K, M * 3 + 1)
    W = synth.bf16_bits_to_f32(Wb).astype(np.float64)
    res = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    _close(eng.debug_gemm(0, X, Wb[:N], N, gamma=g), Xn @ W[:N].T)
    _close(eng.debug_gemm(1, X, Wb[:N], N, res=res), res + X.astype(np.float64) @ W[:N].T)
    _close(eng.debug_gemm(3, X, Wb[:N], N, bias=bias), X.astype(np.float64) @ W[:N].T + bias)
    gate, up = Xn @ W[:N].T, Xn @ W[N:].T
    _close(eng.debug_gemm(2, X, Wb, N, gamma=g), gate / (1 + np.exp(-gate)) * up)
