"""Codec decoder on the GPU (q3t_decode_codes, q3t_stream_next_audio) against the float64 CPU
oracle of the reference's decoder (oracle/codec.py), on the synthetic speech-tokenizer
checkpoint.  Frame counts 3 and 10 put the decoder stages on both matrix-core GEMM paths
(fewer and more than 128 rows); 70 frames take the pre-transformer attention past one pass of
its four waves' 32-key stride and its 64-key softmax loop."""
import numpy as np
import pytest

from oracle import codec as C
from q3t import engine as E
from q3t import synth

pytestmark = pytest.mark.gpu

# fp32 pipeline (exact bf16 x fp32 products, fp32 sums) over ~45 layers vs float64; samples
# are ~0.3 in magnitude and clamped to [-1, 1]
WAVE_TOL = 2e-3


@pytest.fixture(scope="module")
def codec_case(models):
    model, d = models.get_with_text("tiny")
    eng = E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=128))
    yield eng, C.CodecOracle(synth.codec_tensors(0))
    eng.close()


@pytest.mark.parametrize("frames", [3, 10, 70])
def test_decode_matches_oracle(codec_case, frames):
    eng, oracle = codec_case
    assert eng.has_codec and eng.info["samples_per_frame"] == C.SAMPLES_PER_FRAME
    codes = np.random.default_rng(frames).integers(0, 2048, (frames, 16)).astype(np.int32)
    print(f"[gpu] decode_codes frames={frames}", flush=True)
    got = eng.decode_codes(codes)
    ref = oracle.decode(codes)
    assert got.shape == ref.shape == (frames * C.SAMPLES_PER_FRAME,)
    err = float(np.abs(got - ref).max())
    print(f"decode {frames} frames: max err {err:.2e}, mean |x| {float(np.abs(ref).mean()):.3f}")
    assert err <= WAVE_TOL


def test_decode_is_causal_and_wraps_codes(codec_case):
    eng, _ = codec_case
    codes = np.random.default_rng(7).integers(0, 2048, (8, 16)).astype(np.int32)
    full = eng.decode_codes(codes)
    head = eng.decode_codes(codes[:5])
    np.testing.assert_allclose(head, full[:5 * C.SAMPLES_PER_FRAME], rtol=0, atol=1e-5)
    wrapped = codes.copy()
    wrapped[:, 4] += 2048                      # codes are taken modulo the codebook size
    np.testing.assert_array_equal(eng.decode_codes(wrapped), full)
    assert eng.decode_codes(np.zeros((0, 16), np.int32)).size == 0


def test_stream_audio_chunks(codec_case):
    eng, oracle = codec_case
    from q3t.workloads import WORKLOADS
    w = WORKLOADS["tiny_greedy"]
    model, _ = eng, None
    inputs = w.inputs(synth.SyntheticModel.build("tiny", 0))
    opts = E.GenerateOptions.greedy(10)
    for ctx in (25, 2):
        st = eng.start_stream(inputs, opts, E.StreamOptions(left_context_frames=ctx))
        chunks = []
        while (c := st.next_audio_chunk(4)) is not None:
            assert c.samples.shape == (c.frames * C.SAMPLES_PER_FRAME,) and c.sample_rate == 24000
            chunks.append(c)
        codes = np.concatenate(st._codes)
        st.close()
        assert [c.frames for c in chunks] == [4, 4, 2]
        got = np.concatenate([c.samples for c in chunks])
        ref = np.concatenate([C.stream_chunk_samples(oracle, codes, s, e, ctx) for s, e in ((0, 4), (4, 8), (8, 10))])
        err = float(np.abs(got - ref).max())
        print(f"stream audio, left context {ctx}: max err {err:.2e}")
        assert err <= WAVE_TOL


def test_generate_returns_audio(codec_case):
    eng, _ = codec_case
    text = "hello world"
    sp = eng.generate(text, E.GenerateOptions.greedy(6, decode_audio=True))
    assert sp.frames == 6 and sp.samples.shape == (6 * C.SAMPLES_PER_FRAME,) and sp.sample_rate == 24000
    np.testing.assert_allclose(sp.samples, eng.decode_codes(sp.codes), rtol=0, atol=0)


def test_no_codec_checkpoint(models):
    _, plain = models.get("tiny")
    with E.HipTtsEngine(plain, E.EngineOptions(max_cache_steps=64)) as e2:
        assert not e2.has_codec
        with pytest.raises(E.NotFoundError):
            e2.decode_codes(np.zeros((2, 16), np.int32))
