"""16-bit PCM / WAV output (q3t.wav) against GeneratedSpeech::to_wav_bytes
(src/generation.rs:1530-1553): the header fields and the sample conversion, checked against
hand-computed values and against the standard-library wave reader."""
import io
import struct
import wave

import numpy as np
import pytest

from q3t import wav
from q3t.engine import GeneratedSpeech


def test_sample_conversion_known_values():
    x = np.array([0.0, 1.0, -1.0, 2.0, -3.0, 0.5, -0.5, 1e-5, -1e-5, 0.99999, np.nan, np.inf, -np.inf],
                 dtype=np.float32)
    got = np.frombuffer(wav.pcm_s16le(x), dtype="<i2")
    # (clamp(x) * 32767) truncated toward zero; NaN -> 0
    assert got.tolist() == [0, 32767, -32767, 32767, -32767, 16383, -16383, 0, 0, 32766, 0, 32767, -32767]
    g = np.frombuffer(wav.pcm_s16le(np.array([0.25, -0.3], np.float32), gain=2.0), dtype="<i2")
    assert g.tolist() == [int(np.float32(0.5) * np.float32(32767)), int(np.float32(-0.6) * np.float32(32767))]


def test_header_layout_and_round_trip(tmp_path):
    rng = np.random.default_rng(0)
    s = (rng.standard_normal(4801) * 0.3).astype(np.float32)
    b = wav.wav_bytes(s, 24000, gain=1.5)
    assert len(b) == 44 + 2 * s.size
    assert b[:4] == b"RIFF" and struct.unpack("<I", b[4:8])[0] == 36 + 2 * s.size and b[8:16] == b"WAVEfmt "
    assert struct.unpack("<IHHIIHH", b[16:36]) == (16, 1, 1, 24000, 48000, 2, 16)
    assert b[36:40] == b"data" and struct.unpack("<I", b[40:44])[0] == 2 * s.size
    with wave.open(io.BytesIO(b)) as w:
        assert (w.getnchannels(), w.getsampwidth(), w.getframerate(), w.getnframes()) == (1, 2, 24000, s.size)
        pcm = np.frombuffer(w.readframes(s.size), dtype="<i2")
    ref = np.trunc(np.clip(s * np.float32(1.5), -1, 1) * np.float32(32767)).astype(np.int16)
    np.testing.assert_array_equal(pcm, ref)
    sp = GeneratedSpeech("t", 2, False, np.zeros((2, 16), np.int32), s, 24000)
    assert sp.audio_seconds() == pytest.approx(4801 / 24000)
    assert sp.to_wav_bytes(1.5) == b
    sp.write_wav(tmp_path / "a.wav", 1.5)
    assert (tmp_path / "a.wav").read_bytes() == b


def test_empty_and_errors(tmp_path):
    b = wav.wav_bytes(np.zeros(0, np.float32), 24000)
    assert len(b) == 44 and struct.unpack("<I", b[40:44])[0] == 0
    with pytest.raises(wav.WavError, match="failed to create"):
        wav.write_wav(tmp_path / "missing_dir" / "a.wav", np.zeros(4, np.float32), 24000)
