"""16-bit PCM output of generated audio: ``GeneratedSpeech::to_wav_bytes`` / ``write_wav``
(src/generation.rs:1521-1553, src/audio/codec.rs:5-27).

A sample becomes ``(sample * gain)`` clamped to [-1, 1], times 32767, converted to int16 with
Rust's float-to-integer cast (truncation toward zero; NaN becomes 0).  The file is mono,
little-endian, with the 44-byte RIFF / ``fmt `` (PCM, 16 bytes) / ``data`` header.
"""
from __future__ import annotations

import os
import struct
from typing import Union

import numpy as np

MAX_DATA_BYTES = 0xFFFFFFFF - 36  # generation.rs:1531-1534


class WavError(ValueError):
    """``Error::InvalidInput`` of the wav writers."""


def pcm_s16le(samples: np.ndarray, gain: float = 1.0) -> bytes:
    """The data bytes: one little-endian int16 per sample."""
    x = np.asarray(samples, dtype=np.float32) * np.float32(gain)
    x = np.clip(x, np.float32(-1.0), np.float32(1.0)) * np.float32(32767.0)
    x = np.where(np.isnan(x), np.float32(0.0), x)
    return np.trunc(x).astype("<i2").tobytes()


def wav_bytes(samples: np.ndarray, sample_rate: int, gain: float = 1.0) -> bytes:
    """``to_wav_bytes``: header + data."""
    n = int(np.asarray(samples).size)
    data_bytes = 2 * n
    if data_bytes > MAX_DATA_BYTES:
        raise WavError("wav is too large")
    header = b"RIFF" + struct.pack("<I", 36 + data_bytes) + b"WAVEfmt " + struct.pack(
        "<IHHIIHH", 16, 1, 1, sample_rate, sample_rate * 2, 2, 16) + b"data" + struct.pack("<I", data_bytes)
    return header + pcm_s16le(samples, gain)


def write_wav(path: Union[str, os.PathLike], samples: np.ndarray, sample_rate: int, gain: float = 1.0) -> None:
    """``write_wav``: the same bytes in a file."""
    data = wav_bytes(samples, sample_rate, gain)
    try:
        with open(path, "wb") as f:
            f.write(data)
    except OSError as err:
        raise WavError(f"failed to create {path}: {err}") from None
