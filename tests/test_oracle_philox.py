"""Philox4x32-10 against the Random123 known-answer vectors (Salmon et al., SC'11,
kat_vectors: philox4x32 with 10 rounds)."""
import numpy as np
import pytest

from oracle.philox import philox4x32_10, sampler_uniform

KAT = [
    ([0x00000000, 0x00000000, 0x00000000, 0x00000000], [0x00000000, 0x00000000],
     [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]),
    ([0xffffffff, 0xffffffff, 0xffffffff, 0xffffffff], [0xffffffff, 0xffffffff],
     [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]),
    ([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], [0xa4093822, 0x299f31d0],
     [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]),
]


@pytest.mark.parametrize("ctr,key,want", KAT)
def test_known_answers(ctr, key, want):
    got = philox4x32_10(np.array(ctr, dtype=np.uint64), np.array(key, dtype=np.uint64))
    assert [int(x) for x in got] == want


def test_vectorised_matches_scalar():
    ctrs = np.array([[i, 3, 0, 0] for i in range(16)], dtype=np.uint64)
    keys = np.tile(np.array([5, 0], dtype=np.uint64), (16, 1))
    batch = philox4x32_10(ctrs, keys)
    for i in range(16):
        assert np.array_equal(batch[i], philox4x32_10(ctrs[i], keys[i]))


def test_uniform_range_and_mean():
    u = np.array([sampler_uniform(0, s, k) for s in range(400) for k in range(5)])
    assert u.min() >= 0.0 and u.max() < 1.0
    assert abs(u.mean() - 0.5) < 0.03
    # 24-bit resolution
    assert np.all((u * (1 << 24)) == np.floor(u * (1 << 24)))
