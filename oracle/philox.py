"""Philox4x32-10 counter-based RNG (Salmon, Moraes, Dror, Shaw, "Parallel random numbers:
as easy as 1, 2, 3", SC'11), restated in numpy.

TEST INFRASTRUCTURE ONLY: this module is the checker for the GPU sampler's random
stream.  Pinned by the Random123 known-answer vectors in tests/test_oracle_philox.py.

The sampler draws one uniform per sampled token (the reference draws one f32 per
token from its LCG, src/model/sampling.rs:120-126 and code_predictor.rs:433-440).
Stream layout used by both the GPU and this oracle:

    key     = (seed & 0xffffffff, seed >> 32)
    counter = (step, kind, slot, 0)
        kind 0       Talker token; step 0 is the prefill token, step f+1 the token
                     decoded after frame f
        kind 1 + g   CodePredictor acoustic group g (0..14) of frame ``step``
    u       = (word0 >> 8) * 2**-24          in [0, 1)
"""
from __future__ import annotations

import numpy as np

M0 = 0xD2511F53
M1 = 0xCD9E8D57
W0 = 0x9E3779B9
W1 = 0xBB67AE85
MASK = 0xFFFFFFFF


def philox4x32_10(counter, key):
    """Vectorised Philox4x32 with 10 rounds.  counter: (..., 4) uint32, key: (..., 2) uint32."""
    c = np.asarray(counter, dtype=np.uint64) & MASK
    k = np.asarray(key, dtype=np.uint64) & MASK
    c0, c1, c2, c3 = (c[..., i].copy() for i in range(4))
    k0, k1 = k[..., 0].copy(), k[..., 1].copy()
    for r in range(10):
        p0 = np.uint64(M0) * c0
        p1 = np.uint64(M1) * c2
        hi0, lo0 = p0 >> np.uint64(32), p0 & np.uint64(MASK)
        hi1, lo1 = p1 >> np.uint64(32), p1 & np.uint64(MASK)
        c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
        if r != 9:
            k0 = (k0 + np.uint64(W0)) & np.uint64(MASK)
            k1 = (k1 + np.uint64(W1)) & np.uint64(MASK)
    return np.stack([c0, c1, c2, c3], axis=-1).astype(np.uint32)


def sampler_uniform(seed: int, step: int, kind: int, slot: int = 0) -> float:
    key = np.array([seed & MASK, (seed >> 32) & MASK], dtype=np.uint64)
    ctr = np.array([step & MASK, kind & MASK, slot & MASK, 0], dtype=np.uint64)
    w0 = int(philox4x32_10(ctr, key)[0])
    return (w0 >> 8) * (1.0 / (1 << 24))
