"""The algorithmic byte counts behind bench.py's rooflines (per-step, per-frame and batched
multi-stream figures), pinned by their closed forms: parameter counts of the 0.6B and 1.7B
shapes (weights in bf16), KV rows per cached position, and a brute-force walk over batched
frames."""
import numpy as np
import pytest

import bench
from q3t import synth


def _params(s):
    """Matrices and the four norm gains of every layer."""
    q, kv = s.q_heads * s.head_dim, s.kv_heads * s.head_dim
    per_layer = (q + 2 * kv) * s.hidden + s.hidden * q + 3 * s.intermediate * s.hidden + 2 * s.hidden + 2 * s.head_dim
    return s.layers * per_layer


@pytest.mark.parametrize("name,layer_params,talker_step,cp_pass", [
    ("0.6b", 15_730_944, 887_226_368, 161_505_792),
    ("1.7b", 50_336_000, 2_831_403_008, 165_700_096),
])
def test_step_bytes_closed_forms(name, layer_params, talker_step, cp_pass):
    spec = synth.SPECS[name]
    assert _params(spec.talker) == 28 * layer_params
    assert _params(spec.code_predictor) == 5 * 15_730_944
    for kv_elem in (2, 4):
        t, c, kv_t, kv_c = bench.step_bytes(spec, kv_elem)
        # Talker: stack + codec head (3072 x H) + final norm; CodePredictor pass: stack + one LM
        # head (2048 x 1024) + final norm (+ the 2048 -> 1024 projection of the 1.7B shape)
        assert (t, c) == (talker_step, cp_pass)
        # K and V, every layer, 8 KV heads x 128 dims per cached position
        assert kv_t == 28 * 2 * 8 * 128 * kv_elem and kv_c == 5 * 2 * 8 * 128 * kv_elem
    assert bench.step_bytes(spec, 2)[2] == 114_688


@pytest.mark.parametrize("name,weights", [("0.6b", 3_309_813_248), ("1.7b", 5_316_904_448)])
def test_frame_bytes_weights_and_kv(name, weights):
    spec = synth.SPECS[name]
    t, c, kv_t, kv_c = bench.step_bytes(spec, 4)
    assert t + 15 * c == weights
    # the frame adds the Talker rows at the mean active length and the CodePredictor's rows
    for active in (0.0, 40.5, 136.5):
        got = bench.frame_bytes(spec, active, 4)
        assert got == pytest.approx(weights + kv_t * active + kv_c * sum(range(1, 17)), rel=0, abs=1e-3)


def test_batched_bytes_is_a_walk_over_batched_frames():
    spec = synth.SPECS["0.6b"]
    rng = np.random.default_rng(7)
    prefill = [int(p) for p in rng.integers(25, 521, 9)]
    frames = [int(f) for f in rng.integers(1, 40, 9)]
    for kv_elem in (2, 4):
        t, c, kv_t, kv_c = bench.step_bytes(spec, kv_elem)
        cp_rows = sum(range(2, 17)) + 2  # the prefix pass and the 14 single-row groups of one frame
        want = 0
        for f in range(max(frames)):
            want += t + 15 * c                       # every weight once per batched frame
            for p, fr in zip(prefill, frames):
                if f < fr:                           # the stream is live in batched frame f
                    want += kv_c * cp_rows
                    if f < fr - 1:                   # its Talker step at position p + f
                        want += kv_t * (p + f + 2)
        assert bench.batched_bytes(spec, prefill, frames, kv_elem) == want
    # a bf16 cache halves exactly the KV part
    w = max(frames) * (t + 15 * c)
    b4, b2 = bench.batched_bytes(spec, prefill, frames, 4), bench.batched_bytes(spec, prefill, frames, 2)
    assert b4 - w == 2 * (b2 - w)
