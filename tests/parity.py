"""Comparison rules between a GPU rollout and an oracle fixture.

Codes are compared exactly and over the whole length: the GPU path computes in fp32 with
an fp32 KV cache against a float64 oracle, so its tokens must equal the oracle's at every
frame of every committed fixture.  A failure prints the oracle's top-2 margin at the first
differing token, which tells a near tie (a margin of the order of the logit error) from a
real fault.

``check_codes_near_tie`` is for comparisons with a model that rounds differently by
design (a bf16 KV cache): there a divergence is accepted only at an argmax whose oracle
top-2 margin is below TIE_TOL, and everything after it is a different trajectory.

Logits are compared on every row computed from an identical token history, against the
north-star bound of 2e-2 max-abs.  Fixtures keep every row as float16 (enough for the bound)
and their first rows again as float32, from which the reported error is measured.
"""
from __future__ import annotations

import json
import os
import warnings
from typing import Optional, Tuple

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TIE_TOL = 1e-3
LOGIT_TOL = 2e-2


def load_fixture(name: str) -> dict:
    z = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    out = {k: z[k] for k in z.files}
    out["meta"] = json.loads(str(out["meta"]))
    return out


def fixture_exists(name: str) -> bool:
    return os.path.exists(os.path.join(GOLDEN, f"{name}.npz"))


def first_divergence(a: np.ndarray, b: np.ndarray) -> Optional[Tuple[int, int]]:
    n = min(len(a), len(b))
    diff = np.nonzero(a[:n] != b[:n])
    if diff[0].size == 0:
        return None
    order = np.lexsort((diff[1], diff[0]))
    return int(diff[0][order[0]]), int(diff[1][order[0]])


def _divergence_message(gpu_codes, fx, f, g) -> str:
    ref = fx["codes"]
    margin = fx["talker_margins"][f] if g == 0 else fx["cp_margins"][f][g - 1]
    return (f"codes diverge at frame {f} group {g}: GPU {gpu_codes[f].tolist()} vs oracle "
            f"{ref[f].tolist()} (oracle top-2 margin there {margin:.3g})")


def check_codes(gpu_codes: np.ndarray, gpu_eos: bool, fx: dict) -> int:
    """Full-length identity: every frame, the frame count and the EOS flag.  Returns the
    number of frames."""
    ref = fx["codes"]
    d = first_divergence(gpu_codes, ref)
    assert d is None, _divergence_message(gpu_codes, fx, *d)
    assert len(gpu_codes) == len(ref), f"GPU made {len(gpu_codes)} frames, oracle {len(ref)}"
    assert bool(gpu_eos) == bool(fx["meta"]["ended_by_eos"]), "EOS flag differs"
    return len(ref)


def check_codes_near_tie(gpu_codes: np.ndarray, gpu_eos: bool, fx: dict) -> int:
    """Returns the number of leading identical frames; a divergence must sit at a near tie."""
    d = first_divergence(gpu_codes, fx["codes"])
    if d is None:
        return check_codes(gpu_codes, gpu_eos, fx)
    f, g = d
    margin = fx["talker_margins"][f] if g == 0 else fx["cp_margins"][f][g - 1]
    msg = _divergence_message(gpu_codes, fx, f, g)
    assert margin < TIE_TOL, msg
    warnings.warn("near-tie divergence accepted: " + msg)
    return f


def check_talker_logits(gpu_logits: np.ndarray, fx: dict, same_frames: int) -> float:
    """Row r is computed from the tokens of frames < r, so rows 0..same_frames are comparable.
    Every comparable row is held to LOGIT_TOL; the returned error is measured on the float32
    rows where the fixture has them."""
    ref = fx["talker_logits"].astype(np.float32)
    rows = min(len(gpu_logits), len(ref), same_frames + 1)
    assert rows > 0
    err = float(np.abs(gpu_logits[:rows] - ref[:rows]).max())
    assert err <= LOGIT_TOL, f"Talker logits differ by {err:.3g} (> {LOGIT_TOL})"
    if "talker_logits_f32" in fx:
        ref32 = fx["talker_logits_f32"]
        rows = min(len(gpu_logits), len(ref32), same_frames + 1)
        err = float(np.abs(gpu_logits[:rows] - ref32[:rows]).max())
    return err


def check_cp_logits(gpu_cp_logits: np.ndarray, fx: dict) -> float:
    """CodePredictor logits of the fixture's first frames ([frames, 15, Vc])."""
    ref = fx["cp_logits"].astype(np.float32)
    n = min(len(gpu_cp_logits), len(ref))
    assert n > 0
    err = float(np.abs(gpu_cp_logits[:n] - ref[:n]).max())
    assert err <= LOGIT_TOL, f"CodePredictor logits differ by {err:.3g} (> {LOGIT_TOL})"
    return err
