"""Logit post-processing and token selection, restated on the CPU.

TEST INFRASTRUCTURE ONLY (the checker for the GPU's fused select kernel).

Order of operations, following the reference's Talker head
(src/model/talker.rs:431-496) and its CPU sampler (src/model/sampling.rs:57-118):

1. repetition penalty over the semantic-token history (Talker only; applied when
   ``penalty != 1`` or sampling is on and the history is non-empty,
   generation.rs:726-734).  ``l < 0 ? l * p : l / p`` (kernels.rs:408-426).  The
   reference's GPU kernel applies it once per *occurrence*; HF's processor (which the
   Python reference runs) applies it once per *distinct* token.  This build follows
   HF: once per distinct token.
2. suppression (Talker only): ``l[i] = -inf`` for ``i in [V-1024, V)`` except
   ``codec_eos`` (kernels.rs:248-263).
3. greedy: argmax, ties to the lowest index (kernels.rs:176-221).
4. sampling: candidates are the finite logits sorted by (value desc, index asc);
   keep ``top_k`` of them (0 keeps all); ``p_i = exp((l_i - l_max) / T)``; nucleus
   keeps the shortest prefix whose normalised mass reaches ``top_p`` (at least one);
   then inverse CDF with ``target = u * sum(kept p)``: the first ``i`` with
   ``target <= p_i`` (subtracting as it goes), else the last kept
   (sampling.rs:57-118, kernels.rs:265-334).
"""
from __future__ import annotations

import dataclasses
from typing import Optional, Sequence, Tuple

import numpy as np


@dataclasses.dataclass(frozen=True)
class SamplingConfig:
    """``SamplingConfig`` (sampling.rs:3-9)."""
    do_sample: bool = False
    top_k: int = 0
    top_p: float = 1.0
    temperature: float = 1.0

    def validate(self, name: str) -> None:
        """sampling.rs:11-26."""
        if not (0.0 < self.top_p <= 1.0):
            raise ValueError(f"{name}.top_p must be in (0, 1], got {self.top_p}")
        if not self.temperature > 0.0:
            raise ValueError(f"{name}.temperature must be positive, got {self.temperature}")


GREEDY = SamplingConfig()


def apply_repetition_penalty(logits: np.ndarray, history: Sequence[int], penalty: float,
                             per_occurrence: bool = False) -> np.ndarray:
    """``l < 0 ? l * p : l / p`` on each penalised token.  Default: once per distinct token of
    the history (HF's processor, which the Python reference runs).  ``per_occurrence``: once per
    history entry, in order, compounding, as apply_repetition_penalty_f32 does over the crate's
    full semantic_history (src/gpu/kernels.rs:408-426; generation.rs:717-727)."""
    out = np.array(logits, copy=True)
    if penalty == 1.0 or len(history) == 0:
        return out
    v = out.shape[-1]
    tokens = [int(h) for h in history] if per_occurrence else sorted(set(int(h) for h in history))
    for t in tokens:
        if 0 <= t < v:
            out[t] = out[t] * penalty if out[t] < 0 else out[t] / penalty
    return out


def suppress(logits: np.ndarray, eos: int) -> np.ndarray:
    out = np.array(logits, copy=True)
    v = out.shape[-1]
    keep = out[eos] if 0 <= eos < v else None
    out[v - 1024:] = -np.inf
    if keep is not None and eos >= v - 1024:
        out[eos] = keep
    return out


def argmax_lowest(logits: np.ndarray) -> int:
    return int(np.argmax(logits))


def kept_distribution(logits: np.ndarray, cfg: SamplingConfig) -> Tuple[np.ndarray, np.ndarray]:
    """(token ids, unnormalised probabilities) of the candidates the sampler can draw."""
    logits = np.asarray(logits, dtype=np.float64)
    finite = np.nonzero(np.isfinite(logits))[0]
    if finite.size == 0:
        raise ValueError("cannot sample from logits with no finite values")
    order = finite[np.lexsort((finite, -logits[finite]))]
    if 0 < cfg.top_k < order.size:
        order = order[:cfg.top_k]
    vals = logits[order]
    probs = np.exp((vals - vals[0]) / cfg.temperature)
    if cfg.top_p < 1.0:
        cum = np.cumsum(probs) / probs.sum()
        keep = int(np.searchsorted(cum, cfg.top_p, side="left")) + 1
        keep = max(1, min(keep, order.size))
        order, probs = order[:keep], probs[:keep]
    return order, probs


def sample(logits: np.ndarray, cfg: SamplingConfig, u: float) -> int:
    tokens, probs = kept_distribution(logits, cfg)
    target = u * probs.sum()
    for t, p in zip(tokens, probs):
        if target <= p:
            return int(t)
        target -= p
    return int(tokens[-1])


def select(logits: np.ndarray, cfg: SamplingConfig, u: Optional[float]) -> int:
    if not cfg.do_sample:
        return argmax_lowest(logits)
    return sample(logits, cfg, u)


def top2_margin(logits: np.ndarray) -> float:
    """Gap between the two largest finite logits (how close an argmax is to a tie)."""
    finite = np.asarray(logits, dtype=np.float64)
    finite = finite[np.isfinite(finite)]
    if finite.size < 2:
        return float("inf")
    a = np.partition(finite, -2)[-2:]
    return float(a[1] - a[0])
