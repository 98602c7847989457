"""The BASELINE workloads (configs 1-5) as concrete, seeded inputs.

Every workload fixes the synthetic model (spec + weight seed), the prompt (random content
ids), how the prompt is split between prefill and trailing text, the KV capacity and the
generation options.  Tests, fixtures and bench.py all build their inputs from here.

KV capacity: the reference requires ``P + max_frames <= max_cache_steps``
(src/generation.rs:608-617).  Config 2 states a capacity of 256 for 240 frames; with
streaming pulls the prefill holds 9 + ``text_lookahead_tokens`` rows, so a lookahead of 7
(P = 16) is the largest that fits 256 exactly.  Config 4 (capacity 512, 480 frames) fits
with the default lookahead of 8 (P = 17).
"""
from __future__ import annotations

import dataclasses
from typing import Dict, Optional

import numpy as np

from . import synth, textprep


@dataclasses.dataclass(frozen=True)
class Workload:
    name: str
    spec: str
    prompt_tokens: int
    prompt_seed: int
    frames: int
    max_cache_steps: int
    lookahead: Optional[int]      # None: non-streaming generate_codes (all text in the prefill)
    chunk_frames: int = 6
    do_sample: bool = False
    top_k: int = 50
    top_p: float = 1.0
    temperature: float = 0.9
    repetition_penalty: float = 1.0
    sample_seed: int = 0
    weight_seed: int = 0

    def options_kwargs(self) -> dict:
        if self.do_sample:
            return dict(max_frames=self.frames, do_sample=True, top_k=self.top_k, top_p=self.top_p,
                        temperature=self.temperature, repetition_penalty=self.repetition_penalty,
                        subtalker_dosample=True, subtalker_top_k=self.top_k, subtalker_top_p=self.top_p,
                        subtalker_temperature=self.temperature, seed=self.sample_seed)
        return dict(max_frames=self.frames, do_sample=False, repetition_penalty=self.repetition_penalty,
                    subtalker_dosample=False, seed=self.sample_seed)

    def prompt(self) -> np.ndarray:
        return textprep.random_prompt(self.prompt_tokens, self.prompt_seed)

    def inputs(self, model: "synth.SyntheticModel") -> "textprep.PreparedInputs":
        prep = textprep.TextPrep(model)
        look = (1 << 30) if self.lookahead is None else self.lookahead
        return prep.prepare(self.prompt(), text_lookahead_tokens=look)


WORKLOADS: Dict[str, Workload] = {w.name: w for w in [
    # config 1: CPU reference case (non-streaming, P = 41)
    Workload("cfg1_cpu_0.6b", "0.6b", 32, 1, 40, 512, None),
    # config 2: 0.6B bf16 greedy, 64-token prompt, 240 frames, KV 256, pulls of 6
    Workload("cfg2_0.6b_greedy", "0.6b", 64, 1, 240, 256, 7),
    # config 3: config 2 with sampling on both heads
    Workload("cfg3_0.6b_sampled", "0.6b", 64, 1, 240, 256, 7, do_sample=True, top_k=50, top_p=1.0,
             temperature=0.9, repetition_penalty=1.05, sample_seed=0),
    # config 4: 1.7B greedy, 128-token prompt, 480 frames, KV 512
    Workload("cfg4_1.7b_greedy", "1.7b", 128, 1, 480, 512, 8),
    # small shapes for quick parity runs
    Workload("tiny_greedy", "tiny", 32, 1, 24, 128, None),
    Workload("tiny_sampled", "tiny", 32, 1, 24, 128, 4, do_sample=True, top_k=50, top_p=0.9,
             temperature=0.9, repetition_penalty=1.05, sample_seed=7),
    Workload("tinyproj_greedy", "tiny-proj", 24, 3, 16, 128, None),
]}


@dataclasses.dataclass(frozen=True)
class MultiWorkload:
    """independent streams generated together on one engine.

    Stream j's prompt length, frame budget and content ids come from one generator seeded
    with `seed`, in this order: all lengths, all frame budgets, then each prompt.  Every
    prompt goes into the prefill whole (non-streaming, P = 9 + length), so the prefill is one
    matrix-core GEMM over all streams' rows.  The KV capacity is max(P + frames) rounded up
    to 64.  With `sampled_every` = k > 0, every k-th stream (j % k == k - 1) samples with
    the config-3 options and seed j; the rest are greedy."""
    name: str
    spec: str
    streams: int
    prompt_range: tuple   # content tokens, inclusive
    frames_range: tuple   # inclusive
    seed: int
    chunk_frames: int = 6
    sampled_every: int = 0
    weight_seed: int = 0

    def plan(self):
        rng = np.random.default_rng(self.seed)
        lengths = rng.integers(self.prompt_range[0], self.prompt_range[1] + 1, self.streams)
        frames = rng.integers(self.frames_range[0], self.frames_range[1] + 1, self.streams)
        prompts = [rng.integers(0, 151643, int(n)) for n in lengths]
        return [int(n) for n in lengths], [int(f) for f in frames], prompts

    @property
    def max_cache_steps(self) -> int:
        lengths, frames, _ = self.plan()
        need = max(9 + n + f for n, f in zip(lengths, frames))
        return (need + 63) // 64 * 64

    def options_kwargs(self):
        _, frames, _ = self.plan()
        out = []
        for j, f in enumerate(frames):
            if self.sampled_every and j % self.sampled_every == self.sampled_every - 1:
                out.append(dict(max_frames=f, do_sample=True, top_k=50, top_p=1.0, temperature=0.9,
                                repetition_penalty=1.05, subtalker_dosample=True, subtalker_top_k=50,
                                subtalker_top_p=1.0, subtalker_temperature=0.9, seed=j))
            else:
                out.append(dict(max_frames=f, do_sample=False, repetition_penalty=1.0, subtalker_dosample=False,
                                seed=0))
        return out

    def inputs(self, model: "synth.SyntheticModel"):
        prep = textprep.TextPrep(model)
        return [prep.prepare(p) for p in self.plan()[2]]


MULTI_WORKLOADS: Dict[str, MultiWorkload] = {w.name: w for w in [
    # config 5: 16 streams, prompts U[16, 512], frames U[64, 240], seed 2
    MultiWorkload("cfg5_0.6b_multistream", "0.6b", 16, (16, 512), (64, 240), 2),
    # small shapes: ragged greedy + sampled streams for quick parity runs
    MultiWorkload("tiny_multistream", "tiny", 6, (4, 40), (8, 24), 5, chunk_frames=5, sampled_every=3),
    # every stream greedy: the batched frame's token hand-off (no CodePredictor selection
    # kernels before the last group)
    MultiWorkload("tiny_multistream_greedy", "tiny", 5, (4, 40), (8, 24), 7, chunk_frames=5),
    # the Talker -> CodePredictor projection (1.7B layout) on the batched path
    MultiWorkload("tinyproj_multistream", "tiny-proj", 3, (4, 24), (6, 14), 6, chunk_frames=4, sampled_every=2),
    # a CodePredictor wide enough for the split O / down GEMMs and the two-position prefix
    # pass (hidden 1024), behind a 512 -> 1024 projection, one query head per KV head
    MultiWorkload("tinyg1_multistream", "tiny-g1", 4, (4, 24), (6, 14), 8, chunk_frames=4, sampled_every=3),
]}
