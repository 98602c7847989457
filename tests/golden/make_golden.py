"""Writes the golden fixtures under tests/golden/ from the float64 CPU oracle.

    python tests/golden/make_golden.py [workload ...]

Each fixture holds one oracle rollout of a workload from q3t/workloads.py: the codes,
the raw Talker logits (every row as float16 for the 2e-2 bound, and the first rows again as
float32 so the measured error is not the fixture's rounding), the top-2 margins of every
argmax (printed when a parity check fails) and the first frames' CodePredictor logits
(float32), plus the weight checksum so a test can tell that it rebuilt the same synthetic
model.

A multi-stream workload (MULTI_WORKLOADS) holds one independent single-stream rollout per
stream (streams do not interact), with the first Talker logit rows of each.
"""
from __future__ import annotations

import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "qwen3-tts-hip_amd"))

from oracle.model import GenerateOptions, Oracle  # noqa: E402
from q3t import synth  # noqa: E402
from q3t.workloads import MULTI_WORKLOADS, WORKLOADS  # noqa: E402

# Talker-logit rows kept per fixture (the codes and margins are always complete).
MAX_LOGIT_ROWS = 256
F32_LOGIT_ROWS = 48
CP_LOGIT_FRAMES = 2
MULTI_LOGIT_ROWS = 4


def make(name: str) -> str:
    w = WORKLOADS[name]
    t0 = time.time()
    model = synth.SyntheticModel.build(w.spec, w.weight_seed)
    inputs = w.inputs(model)
    oracle = Oracle(model.tensors, model.config(), max_cache_steps=w.max_cache_steps, dtype=np.float64)
    opts = GenerateOptions(**w.options_kwargs())
    tr = oracle.rollout(inputs.prefill, inputs.trailing_text, inputs.tts_pad_embed, opts,
                        keep_cp_logits=CP_LOGIT_FRAMES)
    meta = dict(workload=name, spec=w.spec, weight_seed=w.weight_seed, checksum=model.checksum(),
                prefill_steps=inputs.prefill_steps, trailing_steps=inputs.trailing_steps,
                frames=tr.frames, ended_by_eos=tr.ended_by_eos, options=w.options_kwargs(),
                oracle_dtype="float64", seconds=round(time.time() - t0, 1))
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(
        path, meta=np.array(json.dumps(meta)), codes=tr.codes,
        talker_logits=tr.talker_logits[:MAX_LOGIT_ROWS].astype(np.float16),
        talker_logits_f32=tr.talker_logits[:F32_LOGIT_ROWS].astype(np.float32),
        talker_margins=tr.talker_margins, cp_margins=tr.cp_margins,
        cp_logits=np.asarray(tr.cp_logits, dtype=np.float32),
        prefill_sum=np.array([float(np.sum(inputs.prefill, dtype=np.float64))]))
    print(f"{name}: {tr.frames} frames, eos={tr.ended_by_eos}, {meta['seconds']} s -> {path}", flush=True)
    return path


def deterministic_hidden(length: int, modulus: float, center: float) -> np.ndarray:
    """The reference's fixture input (python-reference/qwen3_tts_reference.py:620-626)."""
    return np.array([((i % int(modulus)) - center) / modulus for i in range(length)], dtype=np.float32)


# Parity-hook fixtures: one per model spec, from the workload whose prefill they reuse.
HOOK_WORKLOADS = {"tiny": "tiny_greedy", "tiny-proj": "tinyproj_greedy", "0.6b": "cfg2_0.6b_greedy",
                  "1.7b": "cfg4_1.7b_greedy"}


def make_hooks(spec: str) -> str:
    """The reference's Talker-prefill and CodePredictor parity fixtures
    (qwen3_tts_reference.py:487-523, 629-676; talker-prefill-parity.rs, code-predictor-parity.rs),
    same array names, from the float64 oracle on the synthetic model of `spec`."""
    from oracle.sampling import GREEDY
    w = WORKLOADS[HOOK_WORKLOADS[spec]]
    t0 = time.time()
    model = synth.SyntheticModel.build(w.spec, w.weight_seed)
    inputs = w.inputs(model)
    o = Oracle(model.tensors, model.config(), max_cache_steps=w.max_cache_steps, dtype=np.float64)
    P = inputs.prefill_steps
    logits = o.prefill(inputs.prefill)
    last_hidden = o.hidden.copy()
    first_semantic, margin0 = o.talker_select(logits, None, 1.0, GREEDY, None)
    prefix = o.prepare_code_predictor_prefix(first_semantic)
    first_acoustic, emb_sum, _, cp_m = o.code_predictor(prefix)
    step_input = o.build_step_input(first_semantic, emb_sum, inputs.trailing_text[0])
    next_logits = o.decode(step_input, P)
    next_semantic, margin1 = o.talker_select(next_logits, None, 1.0, GREEDY, None)
    th = deterministic_hidden(o.t_dims.hidden, 17.0, 15.0)
    se = deterministic_hidden(o.t_dims.hidden, 23.0, 11.0)
    ac_tokens, ac_sum, _, ac_m = o.code_predictor(np.stack([th, se]).astype(np.float64))
    path = os.path.join(HERE, f"hooks_{spec}.npz")
    meta = dict(spec=spec, weight_seed=w.weight_seed, checksum=model.checksum(), workload=w.name,
                prefill_steps=P, oracle_dtype="float64", seconds=round(time.time() - t0, 1))
    np.savez_compressed(
        path, meta=np.array(json.dumps(meta)), prefill=inputs.prefill.astype(np.float32),
        last_hidden=last_hidden.astype(np.float32), logits=logits.astype(np.float32),
        first_semantic=np.array([first_semantic]), first_acoustic=np.asarray(first_acoustic),
        first_step_input=step_input.astype(np.float32), forward_next_logits=next_logits.astype(np.float32),
        next_semantic=np.array([next_semantic]), talker_margins=np.array([margin0, margin1]),
        first_cp_margins=np.asarray(cp_m), talker_hidden=th, semantic_embed=se,
        acoustic_tokens=np.asarray(ac_tokens), embedding_sum=ac_sum.astype(np.float32),
        acoustic_margins=np.asarray(ac_m))
    print(f"hooks {spec}: {meta['seconds']} s -> {path}", flush=True)
    return path


def make_multi(name: str) -> str:
    w = MULTI_WORKLOADS[name]
    t0 = time.time()
    model = synth.SyntheticModel.build(w.spec, w.weight_seed)
    inputs = w.inputs(model)
    oracle = Oracle(model.tensors, model.config(), max_cache_steps=w.max_cache_steps, dtype=np.float64)
    arrays, frames, eos = {}, [], []
    for j, (inp, kw) in enumerate(zip(inputs, w.options_kwargs())):
        tr = oracle.rollout(inp.prefill, inp.trailing_text, inp.tts_pad_embed, GenerateOptions(**kw))
        arrays[f"codes_{j}"] = tr.codes
        arrays[f"talker_margins_{j}"] = tr.talker_margins
        arrays[f"cp_margins_{j}"] = tr.cp_margins
        arrays[f"talker_logits_{j}"] = tr.talker_logits[:MULTI_LOGIT_ROWS].astype(np.float32)
        frames.append(tr.frames)
        eos.append(bool(tr.ended_by_eos))
        print(f"  stream {j}: P={inp.prefill_steps} frames={tr.frames} ({time.time() - t0:.0f} s)", flush=True)
    meta = dict(workload=name, spec=w.spec, weight_seed=w.weight_seed, checksum=model.checksum(),
                streams=w.streams, prefill_steps=[int(i.prefill_steps) for i in inputs], frames=frames,
                ended_by_eos=eos, options=w.options_kwargs(), max_cache_steps=w.max_cache_steps,
                oracle_dtype="float64", seconds=round(time.time() - t0, 1))
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(path, meta=np.array(json.dumps(meta)), **arrays)
    print(f"{name}: {sum(frames)} frames over {w.streams} streams, {meta['seconds']} s -> {path}", flush=True)
    return path


if __name__ == "__main__":
    names = sys.argv[1:] or (list(WORKLOADS) + list(MULTI_WORKLOADS) +
                             [f"hooks_{s}" for s in HOOK_WORKLOADS])
    for n in names:
        if n.startswith("hooks_"):
            make_hooks(n[len("hooks_"):])
        elif n in MULTI_WORKLOADS:
            make_multi(n)
        else:
            make(n)
