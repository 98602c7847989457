"""Benchmark: codec frames/s and RTF of the Qwen3-TTS token loop on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload cfg2_0.6b_greedy]

A step is one full generation of the workload (BASELINE config 2 by default: 0.6B shape,
bf16 weights, greedy, batch 1, 64-token prompt, 240 frames pulled in chunks of 6, KV
capacity 256): Talker prefill, then every frame's CodePredictor groups and Talker step.
Inputs (weights, prefill rows) are resident in HBM before the timed region; the timed
region is K steps bracketed by device synchronisation.  RTF = seconds / (frames * 0.080).

Prints one JSON line.  Besides the contract fields it carries:
  rtf, frame_ms                  per-frame latency view of the same run
  frame_algorithmic_GBps         bytes one frame must move (weights + KV) / frame time
  roofline                       the dominant kernel, timed live with HIP events
  per_step                       Talker-step and CodePredictor-pass rooflines (phases timed as graphs)
  kv_bf16, per_step_kv_bf16      the headline workload again on the bf16 KV cache: frames/s, per-step
                                 rooflines (bf16 KV bytes), leading frames equal to the fp32 run's codes
  multistream                    BASELINE config 5 (16 streams together) on the same model, with
                                 the batched frame's roofline
  multistream_kv_bf16            the same on the bf16 KV cache
  sampled                        BASELINE config 3 (sampling on both heads) on the same model
  cfg4                           BASELINE config 4 (1.7B, 480 frames, KV 512), one generation
  first_audio                    time from start_stream to the first audio chunk
  cpu_baseline                   the float32 CPU oracle on BASELINE config 1 (1 warmup + 3 x 40 frames)
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "qwen3-tts-hip_amd"))

HBM_PEAK_GBPS = 8000.0
FRAME_SECONDS = 0.080


def step_bytes(spec, kv_elem: int):
    """Algorithmic bytes of one Talker step (stack + codec head + final norm, bf16) and of one
    CodePredictor pass (stack + one LM head + final norm (+ projection)), without KV, and the
    KV bytes of one cached position of each stack (K and V, all layers)."""
    t, c = spec.talker, spec.code_predictor

    def stack_params(s):
        # per layer: q/k/v, o, gate/up and down matrices, plus the four norm gains (input,
        # post-attention, q head, k head)
        q, kv = s.q_heads * s.head_dim, s.kv_heads * s.head_dim
        return s.layers * ((q + 2 * kv) * s.hidden + s.hidden * q + 3 * s.intermediate * s.hidden +
                           2 * s.hidden + 2 * s.head_dim)

    talker = 2 * (stack_params(t) + t.vocab * t.hidden + t.hidden)
    proj = c.hidden * t.hidden if spec.has_projection else 0
    cp_pass = 2 * (stack_params(c) + c.vocab * c.hidden + c.hidden + proj)
    kv_t = t.layers * 2 * t.kv_heads * t.head_dim * kv_elem
    kv_c = c.layers * 2 * c.kv_heads * c.head_dim * kv_elem
    return talker, cp_pass, kv_t, kv_c


def frame_bytes(spec, active_steps_mean: float, kv_elem: int) -> float:
    """Algorithmic bytes of one frame: every bf16 weight the frame reads once per pass (the
    Talker step, then 15 CodePredictor passes), plus the KV cache rows attention reads and
    writes: the Talker's at the mean active length, the CodePredictor's 1 .. 16 rows."""
    talker, cp_pass, kv_t, kv_c = step_bytes(spec, kv_elem)
    groups = spec.num_code_groups - 1
    kv = kv_t * active_steps_mean + kv_c * sum(range(1, spec.num_code_groups + 1))
    return talker + groups * cp_pass + kv


def batched_bytes(spec, prefill_steps, frames, kv_elem: int) -> int:
    """Algorithmic bytes of a multi-stream generation run as batched frames: every weight once
    per batched frame (as many batched frames as the longest stream has frames), plus each
    live stream's KV rows.  In batched frame f a stream with more than f frames is live (no
    EOS); at prefill P it runs the Talker step after frame f at position P + f, which reads
    P + f + 1 rows and writes one (none after its last frame), and its frame's CodePredictor
    passes.  kv_elem: bytes per cached element (4 fp32, 2 bf16)."""
    talker_w, cp_w, kv_t, kv_c = step_bytes(spec, kv_elem)
    groups = spec.num_code_groups - 1
    weights = talker_w + groups * cp_w
    cp_kv = kv_c * (sum(range(2, groups + 2)) + 2)
    kv = sum(sum(kv_t * (p + f + 2) for f in range(fr - 1)) + fr * cp_kv for p, fr in zip(prefill_steps, frames))
    return int(max(frames) * weights + kv)


def per_step(st, spec, prefill_steps: int, chunk: int, kv_elem: int) -> dict:
    """Runs the stream `st` to its end with both phases of every frame timed on the GPU
    (q3t_debug_phase_times: the CodePredictor and the Talker step each replayed as its own
    graph) and returns the per-step rooflines: Talker step = bytes / time over the frames that
    run a Talker step (all but the last), CodePredictor pass = the frame's 15 passes / 15."""
    import numpy as np
    cp, tk = [], []
    while True:
        c, a, b = st.next_codes_chunk_timed(chunk)
        cp += list(a)
        tk += list(b)
        if c is None:
            break
    F = len(cp)
    talker_w, cp_w, kv_t, kv_c = step_bytes(spec, kv_elem)
    groups = spec.num_code_groups - 1
    # frame f: the Talker attention at position P + f reads P + f + 1 rows and writes one; the
    # CodePredictor's pass at position p (1 .. groups) reads p + 1 rows (the prefix pass 2)
    t_bytes = [talker_w + kv_t * (prefill_steps + f + 2) for f in range(F - 1)]
    c_bytes = groups * cp_w + kv_c * (sum(range(2, groups + 2)) + 2)
    t_us = np.asarray(tk[:F - 1], np.float64)
    c_us = np.asarray(cp, np.float64)
    t_gbps = sum(t_bytes) / (t_us.sum() * 1e-6) / 1e9
    c_gbps = F * c_bytes / (c_us.sum() * 1e-6) / 1e9
    return {"frames": F, "timing": "each phase replayed as its own graph, hipEvents between them",
            "talker_step_us": round(float(t_us.mean()), 3), "talker_step_us_median": round(float(np.median(t_us)), 3),
            "talker_step_bytes_mean": int(np.mean(t_bytes)), "talker_step_GBps": round(t_gbps, 1),
            "talker_step_frac": round(t_gbps / HBM_PEAK_GBPS, 4),
            "cp_pass_us": round(float(c_us.mean()) / groups, 3), "cp_pass_bytes": int(c_bytes / groups),
            "cp_pass_GBps": round(c_gbps, 1), "cp_pass_frac": round(c_gbps / HBM_PEAK_GBPS, 4),
            "frame_us_sum_of_phases": round(float(c_us.mean() + t_us.mean()), 3)}


def measured_traffic(workload: str, kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC summary of this
    workload (FETCH_SIZE and WRITE_SIZE, each scaled by its copy-kernel calibration)."""
    path = os.path.join(ROOT, "profiles", f"pmc_traffic_{workload.split('_', 1)[1]}.json")
    path = path if os.path.exists(path) else os.path.join(ROOT, "profiles", "pmc_traffic_cfg2_0.6b.json")
    try:
        d = json.load(open(path))
    except (OSError, ValueError):
        return None
    if d.get("workload") != workload or kernel not in d.get("kernels", {}):
        return None
    k, c = d["kernels"][kernel], d["calibration"]
    return int(1024 * (k["fetch_kib"] * c["fetch_scale"] + k["write_kib"] * c["write_scale"]))


def cpu_baseline(runs: int = 3) -> dict:
    """BASELINE config 1 on the host CPU, the reported CPU baseline: the float32 oracle,
    0.6B shape, 32-token prompt (non-streaming, P = 41), greedy, 40 frames; one warmup
    generation, then `runs` measured ones.  frames/s and ms/frame count the frames only (the
    prefill is reported beside them), as the reference's GenerationProfile splits them."""
    import numpy as np
    from threadpoolctl import threadpool_info

    sys.path.insert(0, ROOT)
    from oracle.model import GenerateOptions as OO
    from oracle.model import Oracle
    from q3t import synth
    from q3t.workloads import WORKLOADS

    w = WORKLOADS["cfg1_cpu_0.6b"]
    model = synth.SyntheticModel.build(w.spec, w.weight_seed)
    inputs = w.inputs(model)
    o = Oracle(model.tensors, model.config(), max_cache_steps=w.max_cache_steps, dtype=np.float32)
    del model
    opts = OO.greedy(w.frames)

    def one():
        t = {}
        tr = o.rollout(inputs.prefill, inputs.trailing_text, inputs.tts_pad_embed, opts, timings=t)
        return tr.frames, t["prefill_s"], t["frames_s"]

    one()
    res = [one() for _ in range(runs)]
    frames = sum(r[0] for r in res)
    frames_s = sum(r[2] for r in res)
    prefill_s = sum(r[1] for r in res) / runs
    blas = [i for i in threadpool_info() if i.get("user_api") == "blas"]
    threads = int(blas[0]["num_threads"]) if blas else 1
    try:
        model_name = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name"))
    except Exception:
        model_name = "unknown"
    return {"value": round(frames / frames_s, 3), "unit": "frames/s", "cores": threads, "kind": "port",
            "ms_per_frame": round(1000 * frames_s / frames, 2), "rtf": round(frames_s / (frames * FRAME_SECONDS), 4),
            "prefill_ms": round(1000 * prefill_s, 1), "runs": runs, "warmup": 1, "frames_per_run": w.frames,
            "os_cpu_count": os.cpu_count(), "blas_threads": threads, "cpu_model": model_name,
            "sample": f"config 1: 0.6B float32 oracle (numpy/BLAS, {threads} threads), 32-token prompt (P=41), "
                      f"greedy, 1 warmup + {runs} x {w.frames} frames; frames timed without the prefill"}


def multistream(eng_cls, model_dir: str, name: str, steps: int, warmup: int, use_graph: bool,
                frames_cap: int = 0, kv_bf16: bool = False) -> dict:
    """BASELINE config 5 on the same model: every stream started together (one prefill over
    all prompts), then chunks pulled for all live streams at once until each has ended.
    A step is one such generation; value = frames of all streams / seconds.  `roofline`: the
    algorithmic bytes of the batched frames (every weight once per batched frame, plus each
    live stream's KV rows) over the step time without the prefill."""
    from q3t import engine as E
    from q3t import synth
    from q3t.workloads import MULTI_WORKLOADS

    w = MULTI_WORKLOADS[name]
    model = synth.SyntheticModel.build(w.spec, w.weight_seed)
    inputs = w.inputs(model)
    del model
    opts = [E.GenerateOptions(**kw) for kw in w.options_kwargs()]
    if frames_cap > 0:  # profiling runs: the same prefill, fewer frames
        opts = [E.GenerateOptions(**{**kw, "max_frames": min(kw["max_frames"], frames_cap)})
                for kw in w.options_kwargs()]
    eng = eng_cls(model_dir, E.EngineOptions(max_cache_steps=w.max_cache_steps, max_streams=w.streams,
                                             use_graph=use_graph, kv_bf16=kv_bf16))
    lk = E.StreamOptions(text_lookahead_tokens=1 << 30)

    def one():
        t0 = time.perf_counter()
        streams = eng.start_streams(inputs, opts, lk)
        t1 = time.perf_counter()
        live, n = list(streams), 0
        while live:
            chunks = eng.next_codes_chunks(live, w.chunk_frames)
            n += sum(c.frames for c in chunks if c is not None)
            live = [s for s, c in zip(live, chunks) if c is not None]
        for s in streams:
            s.close()
        return n, t1 - t0

    for _ in range(warmup):
        one()
    eng.synchronize()
    t0 = time.perf_counter()
    frames, prefill_s = 0, 0.0
    for _ in range(steps):
        n, p = one()
        frames += n
        prefill_s += p
    eng.synchronize()
    el = time.perf_counter() - t0
    eng.close()
    lengths, budgets, _ = w.plan()
    if frames_cap > 0:
        budgets = [min(f, frames_cap) for f in budgets]
    spec = synth.SPECS[w.spec]
    n_batched = max(budgets)
    alg_bytes = batched_bytes(spec, [9 + n for n in lengths], budgets, 2 if kv_bf16 else 4)
    decode_s = (el - prefill_s) / steps
    gbps = alg_bytes / decode_s / 1e9
    # the per-frame algorithmic-byte definition counts KV rows at bf16 width whatever the cache type
    alg_bytes_8d = batched_bytes(spec, [9 + n for n in lengths], budgets, 2)
    gbps_8d = alg_bytes_8d / decode_s / 1e9
    return {"workload": name, "streams": w.streams, "value": round(frames / el, 2), "unit": "frames/s (all streams)",
            "steps": steps, "warmup": warmup, "ms_per_step": round(1000 * el / steps, 3),
            "frames_per_step": frames // steps, "prefill_rows": sum(9 + n for n in lengths),
            "prefill_ms": round(1000 * prefill_s / steps, 3), "kv_capacity": w.max_cache_steps,
            "kv_cache": "bf16" if kv_bf16 else "fp32",
            "rtf_per_stream": round(el / steps * w.streams / (frames / steps) / FRAME_SECONDS, 5),
            "decode_frames_per_s": round(frames / steps / decode_s, 2),
            "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": round(gbps / HBM_PEAK_GBPS, 4), "batched_frames": n_batched,
                         "algorithmic_bytes_per_step": int(alg_bytes),
                         "batched_frame_ms": round(1000 * decode_s / n_batched, 4),
                         "kv_bytes_counted": "bf16" if kv_bf16 else "fp32",
                         "frac_bf16_kv_bytes": round(gbps_8d / HBM_PEAK_GBPS, 4),
                         "note": "every weight once per batched frame + each live stream's KV rows at the "
                                 "cache's own width (frac) or at bf16 width, the width of the per-frame "
                                 "byte definition (frac_bf16_kv_bytes), over the step time without the "
                                 "prefill"}}


def big_model_line(E, synth, w, use_graph: bool) -> dict:
    """the 1.7B-shaped model (Talker hidden 2048, the 2048 -> 1024
    projection into the CodePredictor), greedy, 128-token prompt, 480 frames, KV 512; one
    warmup generation, then one timed."""
    import shutil
    model = synth.SyntheticModel.build(w.spec, w.weight_seed)
    inputs = w.inputs(model)
    tmp = tempfile.mkdtemp(prefix="q3t_bench4_")
    model.write(tmp)
    spec = model.spec
    del model
    try:
        eng = E.HipTtsEngine(tmp, E.EngineOptions(max_cache_steps=w.max_cache_steps, use_graph=use_graph))
        opts = E.GenerateOptions(**w.options_kwargs())

        def one():
            with eng.start_stream(inputs, opts) as st:
                n = 0
                while (c := st.next_codes_chunk(w.chunk_frames)) is not None:
                    n += c.frames
            return n
        one()
        eng.synchronize()
        t0 = time.perf_counter()
        n = one()
        eng.synchronize()
        el = time.perf_counter() - t0
        with eng.start_stream(inputs, opts) as st:
            steps = per_step(st, spec, inputs.prefill_steps, w.chunk_frames, 4)
        eng.close()
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    fb = frame_bytes(spec, inputs.prefill_steps + (n - 1) / 2.0, 4)
    return {"workload": w.name, "frames": n, "value": round(n / el, 2), "unit": "frames/s",
            "rtf": round(el / (n * FRAME_SECONDS), 5), "frame_ms": round(1000 * el / n, 4),
            "frame_algorithmic_GBps": round(fb / (el / n) / 1e9, 1), "prefill_steps": inputs.prefill_steps,
            "kv_capacity": w.max_cache_steps, "per_step": steps}


def batch1_kv_bf16(E, model_dir, w, inputs, opts, spec, P, args, fp32_codes) -> dict:
    """The headline workload on a bf16 KV cache (engine option kv_dtype = 1): frames/s over the
    same steps after one warmup, the per-step rooflines with bf16 KV bytes, and how many
    leading frames equal the fp32-cache run's codes (the bf16 cache rounds K/V once at the
    store, so greedy codes part from the fp32 run after some frames)."""
    import numpy as np
    eng = E.HipTtsEngine(model_dir, E.EngineOptions(max_cache_steps=w.max_cache_steps, use_graph=not args.eager,
                                                    kv_bf16=True))
    codes = []

    def one():
        with eng.start_stream(inputs, opts) as st:
            got = []
            while (c := st.next_codes_chunk(w.chunk_frames)) is not None:
                got.append(c.codes)
        codes[:] = got
        return sum(g.shape[0] for g in got)
    for _ in range(args.warmup):
        one()
    eng.synchronize()
    t0 = time.perf_counter()
    frames = 0
    for _ in range(args.steps):
        frames += one()
    eng.synchronize()
    el = time.perf_counter() - t0
    with eng.start_stream(inputs, opts) as st:
        steps_line = per_step(st, spec, P, w.chunk_frames, 2)
    eng.close()
    a, b = np.concatenate(codes), np.concatenate(fp32_codes)
    n = min(len(a), len(b))
    same = np.all(a[:n] == b[:n], axis=1)
    lead = int(n if same.all() else np.argmin(same))
    frame_s = el / frames
    fb = frame_bytes(spec, P + (frames / max(args.steps, 1) - 1) / 2.0, 2)
    return {"kv_cache": "bf16", "value": round(frames / el, 2), "unit": "frames/s", "steps": args.steps,
            "rtf": round(frame_s / FRAME_SECONDS, 5), "frame_ms": round(1000 * frame_s, 4),
            "frame_algorithmic_GBps": round(fb / frame_s / 1e9, 1),
            "frames_equal_to_fp32_cache_codes": lead, "frames_per_step": frames // max(args.steps, 1),
            "per_step_kv_bf16": steps_line}


def copy_calibration(nbytes: int = 256 << 20) -> int:
    """One device-to-device copy of `nbytes` through the HIP runtime (its copy kernel), the
    known-size reference for scaling rocprofv3's FETCH_SIZE / WRITE_SIZE counters.  No torch
    import, no engine: the copy is the only kernel of the process."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    n = ctypes.c_size_t(nbytes)
    for rc in (hip.hipMalloc(ctypes.byref(a), n), hip.hipMalloc(ctypes.byref(b), n), hip.hipMemset(a, 1, n),
               hip.hipMemcpy(b, a, n, 3), hip.hipDeviceSynchronize()):  # 3 = hipMemcpyDeviceToDevice
        if rc != 0:
            print(json.dumps({"copy_calibration": "failed", "hip_error": rc}))
            return 1
    hip.hipFree(a)
    hip.hipFree(b)
    print(json.dumps({"copy_calibration_bytes": nbytes, "kernel": "the runtime's device-to-device copy"}))
    return 0


def codec_decode_only(E, synth, frames: int, steps: int) -> int:
    """decode_codes of `frames` random frames, `steps` timed calls after one warmup (the codec
    decoder alone: profiling runs)."""
    import numpy as np
    import shutil
    tmp = tempfile.mkdtemp(prefix="q3t_codec_")
    synth.SyntheticModel.build("tiny", 0).write(tmp)
    synth.write_codec(tmp, 0)
    eng = E.HipTtsEngine(tmp, E.EngineOptions(max_cache_steps=64))
    codes = np.random.default_rng(0).integers(0, 2048, (frames, 16)).astype(np.int32)
    eng.decode_codes(codes)
    t0 = time.perf_counter()
    for _ in range(steps):
        eng.decode_codes(codes)
    dt = (time.perf_counter() - t0) / steps
    eng.close()
    shutil.rmtree(tmp, ignore_errors=True)
    print(json.dumps({"codec_decode_frames": frames, "decode_ms": round(1000 * dt, 3),
                      "decode_rtf": round(dt / (frames * FRAME_SECONDS), 5), "steps": steps}))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--workload", default="cfg2_0.6b_greedy")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-runs", type=int, default=3, help="measured CPU-baseline generations (after 1 warmup)")
    ap.add_argument("--eager", action="store_true", help="launch every kernel from the host (no graph)")
    ap.add_argument("--kv-bf16", action="store_true")
    ap.add_argument("--frames", type=int, default=0, help="override the workload's frame count (profiling runs)")
    ap.add_argument("--multistream", default="cfg5_0.6b_multistream",
                    help="multi-stream workload reported beside the headline line ('' to skip)")
    ap.add_argument("--multistream-only", action="store_true", help="run only the multi-stream workload")
    ap.add_argument("--codec-decode", type=int, default=0, metavar="FRAMES",
                    help="only time decode_codes of FRAMES random frames (tiny model + codec checkpoint) and exit")
    ap.add_argument("--no-codec", action="store_true",
                    help="skip the codec-decoder timing (and the speech-tokenizer checkpoint it needs)")
    ap.add_argument("--no-text-prep", action="store_true",
                    help="skip the device prompt-preparation timing (and the text-embedding table it needs)")
    ap.add_argument("--no-cfg4", action="store_true", help="skip the 1.7B (config 4) generation")
    ap.add_argument("--no-sampled", action="store_true", help="skip the sampled (config 3) generation")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the dominant kernel's eager per-dispatch timing (no graphs: the command rocprofv3 "
                         "traces for profiles/) and exit")
    ap.add_argument("--no-multistream-bf16", action="store_true",
                    help="skip the config-5 run on the bf16 KV cache")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy 256 MiB device to device (the PMC traffic counters' calibration) and exit")
    ap.add_argument("--no-kv-bf16", action="store_true",
                    help="skip the headline workload's second run on the bf16 KV cache")
    ap.add_argument("--kernel-classes", action="store_true",
                    help="graph-time every kernel class of q3t_bench_kernel on the workload's model and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        return copy_calibration()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "streams shard across GPUs by data parallelism with no exchange step, so N GPUs = N x one GPU.",
              file=sys.stderr)
        return 2

    import numpy as np
    from q3t import engine as E
    from q3t import synth
    from q3t.workloads import WORKLOADS

    if args.codec_decode > 0:
        return codec_decode_only(E, synth, args.codec_decode, max(args.steps, 1))

    w = WORKLOADS[args.workload]
    if args.frames > 0:
        import dataclasses
        w = dataclasses.replace(w, frames=min(args.frames, w.frames))
    model = synth.SyntheticModel.build(w.spec, w.weight_seed)
    inputs = w.inputs(model)
    tmp = tempfile.mkdtemp(prefix="q3t_bench_")
    with_text = not (args.no_text_prep or args.kernel_classes or args.multistream_only)
    model.write(tmp, text_embedding=with_text)
    with_codec = not (args.no_codec or args.kernel_classes or args.multistream_only)
    if with_codec:
        synth.write_codec(tmp, 0)
    spec = model.spec
    w3 = WORKLOADS["cfg3_0.6b_sampled"]
    inputs3 = (w3.inputs(model) if (w3.spec, w3.weight_seed) == (w.spec, w.weight_seed) and args.frames == 0
               and not args.no_sampled else None)
    host_prep = None
    if with_text:
        from q3t import textprep
        tp = textprep.TextPrep(model)
        t0 = time.perf_counter()
        look = (1 << 30) if w.lookahead is None else w.lookahead
        for _ in range(3):
            tp.prepare(w.prompt(), text_lookahead_tokens=look)
        host_prep = (time.perf_counter() - t0) / 3
    del model
    if args.roofline_only:
        eng = E.HipTtsEngine(tmp, E.EngineOptions(max_cache_steps=w.max_cache_steps))
        eng.bench_kernel_timed(2, 103)
        us, b = eng.bench_kernel_timed(2, 1030)
        eng.close()
        import shutil
        shutil.rmtree(tmp, ignore_errors=True)
        gbps = b / (us * 1e-6) / 1e9
        print(json.dumps({"kernel": E.HipTtsEngine.KERNELS[2], "avg_launch_us": round(us, 3),
                          "algorithmic_bytes_per_launch": int(b), "achieved": round(gbps, 1),
                          "frac": round(gbps / HBM_PEAK_GBPS, 4),
                          "timing": "eager launches, per-dispatch start/stop events (1030 + 103 warm + 1133 warm)"}))
        return 0
    if args.kernel_classes:
        eng = E.HipTtsEngine(tmp, E.EngineOptions(max_cache_steps=w.max_cache_steps))
        for k, name in E.HipTtsEngine.KERNELS.items():
            us, b = eng.bench_kernel(k, 1020)
            print(json.dumps({"class": k, "kernel": name, "us_per_launch": round(us, 3),
                              "algorithmic_bytes": int(b), "GBps": round(b / us / 1e3, 1)}))
        eng.close()
        import shutil
        shutil.rmtree(tmp, ignore_errors=True)
        return 0
    if args.multistream_only:
        print(json.dumps(multistream(E.HipTtsEngine, tmp, args.multistream, args.steps, args.warmup,
                                     not args.eager, args.frames)))
        import shutil
        shutil.rmtree(tmp, ignore_errors=True)
        return 0
    eng = E.HipTtsEngine(tmp, E.EngineOptions(max_cache_steps=w.max_cache_steps, use_graph=not args.eager,
                                              kv_bf16=args.kv_bf16))
    opts = E.GenerateOptions(**w.options_kwargs())

    last_codes = []

    def one_step():
        st = eng.start_stream(inputs, opts)
        n = 0
        got = []
        while True:
            c = st.next_codes_chunk(w.chunk_frames)
            if c is None:
                break
            n += c.frames
            got.append(c.codes)
        st.close()
        last_codes[:] = got
        return n

    for _ in range(args.warmup):
        one_step()
    eng.synchronize()
    t0 = time.perf_counter()
    frames = 0
    for _ in range(args.steps):
        frames += one_step()
    eng.synchronize()
    elapsed = time.perf_counter() - t0

    P = inputs.prefill_steps
    per_gen = frames / max(args.steps, 1)
    active_mean = P + (per_gen - 1) / 2.0
    fb = frame_bytes(spec, active_mean, 2 if args.kv_bf16 else 4)
    frame_s = elapsed / frames
    # --eager captures no graph anywhere (the form profiled under rocprofv3's kernel tracer)
    roofline = eng.dominant_kernel_roofline(HBM_PEAK_GBPS, graph=not args.eager)
    roofline["traffic"] = measured_traffic(w.name, roofline["kernel"])
    with eng.start_stream(inputs, opts) as st_steps:
        steps_line = per_step(st_steps, spec, P, w.chunk_frames, 2 if args.kv_bf16 else 4)
    kv_bf16_line = None
    if not args.kv_bf16 and not args.no_kv_bf16:
        kv_bf16_line = batch1_kv_bf16(E, tmp, w, inputs, opts, spec, P, args, last_codes)
    text_prep = None
    if with_text:
        # Prompt preparation of the same prompt on the device (q3t_prepare_text, host copies
        # and workspace allocation included), against the package's numpy preparation.
        ids = w.prompt()
        dev = eng.prepare_text(ids, text_lookahead_tokens=look)
        assert np.abs(dev.prefill - inputs.prefill).max() < 1e-4
        t0 = time.perf_counter()
        for _ in range(20):
            eng.prepare_text(ids, text_lookahead_tokens=look)
        text_prep = {"content_ids": int(len(ids)), "rows_projected": int(len(ids)) + 11,
                     "device_ms": round(1000 * (time.perf_counter() - t0) / 20, 3),
                     "host_numpy_ms": round(1000 * host_prep, 3)}
    codec = None
    if with_codec and eng.has_codec:
        # Codec decoder on the generation's own codes: one decode of all frames
        # (generate / decode_codes) and the streaming window (a chunk plus 25 frames of left
        # context, next_audio_chunk), host copies included.
        codes = np.concatenate(last_codes)
        F = codes.shape[0]
        eng.decode_codes(codes)
        t0 = time.perf_counter()
        for _ in range(3):
            eng.decode_codes(codes)
        full_s = (time.perf_counter() - t0) / 3
        win = codes[:w.chunk_frames + 25]
        eng.decode_codes(win)
        t0 = time.perf_counter()
        for _ in range(10):
            eng.decode_codes(win)
        win_s = (time.perf_counter() - t0) / 10
        codec = {"frames": int(F), "decode_ms": round(1000 * full_s, 3),
                 "decode_rtf": round(full_s / (F * FRAME_SECONDS), 5),
                 "stream_window_frames": int(win.shape[0]), "stream_chunk_frames": w.chunk_frames,
                 "stream_window_ms": round(1000 * win_s, 3),
                 "stream_rtf": round(win_s / (w.chunk_frames * FRAME_SECONDS), 5)}
    sampled = None
    if inputs3 is not None:
        # BASELINE config 3 on the same weights: top-k 50 / top-p 1.0 / T 0.9 / repetition
        # penalty 1.05 on the Talker, sampling in every CodePredictor group (no token hand-off).
        o3 = E.GenerateOptions(**w3.options_kwargs())

        def one3():
            with eng.start_stream(inputs3, o3) as st3:
                n3 = 0
                while (c3 := st3.next_codes_chunk(w3.chunk_frames)) is not None:
                    n3 += c3.frames
            return n3
        one3()
        eng.synchronize()
        t0 = time.perf_counter()
        n3 = one3()
        eng.synchronize()
        el3 = time.perf_counter() - t0
        sampled = {"workload": w3.name, "frames": n3, "value": round(n3 / el3, 2), "unit": "frames/s",
                   "rtf": round(el3 / (n3 * FRAME_SECONDS), 5)}
    first_audio = None
    if with_codec and eng.has_codec:
        # start_stream (prefill + first token) through the first next_audio_chunk (chunk_frames
        # frames, decoded), host-prepared prompt rows.
        def first():
            t0 = time.perf_counter()
            with eng.start_stream(inputs, opts) as st:
                c = st.next_audio_chunk(w.chunk_frames)
            return time.perf_counter() - t0, c.frames
        first()
        ts = [first()[0] for _ in range(5)]
        first_audio = {"chunk_frames": w.chunk_frames, "ms": round(1000 * min(ts), 3),
                       "ms_median": round(1000 * sorted(ts)[2], 3)}
    eng.close()
    cfg4 = None
    if not args.no_cfg4 and w.name == "cfg2_0.6b_greedy" and args.frames == 0:
        cfg4 = big_model_line(E, synth, WORKLOADS["cfg4_1.7b_greedy"], not args.eager)
    multi = multi_bf16 = None
    if args.multistream and w.spec == "0.6b" and w.weight_seed == 0:
        multi = multistream(E.HipTtsEngine, tmp, args.multistream, max(1, min(args.steps, 2)), 1, not args.eager)
        if not args.no_multistream_bf16:
            multi_bf16 = multistream(E.HipTtsEngine, tmp, args.multistream, max(1, min(args.steps, 2)), 1,
                                     not args.eager, kv_bf16=True)
    import shutil
    shutil.rmtree(tmp, ignore_errors=True)

    out = {
        "metric": "codec frames/sec + RTF, 0.6B bs=1 greedy; decode HBM GB/s vs peak",
        "value": round(frames / elapsed, 2),
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1000 * elapsed / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init N(0,0.02) bf16 weights, seed 0; random prompt ids, seed 1)",
        "config": {"workload": w.name, "spec": w.spec, "batch": 1, "prompt_tokens": w.prompt_tokens,
                   "prefill_steps": P, "frames_per_step": per_gen, "chunk_frames": w.chunk_frames,
                   "kv_capacity": w.max_cache_steps, "greedy": not w.do_sample,
                   "graph": not args.eager, "kv_cache": "bf16" if args.kv_bf16 else "fp32"},
        "rtf": round(frame_s / FRAME_SECONDS, 5),
        "frame_ms": round(1000 * frame_s, 4),
        "frame_algorithmic_GBps": round(fb / frame_s / 1e9, 1),
        "frame_algorithmic_bytes": int(fb),
        "roofline": roofline,
        "per_step": steps_line,
    }
    if kv_bf16_line is not None:
        out["kv_bf16"] = kv_bf16_line
        out["per_step_kv_bf16"] = kv_bf16_line["per_step_kv_bf16"]
    if multi is not None:
        out["multistream"] = multi
    if multi_bf16 is not None:
        out["multistream_kv_bf16"] = multi_bf16
    if text_prep is not None:
        out["text_prep"] = text_prep
    if codec is not None:
        out["codec"] = codec
    if sampled is not None:
        out["sampled"] = sampled
    if cfg4 is not None:
        out["cfg4"] = cfg4
    if first_audio is not None:
        out["first_audio"] = first_audio
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.cpu_runs)
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
