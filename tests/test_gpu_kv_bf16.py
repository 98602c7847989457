"""The bf16 KV cache ("an LDS-staged bf16 KV cache") at the BASELINE
shapes, bounded against the oracle's bf16-KV model.

With a bf16 cache the GPU and a float64/float32 oracle round some K/V elements to
neighbouring bf16 values (their fp32 inputs differ in the last bits), so greedy codes can
part from the fp32-cache fixtures at a near tie and are not compared with them.  Instead
each run's own codes are fed to the oracle (float32, ``kv_bf16=True``: K and V rounded to
bf16 at the store) as forced tokens, and for every step of that history:

* the GPU's Talker logits (traced runs) are within 2e-2 max-abs of the oracle's, and so are
  the CodePredictor logits;
* every token the GPU chose is the oracle's greedy choice, or one whose oracle logit lies
  within 2 x 2e-2 of the oracle's maximum (a choice logits within the bound could make).

Reference: the fp32 cache of src/model/decode.rs:1897-1906, which this option narrows.
"""
import numpy as np
import pytest

from oracle.model import GenerateOptions as OracleOptions
from oracle.model import Oracle
from oracle.sampling import suppress
from q3t import engine as E
from q3t.workloads import MULTI_WORKLOADS, WORKLOADS

from parity import LOGIT_TOL

pytestmark = pytest.mark.gpu

BAND = 2 * LOGIT_TOL


_ORACLES = {}


def forced_oracle(model, inputs, codes, cap, frames):
    """Float32 bf16-KV oracle rollout teacher-forced to `codes` ([frames, 16]).  One oracle per
    (model, capacity) is kept for the module (a rollout resets its caches)."""
    key = (model.checksum(), cap)
    if key not in _ORACLES:
        _ORACLES.clear()
        _ORACLES[key] = Oracle(model.tensors, model.config(), max_cache_steps=cap, dtype=np.float32,
                               kv_bf16=True)
    o = _ORACLES[key]
    tr = o.rollout(inputs.prefill, inputs.trailing_text, inputs.tts_pad_embed, OracleOptions.greedy(frames),
                   keep_cp_logits=frames, forced_codes=codes[:frames])
    return o, tr


def token_slack(o, tr, codes, frames):
    """Largest (oracle max - oracle logit of the GPU's token) over every Talker and
    CodePredictor choice of the first `frames` frames (greedy: no penalty, suppression on
    the Talker head)."""
    worst = 0.0
    for f in range(frames):
        lt = suppress(tr.talker_logits[f].astype(np.float64), o.codec_eos)
        worst = max(worst, float(lt.max() - lt[codes[f, 0]]))
        lc = np.asarray(tr.cp_logits[f], dtype=np.float64)
        worst = max(worst, float((lc.max(1) - lc[np.arange(lc.shape[0]), codes[f, 1:]]).max()))
    return worst


def test_cfg2_bf16_kv_bounded_by_oracle(models):
    """Config 2 (0.6B, 240 frames, KV 256) on the bf16 cache: all 240 Talker rows and every
    frame's 15 CodePredictor rows."""
    name = "cfg2_0.6b_greedy"
    w = WORKLOADS[name]
    model, d = models.get(w.spec, w.weight_seed)
    inputs = w.inputs(model)
    print(f"[gpu] {name} kv_bf16 traced", flush=True)
    with E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=w.max_cache_steps, kv_bf16=True)) as eng:
        eng.set_trace(True)
        with eng.start_stream(inputs, E.GenerateOptions(**w.options_kwargs())) as st:
            while st.next_codes_chunk(w.chunk_frames) is not None:
                pass
            logits, cp_logits = st.talker_logits(), st.cp_logits()
            codes = st.finish_codes().codes
    frames = len(codes)
    assert frames == w.frames
    o, tr = forced_oracle(model, inputs, codes, w.max_cache_steps, frames)
    t_err = float(np.abs(logits[:frames] - tr.talker_logits[:frames]).max())
    c_err = float(np.abs(cp_logits[:frames] - np.asarray(tr.cp_logits)).max())
    slack = token_slack(o, tr, codes, frames)
    print(f"{name} bf16 KV: {frames} frames, Talker logit err {t_err:.2e}, CodePredictor logit err {c_err:.2e}, "
          f"token slack {slack:.2e}")
    assert t_err <= LOGIT_TOL and c_err <= LOGIT_TOL
    assert slack <= BAND


CFG5_FRAMES = 24   # frames of every stream checked against the oracle (all frames are generated)


def _cfg5(models, trace):
    name = "cfg5_0.6b_multistream"
    w = MULTI_WORKLOADS[name]
    model, d = models.get(w.spec, w.weight_seed)
    inputs = w.inputs(model)
    opts = [E.GenerateOptions(**kw) for kw in w.options_kwargs()]
    print(f"[gpu] {name} kv_bf16 trace={trace}", flush=True)
    with E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=w.max_cache_steps, max_streams=w.streams,
                                           kv_bf16=True)) as eng:
        eng.set_trace(trace)
        streams = eng.start_streams(inputs, opts, E.StreamOptions(text_lookahead_tokens=1 << 30))
        live = list(streams)
        while live:
            chunks = eng.next_codes_chunks(live, w.chunk_frames)
            live = [s for s, c in zip(live, chunks) if c is not None]
        logits = [s.talker_logits() for s in streams] if trace else None
        cp = [s.cp_logits() for s in streams] if trace else None
        codes = [s.finish_codes().codes for s in streams]
    return w, model, inputs, codes, logits, cp


def test_cfg5_bf16_kv_timed_path_tokens_bounded(models):
    """Config 5 on the bf16 cache, untraced: the path bench.py times for its bf16-KV line
    (greedy hand-off through argmax keys and layer-0 tables).  Every stream's first
    CFG5_FRAMES frames: each token within the band of the oracle's greedy choice."""
    w, model, inputs, codes, _, _ = _cfg5(models, trace=False)
    worst = 0.0
    for j in range(w.streams):
        n = min(CFG5_FRAMES, len(codes[j]))
        o, tr = forced_oracle(model, inputs[j], codes[j], w.max_cache_steps, n)
        s = token_slack(o, tr, codes[j], n)
        worst = max(worst, s)
        print(f"stream {j}: P={inputs[j].prefill_steps} token slack {s:.2e}", flush=True)
        assert s <= BAND
    print(f"cfg5 bf16 KV untraced: worst token slack {worst:.2e} (band {BAND})")


def test_cfg5_bf16_kv_logits_bounded(models):
    """Config 5 on the bf16 cache, traced: every stream's Talker and CodePredictor logits over
    its first CFG5_FRAMES frames within 2e-2 of the oracle's on the same tokens."""
    w, model, inputs, codes, logits, cp = _cfg5(models, trace=True)
    for j in range(w.streams):
        n = min(CFG5_FRAMES, len(codes[j]))
        o, tr = forced_oracle(model, inputs[j], codes[j], w.max_cache_steps, n)
        t_err = float(np.abs(logits[j][:n] - tr.talker_logits[:n]).max())
        c_err = float(np.abs(cp[j][:n] - np.asarray(tr.cp_logits)).max())
        s = token_slack(o, tr, codes[j], n)
        print(f"stream {j}: Talker logit err {t_err:.2e}, CodePredictor {c_err:.2e}, token slack {s:.2e}",
              flush=True)
        assert t_err <= LOGIT_TOL and c_err <= LOGIT_TOL and s <= BAND
