"""CPU restatement of the Qwen3-TTS token loop: Talker decode step + 15-group CodePredictor.

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this module; it is the
checker that the GPU path is compared against (tests/, __graft_entry__.smoke() and the
``cpu_baseline`` leg of bench.py).

Sources restated (reference = /root/reference of piedshag/qwen3-tts-hip):

* one decoder layer, decode and prefill forms:   src/model/decode.rs:1300-1475, 1077-1298
* RMSNorm / RoPE / SwiGLU / softmax / attention:  src/gpu/kernels.rs:1-38, 40-77, 106-117,
  120-174, 976-1119
* Talker head, CP prefix, next-step input:         src/model/talker.rs:252-356, 431-496
* CodePredictor groups and positions:              src/model/code_predictor.rs:366-471, 754-862
* frame loop, EOS, trailing text, capacity:        src/generation.rs:608-617, 657-749, 852-963
* logit processing and sampling:                   oracle/sampling.py

Numerics contract shared with the GPU path (the reference itself is fp32 end to end):
weights are the bf16 values of the synthetic checkpoint (exact in any wider type);
activations are carried in ``dtype`` (float64 for parity fixtures, float32 for the
timed CPU baseline); the KV cache keeps the activation precision, as the reference's
does.  ``kv_bf16=True`` models the GPU's optional bf16 KV cache: K and V are rounded to
bf16 when stored and attention reads them back from the cache, also for the current
position.  RoPE angles are ``pos * theta**(-2i/d)`` computed in float64.
"""
from __future__ import annotations

import dataclasses
import time
from typing import Dict, List, Optional, Sequence

import numpy as np

from . import philox
from .sampling import (GREEDY, SamplingConfig, apply_repetition_penalty, select, suppress,
                       top2_margin)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round to the nearest bf16 value (ties to even), returned in x's dtype.

    Rounds the float32 image of x, which is exact for float32 inputs; for float64
    inputs that lie within half a float32 ulp of a bf16 tie this can differ from a
    direct float64 -> bf16 rounding, a case that has probability ~2**-29 per value.
    """
    f = np.asarray(x, dtype=np.float32)
    u = f.view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)) << np.uint32(16)
    return r.view(np.float32).astype(x.dtype, copy=False)


def rmsnorm(x: np.ndarray, gamma: np.ndarray, eps: float) -> np.ndarray:
    """x * rsqrt(mean(x^2) + eps) * gamma over the last axis (kernels.rs:1-38)."""
    ms = np.mean(x * x, axis=-1, keepdims=True)
    return x / np.sqrt(ms + eps) * gamma


def rope_tables(max_pos: int, head_dim: int, theta: float):
    half = head_dim // 2
    inv = theta ** (-(2.0 * np.arange(half, dtype=np.float64)) / head_dim)
    ang = np.arange(max_pos, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang), np.sin(ang)


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Rotate-half RoPE.  x: [S, heads, d]; cos/sin: [S, d/2] (kernels.rs:40-77)."""
    half = x.shape[-1] // 2
    a, b = x[..., :half], x[..., half:]
    c, s = cos[:, None, :].astype(x.dtype), sin[:, None, :].astype(x.dtype)
    return np.concatenate([a * c - b * s, b * c + a * s], axis=-1)


def silu(x: np.ndarray) -> np.ndarray:
    return x / (1.0 + np.exp(-x))


@dataclasses.dataclass
class StackDims:
    hidden: int
    intermediate: int
    layers: int
    q_heads: int
    kv_heads: int
    head_dim: int
    eps: float
    theta: float


class Stack:
    """KV-cached decoder stack (``DecodeStepStack``, decode.rs:84-1001)."""

    def __init__(self, tensors: Dict[str, np.ndarray], prefix: str, dims: StackDims, cap: int,
                 dtype=np.float64, kv_bf16: bool = False):
        self.d = dims
        self.cap = cap
        self.dtype = dtype
        self.kv_bf16 = kv_bf16
        f = lambda n: bf16_bits_to_f32(tensors[n]).astype(dtype)
        self.layers = []
        for i in range(dims.layers):
            p = f"{prefix}.layers.{i}"
            self.layers.append(dict(
                g_in=f(f"{p}.input_layernorm.weight"), g_post=f(f"{p}.post_attention_layernorm.weight"),
                wq=f(f"{p}.self_attn.q_proj.weight"), wk=f(f"{p}.self_attn.k_proj.weight"),
                wv=f(f"{p}.self_attn.v_proj.weight"), wo=f(f"{p}.self_attn.o_proj.weight"),
                gq=f(f"{p}.self_attn.q_norm.weight"), gk=f(f"{p}.self_attn.k_norm.weight"),
                wg=f(f"{p}.mlp.gate_proj.weight"), wu=f(f"{p}.mlp.up_proj.weight"),
                wd=f(f"{p}.mlp.down_proj.weight"),
            ))
        self.cos, self.sin = rope_tables(cap, dims.head_dim, dims.theta)
        self.reset()

    def reset(self) -> None:
        d = self.d
        self.k = np.zeros((d.layers, d.kv_heads, self.cap, d.head_dim), dtype=self.dtype)
        self.v = np.zeros_like(self.k)

    def _layer(self, li: int, x: np.ndarray, pos0: int) -> np.ndarray:
        """One layer over rows x[S, H] at positions pos0 .. pos0+S-1 (causal)."""
        d, w = self.d, self.layers[li]
        S = x.shape[0]
        L = pos0 + S
        if L > self.cap:
            raise ValueError(f"position {L - 1} outside cache length {self.cap}")
        xn = rmsnorm(x, w["g_in"], d.eps)
        q = (xn @ w["wq"].T).reshape(S, d.q_heads, d.head_dim)
        k = (xn @ w["wk"].T).reshape(S, d.kv_heads, d.head_dim)
        v = (xn @ w["wv"].T).reshape(S, d.kv_heads, d.head_dim)
        q = rmsnorm(q, w["gq"], d.eps)
        k = rmsnorm(k, w["gk"], d.eps)
        cos, sin = self.cos[pos0:L], self.sin[pos0:L]
        q = rope(q, cos, sin)
        k = rope(k, cos, sin)
        if self.kv_bf16:
            k, v = round_bf16(k), round_bf16(v)
        self.k[li, :, pos0:L] = k.transpose(1, 0, 2)
        self.v[li, :, pos0:L] = v.transpose(1, 0, 2)
        group = d.q_heads // d.kv_heads
        scale = 1.0 / np.sqrt(d.head_dim)
        out = np.empty((S, d.q_heads, d.head_dim), dtype=self.dtype)
        qpos = np.arange(pos0, L)[:, None]
        kpos = np.arange(L)[None, :]
        mask = kpos > qpos
        for h in range(d.q_heads):
            kv = h // group
            s = (q[:, h, :] @ self.k[li, kv, :L].T) * scale
            s = np.where(mask, -np.inf, s)
            s = s - s.max(axis=-1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=-1, keepdims=True)
            out[:, h, :] = p @ self.v[li, kv, :L]
        x1 = x + out.reshape(S, -1) @ w["wo"].T
        h1 = rmsnorm(x1, w["g_post"], d.eps)
        m = silu(h1 @ w["wg"].T) * (h1 @ w["wu"].T)
        return x1 + m @ w["wd"].T

    def forward(self, x: np.ndarray, pos0: int) -> np.ndarray:
        x = np.asarray(x, dtype=self.dtype).reshape(-1, self.d.hidden)
        for li in range(self.d.layers):
            x = self._layer(li, x, pos0)
        return x

    def prefill(self, x: np.ndarray) -> np.ndarray:
        """decode.rs:845-880: rows at positions 0..P-1; returns every row's output."""
        return self.forward(x, 0)

    def decode_step(self, x: np.ndarray, offset: int) -> np.ndarray:
        """decode.rs:951-1001: one row at position ``offset``."""
        if offset >= self.cap:
            raise ValueError(f"offset {offset} outside cache length {self.cap}")
        return self.forward(x, offset)[0]


def _dims(cfg: dict, eps_key="rms_norm_eps") -> StackDims:
    return StackDims(hidden=cfg["hidden_size"], intermediate=cfg["intermediate_size"],
                     layers=cfg["num_hidden_layers"], q_heads=cfg["num_attention_heads"],
                     kv_heads=cfg["num_key_value_heads"], head_dim=cfg["head_dim"],
                     eps=cfg[eps_key], theta=cfg["rope_theta"])


@dataclasses.dataclass
class GenerateOptions:
    """Fields of the reference's ``GenerateOptions`` that act on the token loop
    (generation.rs:40-77).  ``seed`` keys the Philox stream (oracle/philox.py)."""
    max_frames: int = 240
    do_sample: bool = True
    top_k: int = 50
    top_p: float = 1.0
    temperature: float = 0.9
    repetition_penalty: float = 1.05
    subtalker_dosample: bool = True
    subtalker_top_k: int = 50
    subtalker_top_p: float = 1.0
    subtalker_temperature: float = 0.9
    seed: int = 0
    repetition_penalty_per_occurrence: bool = False   # see sampling.apply_repetition_penalty

    @classmethod
    def greedy(cls, max_frames: int = 240) -> "GenerateOptions":
        return cls(max_frames=max_frames, do_sample=False, repetition_penalty=1.0,
                   subtalker_dosample=False)

    def talker_sampling(self) -> SamplingConfig:
        return SamplingConfig(self.do_sample, self.top_k, self.top_p, self.temperature)

    def subtalker_sampling(self) -> SamplingConfig:
        return SamplingConfig(self.subtalker_dosample, self.subtalker_top_k, self.subtalker_top_p,
                              self.subtalker_temperature)

    def validate(self) -> None:
        """generation.rs:569-583."""
        if self.max_frames <= 0:
            raise ValueError("max_frames must be non-zero")
        if not self.repetition_penalty > 0.0:
            raise ValueError("repetition_penalty must be positive")
        self.talker_sampling().validate("talker")
        self.subtalker_sampling().validate("subtalker")


@dataclasses.dataclass
class RolloutTrace:
    codes: np.ndarray                 # [F, 16] int32, frame-major [semantic, a1..a15]
    ended_by_eos: bool
    talker_logits: np.ndarray         # [T, V] raw logits of every Talker evaluation (T = F or F+1)
    talker_margins: np.ndarray        # [T] top-2 gap of the logits the token was chosen from
    cp_margins: np.ndarray            # [F, 15]
    talker_hidden: np.ndarray         # [T, H] normed hidden fed to the CodePredictor
    cp_logits: List[np.ndarray]       # per frame [15, V_cp] (kept for the first frames only)

    @property
    def frames(self) -> int:
        return int(self.codes.shape[0])


class Oracle:
    """Talker + CodePredictor + frame loop on the CPU."""

    def __init__(self, tensors: Dict[str, np.ndarray], config: dict, max_cache_steps: int = 512,
                 dtype=np.float64, kv_bf16: bool = False):
        tc = config["talker_config"]
        cc = tc["code_predictor_config"]
        self.dtype = dtype
        self.config = config
        self.codec_eos = tc["codec_eos_token_id"]
        self.num_code_groups = tc["num_code_groups"]
        self.max_cache_steps = max_cache_steps
        f = lambda n: bf16_bits_to_f32(tensors[n]).astype(dtype)
        # Talker (talker.rs:64-130)
        self.t_dims = _dims(tc)
        self.talker = Stack(tensors, "talker.model", self.t_dims, max_cache_steps, dtype, kv_bf16)
        self.t_norm = f("talker.model.norm.weight")
        self.codec_head = f("talker.codec_head.weight")
        self.codec_emb = f("talker.model.codec_embedding.weight")
        # CodePredictor (code_predictor.rs:146-263); cache length = num_code_groups
        self.c_dims = _dims(cc)
        self.cp = Stack(tensors, "talker.code_predictor.model", self.c_dims, self.num_code_groups,
                        dtype, kv_bf16)
        self.c_norm = f("talker.code_predictor.model.norm.weight")
        n_ac = self.num_code_groups - 1
        self.lm_heads = [f(f"talker.code_predictor.lm_head.{g}.weight") for g in range(n_ac)]
        self.cp_emb = [f(f"talker.code_predictor.model.codec_embedding.{g}.weight") for g in range(n_ac)]
        if self.t_dims.hidden != self.c_dims.hidden:
            self.proj_w = f("talker.code_predictor.small_to_mtp_projection.weight")
            self.proj_b = f("talker.code_predictor.small_to_mtp_projection.bias")
        else:
            self.proj_w = self.proj_b = None
        self.hidden = None        # normed Talker hidden of the last evaluation
        self.token = None

    # -- Talker ---------------------------------------------------------------------------
    def talker_logits(self, pre_norm: np.ndarray) -> np.ndarray:
        self.hidden = rmsnorm(pre_norm, self.t_norm, self.t_dims.eps)
        return self.codec_head @ self.hidden

    def talker_select(self, logits, history, penalty, cfg: SamplingConfig, u, per_occurrence: bool = False):
        """compute_logits_and_token_with_options (talker.rs:431-496)."""
        l = logits
        if history is not None and len(history):
            l = apply_repetition_penalty(l, history, penalty, per_occurrence)
        l = suppress(l, self.codec_eos)
        return select(l, cfg, u), top2_margin(l)

    def prefill(self, prefill: np.ndarray) -> np.ndarray:
        out = self.talker.prefill(prefill)
        return self.talker_logits(out[-1])

    def decode(self, step_input: np.ndarray, offset: int) -> np.ndarray:
        out = self.talker.decode_step(step_input, offset)
        return self.talker_logits(out)

    def prepare_code_predictor_prefix(self, semantic: int) -> np.ndarray:
        """talker.rs:296-318: [normed hidden ; codec_emb[semantic]]."""
        return np.stack([self.hidden, self.codec_emb[semantic]])

    def build_step_input(self, semantic: int, acoustic_sum: np.ndarray, trailing_row: np.ndarray):
        """talker.rs:320-356: codec_emb[semantic] + acoustic_sum + trailing."""
        return (self.codec_emb[semantic] + acoustic_sum) + trailing_row

    # -- CodePredictor --------------------------------------------------------------------
    def project(self, x: np.ndarray) -> np.ndarray:
        """code_predictor.rs:754-817 (identity when talker and CP widths match)."""
        if self.proj_w is None:
            return x
        return x @ self.proj_w.T + self.proj_b

    def cp_logits(self, pre_norm: np.ndarray, group: int) -> np.ndarray:
        """logits_for_hidden (code_predictor.rs:819-862)."""
        return self.lm_heads[group] @ rmsnorm(pre_norm, self.c_norm, self.c_dims.eps)

    def code_predictor(self, prefix: np.ndarray, cfg: SamplingConfig = GREEDY, seed: int = 0,
                       frame: int = 0, forced: Optional[Sequence[int]] = None):
        """generate_inner(_sampled) (code_predictor.rs:366-471).

        Returns (tokens[15], embedding_sum[talker_H], logits[15, V], margins[15]).
        ``forced`` replaces the chosen tokens (teacher forcing for parity checks).
        """
        n_ac = self.num_code_groups - 1
        self.cp.reset()
        out = self.cp.prefill(self.project(np.asarray(prefix, dtype=self.dtype)))
        pre = out[1]
        tokens = np.zeros(n_ac, dtype=np.int32)
        logits_all = np.zeros((n_ac, self.lm_heads[0].shape[0]), dtype=self.dtype)
        margins = np.zeros(n_ac)
        emb_sum = None
        for g in range(n_ac):
            if g > 0:
                pre = self.cp.decode_step(self.project(cur), g + 1)
            logits = self.cp_logits(pre, g)
            logits_all[g] = logits
            margins[g] = top2_margin(logits)
            u = philox.sampler_uniform(seed, frame, 1 + g) if cfg.do_sample else None
            tok = select(logits, cfg, u)
            if forced is not None:
                tok = int(forced[g])
            tokens[g] = tok
            cur = self.cp_emb[g][tok]
            emb_sum = cur.copy() if emb_sum is None else emb_sum + cur
        return tokens, emb_sum, logits_all, margins

    # -- frame loop -----------------------------------------------------------------------
    def rollout(self, prefill: np.ndarray, trailing_text: np.ndarray, tts_pad: np.ndarray,
                opts: GenerateOptions, keep_cp_logits: int = 0,
                forced_codes: Optional[np.ndarray] = None, timings: Optional[dict] = None) -> RolloutTrace:
        """``HipTtsEngine::rollout`` (generation.rs:657-749).

        ``forced_codes`` ([F, 16]) teacher-forces the chosen tokens: logits are still
        computed from the oracle's own state, but the loop continues with the forced
        tokens, so a GPU run can be checked step by step even past a near-tie.  ``timings``,
        when given, receives the seconds of the prefill (``prefill_s``) and of the frames
        after it (``frames_s``), the split the reference's GenerationProfile reports.
        """
        opts.validate()
        P = int(prefill.shape[0])
        if P == 0:
            raise ValueError("prefill steps must be non-zero")
        if P + opts.max_frames > self.max_cache_steps:
            raise ValueError(f"requested {P + opts.max_frames} cache steps but engine was loaded for "
                             f"{self.max_cache_steps}")
        tcfg, ccfg = opts.talker_sampling(), opts.subtalker_sampling()
        t0 = time.perf_counter()
        self.talker.reset()
        logits = self.prefill(prefill)
        u = philox.sampler_uniform(opts.seed, 0, 0) if tcfg.do_sample else None
        semantic, margin = self.talker_select(logits, None, 1.0, tcfg, u)
        if forced_codes is not None and len(forced_codes):
            semantic = int(forced_codes[0][0])
        t_logits, t_margins, t_hidden = [logits], [margin], [self.hidden.copy()]
        t1 = time.perf_counter()
        codes, cp_margins, cp_logits, history = [], [], [], []
        ended = False
        for frame in range(opts.max_frames):
            if semantic == self.codec_eos:
                ended = True
                break
            prefix = self.prepare_code_predictor_prefix(semantic)
            forced = None
            if forced_codes is not None and frame < len(forced_codes):
                forced = forced_codes[frame][1:]
            acoustic, emb_sum, lg, mg = self.code_predictor(prefix, ccfg, opts.seed, frame, forced)
            codes.append([semantic] + [int(a) for a in acoustic])
            cp_margins.append(mg)
            if frame < keep_cp_logits:
                cp_logits.append(lg)
            history.append(semantic)
            if frame + 1 < opts.max_frames:
                row = trailing_text[frame] if frame < len(trailing_text) else tts_pad
                step = self.build_step_input(semantic, emb_sum, np.asarray(row, dtype=self.dtype))
                logits = self.decode(step, P + frame)
                use_hist = opts.repetition_penalty != 1.0 or tcfg.do_sample
                u = philox.sampler_uniform(opts.seed, frame + 1, 0) if tcfg.do_sample else None
                semantic, margin = self.talker_select(logits, history if use_hist else None,
                                                      opts.repetition_penalty, tcfg, u,
                                                      opts.repetition_penalty_per_occurrence)
                if forced_codes is not None and frame + 1 < len(forced_codes):
                    semantic = int(forced_codes[frame + 1][0])
                t_logits.append(logits)
                t_margins.append(margin)
                t_hidden.append(self.hidden.copy())
        if timings is not None:
            timings["prefill_s"] = t1 - t0
            timings["frames_s"] = time.perf_counter() - t1
        return RolloutTrace(
            codes=np.asarray(codes, dtype=np.int32).reshape(-1, self.num_code_groups),
            ended_by_eos=ended,
            talker_logits=np.asarray(t_logits, dtype=np.float64),
            talker_margins=np.asarray(t_margins),
            cp_margins=np.asarray(cp_margins).reshape(-1, self.num_code_groups - 1),
            talker_hidden=np.asarray(t_hidden, dtype=np.float64),
            cp_logits=cp_logits,
        )
