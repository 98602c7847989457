"""Pins the oracle's decoder stack against independent routines.

* transformers' Qwen3Model (installed library; not the reference) on tiny random weights:
  same block structure as the reference's DecodeStepStack (decode.rs:1077-1475): per-head
  q/k RMSNorm before rotate-half RoPE, GQA with kv head = q head // group, SwiGLU, pre-norm
  residuals.  Full-sequence forward vs the oracle's prefill, and vs prefill + KV-cached
  decode steps (positions, cache reads, causal mask).
* closed forms and invariants of RMSNorm, RoPE and attention.
"""
import numpy as np
import pytest
import torch

import hf_ref
from oracle import model as om
from q3t import synth

# float64 throughout (tests/hf_ref.py): agreement is ~1e-14; a wrong sign, index or operand
# order shows up as O(0.1).
HF_TOL = 1e-10

SHAPE = synth.StackShape(hidden=64, intermediate=96, layers=3, q_heads=4, kv_heads=2, head_dim=16,
                         vocab=32, rope_theta=1e4)


def _tensors(seed=3):
    inv = synth._stack_tensors("m", SHAPE)
    return {n: synth.generate_tensor(seed, n, shape, kind) for n, shape, kind in inv}


def _hf_model(tensors):
    return hf_ref.qwen3_model(tensors, "m", SHAPE.hidden, SHAPE.intermediate, SHAPE.layers, SHAPE.q_heads,
                              SHAPE.kv_heads, SHAPE.head_dim, SHAPE.rms_eps, SHAPE.rope_theta)


def _oracle_stack(tensors, cap=64, dtype=np.float64):
    d = om.StackDims(SHAPE.hidden, SHAPE.intermediate, SHAPE.layers, SHAPE.q_heads, SHAPE.kv_heads,
                     SHAPE.head_dim, SHAPE.rms_eps, SHAPE.rope_theta)
    return om.Stack(tensors, "m", d, cap, dtype)


def _final_norm(tensors, x):
    return om.rmsnorm(x, synth.bf16_bits_to_f32(tensors["m.norm.weight"]).astype(np.float64), SHAPE.rms_eps)


def test_prefill_matches_transformers_qwen3():
    t = _tensors()
    x = np.random.default_rng(0).standard_normal((9, SHAPE.hidden)) * 0.5
    with torch.no_grad():
        ref = _hf_model(t)(inputs_embeds=torch.from_numpy(x)[None]).last_hidden_state[0].numpy()
    got = _final_norm(t, _oracle_stack(t).prefill(x))
    np.testing.assert_allclose(got, ref, rtol=0, atol=HF_TOL)


def test_prefill_then_decode_matches_full_forward():
    t = _tensors(5)
    x = np.random.default_rng(1).standard_normal((12, SHAPE.hidden)) * 0.5
    with torch.no_grad():
        ref = _hf_model(t)(inputs_embeds=torch.from_numpy(x)[None]).last_hidden_state[0].numpy()
    st = _oracle_stack(t)
    st.prefill(x[:7])
    rows = [st.decode_step(x[p], p) for p in range(7, 12)]
    got = _final_norm(t, np.stack(rows))
    np.testing.assert_allclose(got, ref[7:], rtol=0, atol=HF_TOL)


def test_rmsnorm_closed_form():
    g = np.array([1.0, 2.0, 0.5, 1.0])
    x = np.full(4, 3.0)
    np.testing.assert_allclose(om.rmsnorm(x, g, 0.0), g, rtol=1e-15)
    x = np.array([1.0, -1.0, 1.0, -1.0]) * 2
    np.testing.assert_allclose(om.rmsnorm(x, np.ones(4), 1e-6), x / np.sqrt(4 + 1e-6))


def test_rope_invariants():
    d = 16
    cos, sin = om.rope_tables(32, d, 1e6)
    rng = np.random.default_rng(2)
    q = rng.standard_normal((32, 1, d))
    k = rng.standard_normal((1, 1, d))
    r = om.rope(q, cos, sin)
    np.testing.assert_allclose(r[0], q[0])                      # position 0 is the identity
    half = d // 2
    np.testing.assert_allclose(r[..., :half] ** 2 + r[..., half:] ** 2,      # pair norms kept
                               q[..., :half] ** 2 + q[..., half:] ** 2, rtol=1e-12)
    # q(m).k(n) depends only on m - n
    qq = np.repeat(q[:1], 32, axis=0)
    kk = np.repeat(k, 32, axis=0)
    rq, rk = om.rope(qq, cos, sin), om.rope(kk, cos, sin)
    dots = np.array([[rq[m, 0] @ rk[n, 0] for n in range(32)] for m in range(32)])
    for delta in (0, 3, 7):
        diag = np.array([dots[m, m - delta] for m in range(delta, 32)])
        np.testing.assert_allclose(diag, diag[0], rtol=1e-9, atol=1e-9)
    # angle of pair i at position p is p * theta^(-2i/d)
    np.testing.assert_allclose(np.arctan2(sin[5, 1], cos[5, 1]), 5 * 1e6 ** (-2 / d))


def test_attention_single_position_returns_v():
    """L = 1: softmax over one key is 1, so the attention output is that V row."""
    t = _tensors(7)
    st = _oracle_stack(t)
    x = np.random.default_rng(3).standard_normal((1, SHAPE.hidden))
    st.forward(x, 0)
    lw = st.layers[0]
    xn = om.rmsnorm(x, lw["g_in"], SHAPE.rms_eps)
    v = (xn @ lw["wv"].T).reshape(SHAPE.kv_heads, SHAPE.head_dim)
    np.testing.assert_allclose(st.v[0, :, 0], v, rtol=1e-12)


def test_bf16_kv_option_rounds_cache():
    t = _tensors(9)
    d = om.StackDims(SHAPE.hidden, SHAPE.intermediate, SHAPE.layers, SHAPE.q_heads, SHAPE.kv_heads,
                     SHAPE.head_dim, SHAPE.rms_eps, SHAPE.rope_theta)
    st = om.Stack(t, "m", d, 16, np.float64, kv_bf16=True)
    st.prefill(np.random.default_rng(4).standard_normal((5, SHAPE.hidden)))
    k = st.k[:, :, :5]
    np.testing.assert_array_equal(om.round_bf16(k), k)
