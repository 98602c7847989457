"""Talker prompt prefill at prompt lengths around the attention's 16-row query blocks and
16-key tiles (1, 2, 15, 16, 17, 33, and past the 128-row tiles of the prefill GEMM up to
cap - 1), through the q3t_debug_talker_prefill hook, against the float64 oracle's prefill
(decode.rs:1077-1298).  Both query-head groupings (two query heads per KV head and one) and
both KV cache types (the oracle rounds K and V to bf16 where the GPU stores bf16)."""
import numpy as np
import pytest

from q3t import engine as E
from q3t import synth
from oracle.model import Oracle

pytestmark = pytest.mark.gpu

CAP = 200
LENGTHS = (1, 2, 15, 16, 17, 33, 130, CAP - 1)


def _close(got, want, max_tol, mean_tol, what):
    d = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))
    print(f"  {what}: max {d.max():.2e} mean {d.mean():.2e}")
    assert d.max() <= max_tol and d.mean() <= mean_tol, f"{what}: max {d.max():.3g} mean {d.mean():.3g}"


@pytest.mark.parametrize("spec", ["tiny", "tiny-g1"])
@pytest.mark.parametrize("kv_bf16", [False, True])
def test_prefill_lengths_match_oracle(models, spec, kv_bf16):
    model, d = models.get(spec, 0)
    H = model.spec.talker.hidden
    rng = np.random.default_rng(11)
    print(f"[gpu] prefill lengths {spec} kv_bf16={kv_bf16}", flush=True)
    with E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=CAP, kv_bf16=kv_bf16)) as eng:
        for P in LENGTHS:
            x = (rng.standard_normal((P, H)) * 0.5).astype(np.float32)
            hidden, logits, _ = eng.debug_talker_prefill(x)
            o = Oracle(model.tensors, model.config(), max_cache_steps=CAP, kv_bf16=kv_bf16)
            want = o.prefill(x.astype(np.float64))
            # fp32 KV: ~7e-7 measured; bf16 KV: cache values on either side of a bf16
            # rounding boundary, ~6e-5 measured
            tol = (2e-3, 2e-4) if kv_bf16 else (1e-5, 1e-6)
            _close(hidden, o.hidden, *tol, f"P={P} hidden")
            _close(logits, want, *tol, f"P={P} logits")
