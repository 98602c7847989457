"""q3t_prepare_text_noalloc: the prompt rows of q3t_prepare_text with no device allocation
(its workspace in the library's static per-GPU scratch array).

It runs the same kernels on the same plan, with the same K splits (their partials stay in the
engine's own workspace), so its rows must equal q3t_prepare_text's bit for bit: on two calls
in a row, the second with a smaller prompt (the scratch keeps the first call's contents),
and against the host oracle of the text layout.  A prompt past the scratch is refused
before any launch.
"""
import numpy as np
import pytest

from q3t import engine as E
from q3t import textprep

pytestmark = pytest.mark.gpu


def _same(a: textprep.PreparedInputs, b: textprep.PreparedInputs):
    for name in ("prefill", "trailing_text", "tts_pad_embed"):
        x, y = getattr(a, name), getattr(b, name)
        assert x.shape == y.shape, name
        np.testing.assert_array_equal(x, y, err_msg=name)


@pytest.mark.parametrize("spec", ["tiny", "tiny-proj"])
def test_prepare_text_noalloc_equals_prepare_text(models, spec):
    model, d = models.get_with_text(spec)
    host = textprep.TextPrep(model)
    print(f"[gpu] prepare_text_noalloc {spec}", flush=True)
    with E.HipTtsEngine(d, E.EngineOptions(max_cache_steps=128)) as eng:
        for n, look, speaker in ((300, 7, "ryan"), (24, 1 << 30, "serena"), (1, 1, "ryan")):
            ids = textprep.random_prompt(n, 11 + n)
            ref = eng.prepare_text(ids, speaker=speaker, text_lookahead_tokens=look)
            got = eng.prepare_text(ids, speaker=speaker, text_lookahead_tokens=look, no_alloc=True)
            _same(got, ref)
            want = host.prepare(ids, speaker=speaker, text_lookahead_tokens=look)
            err = max(float(np.abs(got.prefill - want.prefill).max()),
                      float(np.abs(got.trailing_text - want.trailing_text).max()),
                      float(np.abs(got.tts_pad_embed - want.tts_pad_embed).max()))
            print(f"{spec}: {n} ids, P={got.prefill_steps} T={got.trailing_steps}, max err vs host {err:.2e}")
            assert err <= 1e-4
        # past the scratch: refused on the host, no launch; the entry point still works after
        with pytest.raises(E.InvalidInputError, match="q3t_prepare_text_noalloc holds at most"):
            eng.prepare_text(textprep.random_prompt(4000, 5), no_alloc=True)
        ids = textprep.random_prompt(40, 6)
        _same(eng.prepare_text(ids, no_alloc=True), eng.prepare_text(ids))
