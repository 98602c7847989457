"""The HTTP server (q3t/server.py) in front of the real engine on the GPU, over a live socket on
127.0.0.1: the WAV of /api/generate and the PCM of /api/stream are byte-identical to what the
engine API returns for the same request (generate_codes + decode_codes; start_stream +
next_audio_chunk), which the other GPU tests hold to the oracle."""
import http.client
import threading

import numpy as np
import pytest

from q3t import engine as E
from q3t import server as S
from q3t.voice_clone import VoiceClonePrompt
from q3t.wav import pcm_s16le, wav_bytes

pytestmark = pytest.mark.gpu

CAP = 16
TEXT = "Hello there, general Kenobi."


@pytest.fixture(scope="module")
def served(models):
    _, d = models.get_with_text("tiny")
    eng = E.HipTtsEngine.load_with_max_frames(d, 0, CAP)
    logs = []
    srv = S.TtsServer(eng, CAP, log=logs.append)
    sock = S.listen("127.0.0.1:0")
    port = sock.getsockname()[1]
    t = threading.Thread(target=srv.serve_forever, args=(sock,), daemon=True)
    t.start()
    yield eng, port, logs, srv
    sock.close()
    try:
        http.client.HTTPConnection("127.0.0.1", port, timeout=5).request("GET", "/health")
    except OSError:
        pass
    t.join(timeout=30)
    eng.close()


def _post(port, path, form):
    c = http.client.HTTPConnection("127.0.0.1", port, timeout=120)
    body = "&".join(f"{k}={v}" for k, v in form.items())
    c.request("POST", path, body=body, headers={"Content-Type": S.FORM_TYPE})
    r = c.getresponse()
    return r, r.read()


GREEDY = {"text": TEXT.replace(" ", "+").replace(",", "%2C"), "max_frames": "12", "do_sample": "false",
          "subtalker_dosample": "false", "repetition_penalty": "1", "speaker": "Serena"}


def _greedy_options():
    return E.GenerateOptions(speaker="Serena", max_frames=12, decode_audio=False, do_sample=False,
                             subtalker_dosample=False, repetition_penalty=1.0)


def test_generate_route_matches_engine_api(served):
    eng, port, logs, _ = served
    print("[gpu] server /api/generate greedy", flush=True)
    r, body = _post(port, "/api/generate", dict(GREEDY, wav_gain="0.7"))
    assert r.status == 200, body
    g = eng.generate_codes(TEXT, _greedy_options())
    samples = eng.decode_codes(g.codes)
    assert g.frames > 0 and samples.size == g.frames * eng.info["samples_per_frame"]
    assert body == wav_bytes(samples, E.SAMPLE_RATE, 0.7)
    assert r.getheader("X-TTS-Frames") == str(g.frames)
    assert r.getheader("X-TTS-Ended-By-EOS") == ("true" if g.ended_by_eos else "false")
    assert r.getheader("X-TTS-Samples") == str(samples.size)
    assert logs[-1].startswith(f"generated: voice_clone=false, frames={g.frames}")


def test_stream_route_matches_engine_api(served):
    eng, port, _, _ = served
    print("[gpu] server /api/stream greedy", flush=True)
    form = dict(GREEDY, stream_chunk_frames="5", text_lookahead_tokens="2", left_context_frames="3")
    r, body = _post(port, "/api/stream", form)
    assert r.status == 200 and r.getheader("Transfer-Encoding") == "chunked"
    want = b""
    with eng.start_stream(TEXT, _greedy_options(), E.StreamOptions(text_lookahead_tokens=2, left_context_frames=3)) as st:
        while (chunk := st.next_audio_chunk(5)) is not None:
            want += pcm_s16le(chunk.samples, 1.0)
    assert len(want) > 0 and body == want


def test_sampled_requests_repeat_by_seed(served):
    _, port, _, _ = served
    print("[gpu] server /api/generate sampled", flush=True)
    form = {"text": "Seeded+sampling.", "max_frames": "10", "seed": "7"}
    r1, b1 = _post(port, "/api/generate", form)
    r2, b2 = _post(port, "/api/generate", form)
    r3, b3 = _post(port, "/api/generate", dict(form, seed="8"))
    assert r1.status == r2.status == r3.status == 200
    assert b1 == b2 and r1.getheader("X-TTS-Seed") == "7"
    assert b3 != b1


def test_voice_clone_routes_match_engine_api(served):
    eng, port, _, srv = served
    print("[gpu] server voice clone routes", flush=True)
    emb = np.random.default_rng(5).standard_normal(eng.info["talker_hidden"]) * 0.05
    prompt = VoiceClonePrompt(emb.astype(np.float32), x_vector_only_mode=True)
    srv.voice_clone_prompt = prompt
    try:
        form = dict(GREEDY, use_voice_clone="true")
        r, body = _post(port, "/api/generate", form)
        assert r.status == 200 and r.getheader("X-TTS-Voice-Clone") == "true", body
        g = eng.generate_voice_clone_codes(TEXT, prompt, _greedy_options())
        assert body == wav_bytes(eng.decode_codes(g.codes), E.SAMPLE_RATE, 1.0)
        r, body = _post(port, "/api/stream", dict(form, stream_chunk_frames="4"))
        assert r.status == 200
        want = b""
        with eng.start_voice_clone_stream(TEXT, prompt, _greedy_options(), E.StreamOptions()) as st:
            while (chunk := st.next_audio_chunk(4)) is not None:
                want += pcm_s16le(chunk.samples, 1.0)
        assert len(want) > 0 and body == want
    finally:
        srv.voice_clone_prompt = None


def test_rejections(served):
    _, port, _, _ = served
    r, body = _post(port, "/api/generate", {"max_frames": str(CAP + 1)})
    assert (r.status, body) == (400, f"max_frames must be in 1..={CAP} for this server\n".encode())
    r, body = _post(port, "/api/stream", {"use_voice_clone": "true", "max_frames": "4"})
    assert r.status == 400 and b"voice_clone_prompt_json" in body
    r, body = _post(port, "/api/generate", {"top_p": "2", "max_frames": "4"})  # the engine's option check: a 500
    assert r.status == 500 and b"top_p" in body
