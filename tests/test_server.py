"""The HTTP serving surface (q3t/server.py) against the reference's tts-server rules
(src/bin/tts-server.rs): routes, form parsing, defaults and limits, status codes, headers, WAV
and chunked-PCM wire formats.  A stand-in engine replaces the GPU; the same server runs the
real engine in tests/test_gpu_server.py."""
import http.client
import struct
import threading

import numpy as np
import pytest

from q3t import server as S
from q3t.engine import GeneratedAudioChunk, GeneratedCodes, InvalidInputError
from q3t.wav import pcm_s16le, wav_bytes

SPF = 1920  # samples per codec frame at 24 kHz / 12.5 Hz


class FakeStream:
    def __init__(self, frames, seed):
        self.frames, self.done, self.closed, self.seed = frames, 0, False, seed

    def next_audio_chunk(self, n):
        if self.done >= self.frames:
            return None
        k = min(n, self.frames - self.done)
        x = np.sin(np.arange(k * SPF, dtype=np.float32) * 0.01 + self.done + self.seed).astype(np.float32) * 1.3
        self.done += k
        return GeneratedAudioChunk(x, 24000, k, self.done, self.done == self.frames)

    def close(self):
        self.closed = True


class FakeEngine:
    """Deterministic codes and audio from the options; records every call."""

    def __init__(self):
        self.calls = []
        self.streams = []
        self.fail = None

    def _codes(self, text, o):
        if self.fail:
            raise self.fail
        n = min(o.max_frames, 5)
        codes = (np.arange(n * 16, dtype=np.int32).reshape(n, 16) + len(text)) % 2048
        return GeneratedCodes(codes, n, n < o.max_frames)

    def generate_codes(self, text, o):
        self.calls.append(("generate_codes", text, o))
        return self._codes(text, o)

    def generate_voice_clone_codes(self, text, prompt, o):
        self.calls.append(("generate_voice_clone_codes", text, o, prompt))
        return self._codes(text, o)

    def decode_codes(self, codes):
        return np.linspace(-1.5, 1.5, codes.shape[0] * SPF, dtype=np.float32)

    def start_stream(self, text, o, so):
        self.calls.append(("start_stream", text, o, so))
        if self.fail:
            raise self.fail
        st = FakeStream(min(o.max_frames, 7), len(text))
        self.streams.append(st)
        return st

    def start_voice_clone_stream(self, text, prompt, o, so):
        self.calls.append(("start_voice_clone_stream", text, o, so, prompt))
        st = FakeStream(min(o.max_frames, 7), len(text))
        self.streams.append(st)
        return st


def _post(path, body, ctype=S.FORM_TYPE):
    return S.Request("POST", path, {"content-type": ctype}, body.encode() if isinstance(body, str) else body)


def _srv(**kw):
    logs = []
    return S.TtsServer(FakeEngine(), kw.pop("cap", 240), log=logs.append, **kw), logs


# ------------------------------------------------------------------------------------- parsers
def test_percent_decode_and_form():
    assert S.percent_decode("a+b%20c") == "a b c"
    assert S.percent_decode("%E2%82%AC") == "€"
    assert S.percent_decode("50%") == "50%" and S.percent_decode("%4") == "%4"
    with pytest.raises(S.BadRequest, match="percent escape"):
        S.percent_decode("%zz")
    with pytest.raises(S.BadRequest, match="UTF-8"):
        S.percent_decode("%ff")
    assert S.parse_form(b"text=Hi+there&flag&&k=1&k=2") == {"text": "Hi there", "flag": "", "k": "2"}
    with pytest.raises(S.BadRequest, match="not UTF-8"):
        S.parse_form(b"\xff=1")


@pytest.mark.parametrize("value,ok", [("0", 0), ("+7", 7), ("18446744073709551615", 2**64 - 1),
                                      ("18446744073709551616", None), ("-1", None), (" 1", None),
                                      ("1_0", None), ("", None), ("1.0", None)])
def test_uint_grammar(value, ok):
    if ok is None:
        with pytest.raises(S.BadRequest):
            S.parse_uint(value, "n")
    else:
        assert S.parse_uint(value, "n") == ok


@pytest.mark.parametrize("value,ok", [("1", 1.0), ("-2.5", -2.5), (".5", 0.5), ("5.", 5.0), ("1e3", 1000.0),
                                      ("1.5E-1", float(np.float32(0.15))), ("inf", np.inf), ("-Infinity", -np.inf),
                                      ("1e60", np.inf), ("0.9", float(np.float32(0.9))), ("e5", None),
                                      (" 1", None), ("1_0", None), ("0x10", None), ("", None)])
def test_f32_grammar(value, ok):
    if ok is None:
        with pytest.raises(S.BadRequest):
            S.parse_f32(value, "x")
    else:
        assert S.parse_f32(value, "x") == ok
    assert np.isnan(S.parse_f32("NaN", "x"))


def test_bool_grammar():
    for v in ("1", "true", "YES", "On"):
        assert S.parse_bool(v, "b") is True
    for v in ("0", "False", "no", "OFF"):
        assert S.parse_bool(v, "b") is False
    with pytest.raises(S.BadRequest, match="invalid b: maybe"):
        S.parse_bool("Maybe", "b")


# ------------------------------------------------------------------------------------- framing
def _reader(data, step):
    chunks = [data[i:i + step] for i in range(0, len(data), step)]
    return lambda: chunks.pop(0) if chunks else b""


def test_request_reading():
    raw = b"POST /api/generate?x=1 HTTP/1.1\r\nHost: a\r\nContent-Type: text/plain\r\nContent-Length: 5\r\n\r\nhello"
    for step in (1, 7, 4096):
        r = S.parse_request_bytes(_reader(raw, step))
        assert (r.method, r.path, r.body) == ("POST", "/api/generate", b"hello")
        assert r.headers["content-type"] == "text/plain" and r.headers["host"] == "a"
    r = S.parse_request_bytes(_reader(b"GET / HTTP/1.1\r\n\r\nextra", 100))
    assert r.body == b"" and r.path == "/"


@pytest.mark.parametrize("raw,msg", [
    (b"", "connection closed"),
    (b"GET / HTTP/1.1\r\n", "connection closed"),
    (b"GET / HTTP/1.1\r\nX: " + b"a" * (64 * 1024), "request is too large"),
    (b"POST / HTTP/1.1\r\nContent-Length: 65537\r\n\r\n", "body is too large"),
    (b"POST / HTTP/1.1\r\nContent-Length: 10\r\n\r\nabc", "truncated request body"),
    (b"POST / HTTP/1.1\r\nContent-Length: x\r\n\r\n", "invalid content-length"),
    (b"\r\n\r\n", "missing method"),
    (b"GET\r\n\r\n", "missing path"),
])
def test_request_errors(raw, msg):
    with pytest.raises(S.BadRequest, match=msg):
        S.parse_request_bytes(_reader(raw, 4096))


def test_response_framing():
    r = S.text_response(404, "Not Found", "not found\n")
    assert S.response_head(r) == (b"HTTP/1.1 404 Not Found\r\nContent-Length: 10\r\nConnection: close\r\n"
                                  b"Content-Type: text/plain; charset=utf-8\r\n\r\n")
    r = S.Response(200, "OK", [("X-A", "1\r\n2")], chunks=iter(()))
    assert S.response_head(r) == b"HTTP/1.1 200 OK\r\nTransfer-Encoding: chunked\r\nConnection: close\r\nX-A: 1  2\r\n\r\n"
    assert S.chunk_frame(b"x" * 26) == b"1a\r\n" + b"x" * 26 + b"\r\n" and S.chunk_frame(b"") == b""
    assert S.CHUNKED_END == b"0\r\n\r\n"


# ------------------------------------------------------------------------------------- requests
def test_generation_request_defaults():
    g = S.parse_generation_request({}, 240, False)
    o = g.options
    assert g.text == "She said she would be here by noon."
    assert (o.max_frames, o.speaker, o.language, o.decode_audio) == (120, "ryan", "english", False)
    assert (o.do_sample, o.top_k, o.top_p, o.temperature) == (True, 50, 1.0, float(np.float32(0.9)))
    assert o.repetition_penalty == float(np.float32(1.05)) and o.seed == 0
    assert (o.subtalker_dosample, o.subtalker_top_k, o.subtalker_top_p) == (True, 50, 1.0)
    assert o.subtalker_temperature == float(np.float32(0.9))
    assert (g.wav_gain, g.stream_chunk_frames, g.use_voice_clone) == (1.0, 6, False)
    assert (g.stream_options.text_lookahead_tokens, g.stream_options.left_context_frames) == (8, 25)


def test_generation_request_fields():
    form = {"text": "  Hello  ", "max_frames": "240", "speaker": "Vivian", "language": "Chinese", "wav_gain": "0.5",
            "repetition_penalty": "1.1", "do_sample": "false", "top_k": "0", "top_p": "0.8", "temperature": "1",
            "subtalker_dosample": "no", "subtalker_top_k": "3", "subtalker_top_p": "0.5",
            "subtalker_temperature": "0.7", "seed": "18446744073709551615", "text_lookahead_tokens": "2",
            "stream_chunk_frames": "4", "left_context_frames": "0", "use_voice_clone": "on"}
    g = S.parse_generation_request(form, 240, True)
    o = g.options
    assert g.text == "Hello" and o.max_frames == 240 and o.speaker == "Vivian" and o.language == "Chinese"
    assert (o.do_sample, o.top_k, o.subtalker_dosample, o.subtalker_top_k) == (False, 0, False, 3)
    assert o.seed == 2**64 - 1 and g.wav_gain == 0.5 and g.use_voice_clone
    assert (g.stream_chunk_frames, g.stream_options.text_lookahead_tokens, g.stream_options.left_context_frames) == (4, 2, 0)


@pytest.mark.parametrize("form,msg", [
    ({"text": "   "}, "text must not be empty"),
    ({"max_frames": "0"}, r"max_frames must be in 1..=240 for this server"),
    ({"max_frames": "241"}, r"max_frames must be in 1..=240"),
    ({"max_frames": "-1"}, "invalid max_frames"),
    ({"speaker": "nobody"}, "unknown speaker"),
    ({"language": "klingon"}, "unknown language"),
    ({"repetition_penalty": "0"}, "repetition_penalty must be positive"),
    ({"repetition_penalty": "-1"}, "repetition_penalty must be positive"),
    ({"do_sample": "2"}, "invalid do_sample"),
    ({"top_p": "x"}, "invalid top_p"),
    ({"seed": "18446744073709551616"}, "invalid seed"),
    ({"text_lookahead_tokens": "0"}, "text_lookahead_tokens must be non-zero"),
    ({"stream_chunk_frames": "0"}, "stream_chunk_frames must be non-zero"),
    ({"use_voice_clone": "true"}, "requires starting the server with voice_clone_prompt_json"),
])
def test_generation_request_errors(form, msg):
    with pytest.raises(S.BadRequest, match=msg):
        S.parse_generation_request(form, 240, False)


# ------------------------------------------------------------------------------------- routes
def test_simple_routes():
    srv, _ = _srv()
    r = srv.handle(S.Request("GET", "/", {}, b""))
    assert r.code == 200 and b"/api/stream" in r.body and ("Cache-Control", "no-store") in r.headers
    assert srv.handle(S.Request("GET", "/health", {}, b"")).body == b"ok\n"
    r = srv.handle(S.Request("GET", "/favicon.ico", {}, b""))
    assert (r.code, r.body) == (204, b"")
    for req in (S.Request("GET", "/api/generate", {}, b""), S.Request("POST", "/", {}, b""),
                S.Request("DELETE", "/health", {}, b"")):
        r = srv.handle(req)
        assert (r.code, r.body) == (404, b"not found\n")
    r = srv.handle(_post("/api/generate", "text=a", "text/plain"))
    assert (r.code, r.body) == (415, b"expected application/x-www-form-urlencoded\n")
    r = srv.handle(_post("/api/stream", "max_frames=999"))
    assert (r.code, r.body) == (400, b"max_frames must be in 1..=240 for this server\n")
    assert srv.engine.calls == []


def test_generate_route_wav_and_headers():
    srv, logs = _srv(load_seconds=1.5)
    r = srv.handle(_post("/api/generate", "text=Hi&max_frames=9&wav_gain=0.5&do_sample=0&seed=42&top_k=7"))
    assert r.code == 200
    (name, text, o), = srv.engine.calls
    assert name == "generate_codes" and text == "Hi" and o.max_frames == 9 and o.decode_audio is False
    samples = np.linspace(-1.5, 1.5, 5 * SPF, dtype=np.float32)
    assert r.body == wav_bytes(samples, 24000, 0.5)
    h = dict(r.headers)
    assert h["Content-Type"] == "audio/wav" and h["X-TTS-Load-Seconds"] == "1.500000"
    assert (h["X-TTS-Frames"], h["X-TTS-Samples"], h["X-TTS-Ended-By-EOS"]) == ("5", str(5 * SPF), "true")
    assert h["X-TTS-Audio-Seconds"] == "0.400000" and h["X-TTS-Voice-Clone"] == "false"
    assert (h["X-TTS-Do-Sample"], h["X-TTS-Top-K"], h["X-TTS-Seed"]) == ("false", "7", "42")
    assert (h["X-TTS-Repetition-Penalty"], h["X-TTS-Temperature"], h["X-TTS-Top-P"]) == ("1.050000", "0.900000", "1.000000")
    for k in ("Generation", "Decode", "Wav", "Time-To-First-Audio", "Inference"):
        assert float(h[f"X-TTS-{k}-Seconds"]) >= 0
    assert float(h["X-TTS-Inference-RTF"]) >= 0
    assert logs and logs[0].startswith("generated: voice_clone=false, frames=5, samples=9600, ended_by_eos=true")


def test_voice_clone_routes_and_engine_errors():
    prompt = object()
    srv, logs = _srv(voice_clone_prompt=prompt)
    r = srv.handle(_post("/api/generate", "use_voice_clone=1&text=x"))
    assert r.code == 200 and srv.engine.calls[-1][0] == "generate_voice_clone_codes" and srv.engine.calls[-1][3] is prompt
    assert dict(r.headers)["X-TTS-Voice-Clone"] == "true"
    r = srv.handle(_post("/api/stream", "use_voice_clone=yes"))
    assert r.code == 200 and srv.engine.calls[-1][0] == "start_voice_clone_stream"
    list(r.chunks)
    srv.engine.fail = InvalidInputError(2, "top_p must be in (0, 1]")
    r = srv.handle(_post("/api/generate", "top_p=2"))
    assert (r.code, r.reason, r.body) == (500, "Internal Server Error", b"top_p must be in (0, 1]")
    r = srv.handle(_post("/api/stream", "top_p=2"))
    assert r.code == 500
    assert logs[-1] == "request failed: top_p must be in (0, 1]"


def test_stream_route_chunks():
    srv, logs = _srv()
    r = srv.handle(_post("/api/stream", "text=abc&stream_chunk_frames=3&wav_gain=2&left_context_frames=4"))
    assert r.code == 200
    h = dict(r.headers)
    assert (h["Content-Type"], h["X-TTS-Sample-Rate"], h["X-TTS-Sample-Format"]) == ("application/octet-stream", "24000", "s16le")
    assert (h["X-TTS-Chunk-Frames"], h["X-TTS-Text-Lookahead-Tokens"], h["X-TTS-Left-Context-Frames"]) == ("3", "8", "4")
    (_, text, o, so), = srv.engine.calls
    assert text == "abc" and so.left_context_frames == 4 and so.text_lookahead_tokens == 8
    chunks = list(r.chunks)
    ref = FakeStream(7, 3)
    want = []
    while (c := ref.next_audio_chunk(3)) is not None:
        want.append(pcm_s16le(c.samples, 2.0))
    assert chunks == want and [len(c) for c in chunks] == [2 * 3 * SPF, 2 * 3 * SPF, 2 * SPF]
    assert srv.engine.streams[0].closed
    r.on_done()
    assert logs[-1].startswith("streamed: voice_clone=false, frames=7, samples=13440, ended_by_eos=true")


def test_pcm_conversion_matches_the_reference_cast():
    """(sample * gain) clamped to [-1, 1], times i16::MAX, truncated (tts-server.rs:571-579)."""
    x = np.array([0.0, 1.0, -1.0, 2.0, -3.0, 0.5, -0.5, 1e-6, np.nan, 0.99999], np.float32)
    got = np.frombuffer(pcm_s16le(x, 1.0), "<i2")
    assert got.tolist() == [0, 32767, -32767, 32767, -32767, 16383, -16383, 0, 0, 32766]


# ------------------------------------------------------------------------------------- sockets
@pytest.fixture()
def live():
    srv, logs = _srv()
    sock = S.listen("127.0.0.1:0")
    port = sock.getsockname()[1]
    t = threading.Thread(target=srv.serve_forever, args=(sock,), daemon=True)
    t.start()
    yield srv, port
    sock.close()
    # wake the accept so the thread sees the closed listener
    try:
        http.client.HTTPConnection("127.0.0.1", port, timeout=1).request("GET", "/health")
    except OSError:
        pass
    t.join(timeout=5)


def test_live_socket_round_trip(live):
    srv, port = live
    c = http.client.HTTPConnection("127.0.0.1", port, timeout=10)
    c.request("GET", "/health")
    r = c.getresponse()
    assert (r.status, r.read(), r.getheader("Connection")) == (200, b"ok\n", "close")
    c = http.client.HTTPConnection("127.0.0.1", port, timeout=10)
    c.request("POST", "/api/generate", body="text=Hi&max_frames=3", headers={"Content-Type": S.FORM_TYPE})
    r = c.getresponse()
    body = r.read()
    assert r.status == 200 and body[:4] == b"RIFF" and r.getheader("X-TTS-Frames") == "3"
    assert struct.unpack("<I", body[40:44])[0] == 2 * 3 * SPF == len(body) - 44
    c = http.client.HTTPConnection("127.0.0.1", port, timeout=10)
    c.request("POST", "/api/stream", body="text=abc&stream_chunk_frames=2", headers={"Content-Type": S.FORM_TYPE})
    r = c.getresponse()
    assert r.status == 200 and r.getheader("Transfer-Encoding") == "chunked"
    pcm = r.read()  # http.client joins the chunks
    ref = FakeStream(7, 3)
    want = b""
    while (ch := ref.next_audio_chunk(2)) is not None:
        want += pcm_s16le(ch.samples, 1.0)
    assert pcm == want
    import socket
    with socket.create_connection(("127.0.0.1", port), timeout=10) as raw:  # declared body over 64 KiB
        raw.sendall(b"POST /api/generate HTTP/1.1\r\nContent-Length: 65537\r\n\r\n")
        got = b""
        while chunk := raw.recv(4096):
            got += chunk
    assert got.startswith(b"HTTP/1.1 500 Internal Server Error\r\n") and got.endswith(b"request body is too large")


class _DroppingConn:
    """A connection whose client goes away after `ok_sends` sendall calls."""

    def __init__(self, request: bytes, ok_sends: int):
        self.request, self.ok_sends, self.sent = request, ok_sends, []

    def recv(self, n):
        data, self.request = self.request[:n], self.request[n:]
        return data

    def sendall(self, data):
        if len(self.sent) >= self.ok_sends:
            raise BrokenPipeError("client went away")
        self.sent.append(data)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False


@pytest.mark.parametrize("ok_sends", [0, 1, 2])
def test_stream_closed_when_client_disconnects(ok_sends):
    """A client that disconnects mid-stream (sendall raises after the head, after one chunk,
    ...) must not leave the engine stream open until garbage collection: the server closes
    the PCM generator, which closes the stream (its slot is free for the next request)."""
    srv, logs = _srv()
    body = b"text=abc&stream_chunk_frames=2"
    raw = (b"POST /api/stream HTTP/1.1\r\nHost: x\r\nContent-Type: " + S.FORM_TYPE.encode() +
           b"\r\nContent-Length: " + str(len(body)).encode() + b"\r\n\r\n" + body)
    conn = _DroppingConn(raw, ok_sends)
    keep = []  # a lingering reference to the generator must not keep the stream open
    orig = srv.handle

    def handle(req):
        r = orig(req)
        keep.append(r.chunks)
        return r
    srv.handle = handle
    srv.serve_connection(conn)
    assert len(conn.sent) == ok_sends
    assert any(l.startswith("request failed:") for l in logs)
    # the stream starts before the head is sent (start errors are answered with a status):
    # it must be closed now, also when no chunk was ever pulled (ok_sends = 0)
    assert len(srv.engine.streams) == 1 and srv.engine.streams[0].closed
    assert not any(l.startswith("streamed:") for l in logs)
