"""HTTP serving surface over ``HipTtsEngine``: the reference's ``tts-server`` binary
(src/bin/tts-server.rs) with the same routes, form fields, defaults, limits, status codes,
response headers and wire formats.

    python -m q3t.server <model_dir> [bind_addr] [max_cache_frames] [voice_clone_prompt_json]

Routes (tts-server.rs:104-116):

* ``GET /``: a small HTML page with a form for the two POST routes;
* ``GET /health``: ``ok``;
* ``GET /favicon.ico``: 204;
* ``POST /api/generate``: one WAV (16-bit PCM, 24 kHz, mono) plus ``X-TTS-*`` timing and
  option headers (tts-server.rs:118-242);
* ``POST /api/stream``: chunked transfer of raw little-endian int16 PCM, one HTTP chunk per
  ``next_audio_chunk`` (tts-server.rs:244-321);
* anything else: 404.

POST bodies are ``application/x-www-form-urlencoded`` (415 otherwise).  A field that does not
parse, or a value outside its range, is a 400 whose body is the message; an error raised by
the engine afterwards is a 500 (tts-server.rs:92-101, 483-496).  Requests are limited to 64 KiB
and served one connection at a time, in accept order, as the reference does: one engine, one
GPU stream of work.

The request layer (``parse_request_bytes``, ``parse_form``, ``parse_generation_request``,
``TtsServer.handle``) never touches the GPU, so its behaviour is tested on the CPU with a
stand-in engine; the GPU tests run the real engine behind a live socket.
"""
from __future__ import annotations

import dataclasses
import html
import re
import socket
import sys
import time
from typing import Callable, Dict, Iterator, List, Optional, Sequence, Tuple, Union

import numpy as np

from .engine import (DEFAULT_STREAM_LEFT_CONTEXT_FRAMES, DEFAULT_TEXT_LOOKAHEAD_TOKENS, SAMPLE_RATE,
                     GeneratedSpeech, GenerateOptions, InvalidInputError, StreamOptions, parse_language,
                     parse_speaker)
from .wav import pcm_s16le, wav_bytes

DEFAULT_BIND = "127.0.0.1:8080"          # tts-server.rs:15-18
DEFAULT_MAX_CACHE_FRAMES = 240
DEFAULT_STREAM_CHUNK_FRAMES = 6
MAX_REQUEST_BYTES = 64 * 1024
DEFAULT_TEXT = "She said she would be here by noon."
FORM_TYPE = "application/x-www-form-urlencoded"


class BadRequest(ValueError):
    """``Error::InvalidInput`` raised while reading or parsing a request (a 400, or a dropped
    connection when the request itself cannot be read)."""


# ---------------------------------------------------------------------------------------------
# Value parsers with the grammar of Rust's ``str::parse`` for the reference's field types
# (tts-server.rs:1031-1060): no surrounding whitespace, no digit separators.
# ---------------------------------------------------------------------------------------------
_UINT = re.compile(r"\+?[0-9]+")
_FLOAT = re.compile(r"[+-]?(inf|infinity|nan|([0-9]+\.?[0-9]*|\.[0-9]+)(e[+-]?[0-9]+)?)", re.IGNORECASE)


def parse_uint(value: str, name: str, bits: int = 64) -> int:
    """``usize`` / ``u64``: decimal digits with an optional ``+``, below 2**bits."""
    if not _UINT.fullmatch(value):
        raise BadRequest(f"invalid {name}: {value!r}")
    v = int(value)
    if v >= 1 << bits:
        raise BadRequest(f"invalid {name}: number too large to fit in target type")
    return v


def parse_f32(value: str, name: str) -> float:
    """``f32``: decimal or exponent form, ``inf`` / ``infinity`` / ``nan`` in any case; the
    nearest float32 (overflow gives an infinity, as Rust's parser does)."""
    if not _FLOAT.fullmatch(value):
        raise BadRequest(f"invalid {name}: {value!r}")
    with np.errstate(over="ignore"):
        return float(np.float32(float(value)))


def parse_bool(value: str, name: str) -> bool:
    v = value.lower()
    if v in ("1", "true", "yes", "on"):
        return True
    if v in ("0", "false", "no", "off"):
        return False
    raise BadRequest(f"invalid {name}: {v}")


def _hex(c: int) -> int:
    if 0x30 <= c <= 0x39:
        return c - 0x30
    if 0x61 <= c <= 0x66:
        return c - 0x61 + 10
    if 0x41 <= c <= 0x46:
        return c - 0x41 + 10
    raise BadRequest("invalid percent escape")


def percent_decode(value: str) -> str:
    """``+`` is a space and ``%XY`` a byte (tts-server.rs:981-1021); a ``%`` without two
    following characters stays as it is; a non-hex digit in an escape is an error; the decoded
    bytes must be UTF-8."""
    raw = value.encode("utf-8")
    out = bytearray()
    i = 0
    while i < len(raw):
        b = raw[i]
        if b == 0x2B:  # '+'
            out.append(0x20)
            i += 1
        elif b == 0x25 and i + 2 < len(raw):  # '%'
            out.append((_hex(raw[i + 1]) << 4) | _hex(raw[i + 2]))
            i += 3
        else:
            out.append(b)
            i += 1
    try:
        return out.decode("utf-8")
    except UnicodeDecodeError as err:
        raise BadRequest(f"form value is not UTF-8: {err}") from None


def parse_form(body: bytes) -> Dict[str, str]:
    """``key=value`` pairs split on ``&``; a pair without ``=`` has an empty value; a repeated
    key keeps its last value (tts-server.rs:968-979)."""
    try:
        text = body.decode("utf-8")
    except UnicodeDecodeError as err:
        raise BadRequest(f"form body is not UTF-8: {err}") from None
    form: Dict[str, str] = {}
    for pair in text.split("&"):
        if not pair:
            continue
        key, _, value = pair.partition("=")
        form[percent_decode(key)] = percent_decode(value)
    return form


# ---------------------------------------------------------------------------------------------
# HTTP framing
# ---------------------------------------------------------------------------------------------
@dataclasses.dataclass
class Request:
    method: str
    path: str
    headers: Dict[str, str]
    body: bytes


@dataclasses.dataclass
class Response:
    code: int
    reason: str
    headers: List[Tuple[str, str]]
    body: bytes = b""
    # A streamed response: chunked transfer of each item (empty items are skipped).
    chunks: Optional[Iterator[bytes]] = None
    # Called after the last byte is written (the reference's per-request log line).
    on_done: Optional[Callable[[], None]] = None


def text_response(code: int, reason: str, text: str) -> Response:
    return Response(code, reason, [("Content-Type", "text/plain; charset=utf-8")], text.encode("utf-8"))


def _header_end(buf: bytes) -> int:
    return buf.find(b"\r\n\r\n")


def parse_request_bytes(read: Callable[[], bytes]) -> Request:
    """Read one request with ``read()`` (returns b"" at end of stream), as ``read_request``
    (tts-server.rs:581-652): headers within 64 KiB, a Content-Length body of at most 64 KiB,
    the path without its query string, header names lower-cased."""
    buf = b""
    while True:
        data = read()
        if not data:
            raise BadRequest("connection closed")
        buf += data
        if len(buf) > MAX_REQUEST_BYTES:
            raise BadRequest("request is too large")
        end = _header_end(buf)
        if end >= 0:
            break
    try:
        head = buf[:end].decode("utf-8")
    except UnicodeDecodeError as err:
        raise BadRequest(f"invalid HTTP headers: {err}") from None
    lines = head.split("\r\n")
    parts = lines[0].split()
    if not parts:
        raise BadRequest("missing method")
    if len(parts) < 2:
        raise BadRequest("missing path")
    method, path = parts[0], parts[1].split("?")[0]
    headers: Dict[str, str] = {}
    for line in lines[1:]:
        name, sep, value = line.partition(":")
        if sep:
            headers[name.strip().lower()] = value.strip()
    length = parse_uint(headers["content-length"], "content-length") if "content-length" in headers else 0
    if length > MAX_REQUEST_BYTES:
        raise BadRequest("request body is too large")
    start = end + 4
    while len(buf) < start + length:
        data = read()
        if not data:
            raise BadRequest("truncated request body")
        buf += data
        if len(buf) > start + MAX_REQUEST_BYTES:
            raise BadRequest("request is too large")
    return Request(method, path, headers, buf[start:start + length])


def _sanitize(value: str) -> str:
    return value.replace("\r", " ").replace("\n", " ")


def response_head(resp: Response) -> bytes:
    lines = [f"HTTP/1.1 {resp.code} {resp.reason}"]
    if resp.chunks is not None:
        lines.append("Transfer-Encoding: chunked")
    else:
        lines.append(f"Content-Length: {len(resp.body)}")
    lines.append("Connection: close")
    lines += [f"{name}: {_sanitize(value)}" for name, value in resp.headers]
    return ("\r\n".join(lines) + "\r\n\r\n").encode("utf-8")


def chunk_frame(data: bytes) -> bytes:
    """One chunk of a chunked transfer: hex length, CRLF, data, CRLF (empty data: nothing)."""
    return f"{len(data):x}\r\n".encode("ascii") + data + b"\r\n" if data else b""


CHUNKED_END = b"0\r\n\r\n"


# ---------------------------------------------------------------------------------------------
# Generation requests
# ---------------------------------------------------------------------------------------------
@dataclasses.dataclass
class GenerationRequest:
    text: str
    options: GenerateOptions
    stream_options: StreamOptions
    wav_gain: float
    stream_chunk_frames: int
    use_voice_clone: bool


def parse_generation_request(form: Dict[str, str], max_cache_frames: int,
                             has_voice_clone_prompt: bool) -> GenerationRequest:
    """The form fields, defaults and checks of ``parse_generation_request``
    (tts-server.rs:323-481).  Ranges the reference leaves to the engine (top_p, temperature,
    ...) are checked by the engine, and their errors are 500s there and here."""

    def get(name, parse, default):
        return parse(form[name], name) if name in form else default

    text = form.get("text", DEFAULT_TEXT).strip()
    if not text:
        raise BadRequest("text must not be empty")
    max_frames = get("max_frames", parse_uint, 120)
    if max_frames == 0 or max_frames > max_cache_frames:
        raise BadRequest(f"max_frames must be in 1..={max_cache_frames} for this server")
    speaker = form.get("speaker", "ryan")
    language = form.get("language", "english")
    for value, check in ((speaker, parse_speaker), (language, parse_language)):
        try:
            check(value)
        except InvalidInputError as err:
            raise BadRequest(str(err)) from None
    wav_gain = get("wav_gain", parse_f32, 1.0)
    repetition_penalty = get("repetition_penalty", parse_f32, float(np.float32(1.05)))
    if repetition_penalty <= 0.0:  # NaN passes here and is left to the engine, as in the reference
        raise BadRequest("repetition_penalty must be positive")
    opts = GenerateOptions(
        speaker=speaker, language=language, max_frames=max_frames, decode_audio=False,
        do_sample=get("do_sample", parse_bool, True),
        top_k=get("top_k", parse_uint, 50),
        top_p=get("top_p", parse_f32, 1.0),
        temperature=get("temperature", parse_f32, float(np.float32(0.9))),
        repetition_penalty=repetition_penalty,
        subtalker_dosample=get("subtalker_dosample", parse_bool, True),
        subtalker_top_k=get("subtalker_top_k", parse_uint, 50),
        subtalker_top_p=get("subtalker_top_p", parse_f32, 1.0),
        subtalker_temperature=get("subtalker_temperature", parse_f32, float(np.float32(0.9))),
        seed=get("seed", parse_uint, 0))
    lookahead = get("text_lookahead_tokens", parse_uint, DEFAULT_TEXT_LOOKAHEAD_TOKENS)
    if lookahead == 0:
        raise BadRequest("text_lookahead_tokens must be non-zero")
    chunk_frames = get("stream_chunk_frames", parse_uint, DEFAULT_STREAM_CHUNK_FRAMES)
    if chunk_frames == 0:
        raise BadRequest("stream_chunk_frames must be non-zero")
    left = get("left_context_frames", parse_uint, DEFAULT_STREAM_LEFT_CONTEXT_FRAMES)
    use_vc = get("use_voice_clone", parse_bool, False)
    if use_vc and not has_voice_clone_prompt:
        raise BadRequest("voice clone mode requires starting the server with voice_clone_prompt_json")
    return GenerationRequest(text, opts, StreamOptions(text_lookahead_tokens=lookahead, left_context_frames=left),
                             wav_gain, chunk_frames, use_vc)


def format_seconds(value: float) -> str:
    return f"{value:.6f}"


def _bool(v: bool) -> str:
    return "true" if v else "false"


def rtf(seconds: float, audio_seconds: float) -> float:
    return seconds / audio_seconds if audio_seconds > 0.0 else 0.0


# ---------------------------------------------------------------------------------------------
# The server
# ---------------------------------------------------------------------------------------------
class TtsServer:
    """Routes requests to an engine with the ``HipTtsEngine`` generation API:
    ``generate_codes``, ``generate_voice_clone_codes``, ``decode_codes``, ``start_stream`` and
    ``start_voice_clone_stream`` (whose streams have ``next_audio_chunk`` and ``close``)."""

    def __init__(self, engine, max_cache_frames: int = DEFAULT_MAX_CACHE_FRAMES, voice_clone_prompt=None,
                 load_seconds: float = 0.0, log: Callable[[str], None] = print):
        if max_cache_frames <= 0:
            raise ValueError("max_cache_frames must be non-zero")
        self.engine = engine
        self.max_cache_frames = int(max_cache_frames)
        self.voice_clone_prompt = voice_clone_prompt
        self.load_seconds = float(load_seconds)
        self.log = log

    # -- routing ---------------------------------------------------------------------------
    def handle(self, req: Request) -> Response:
        """One request -> one response; an engine error becomes a 500 with its message."""
        try:
            route = (req.method, req.path)
            if route == ("GET", "/"):
                return Response(200, "OK", [("Content-Type", "text/html; charset=utf-8"),
                                            ("Cache-Control", "no-store")], self.index_html().encode("utf-8"))
            if route == ("GET", "/health"):
                return text_response(200, "OK", "ok\n")
            if route == ("GET", "/favicon.ico"):
                return Response(204, "No Content", [])
            if route == ("POST", "/api/generate"):
                return self._post(req, self._generate)
            if route == ("POST", "/api/stream"):
                return self._post(req, self._stream)
            return text_response(404, "Not Found", "not found\n")
        except Exception as err:  # tts-server.rs:92-97
            self.log(f"request failed: {err}")
            return text_response(500, "Internal Server Error", str(err))

    def _post(self, req: Request, run) -> Response:
        if not req.headers.get("content-type", "").startswith(FORM_TYPE):
            return text_response(415, "Unsupported Media Type", f"expected {FORM_TYPE}\n")
        try:
            g = parse_generation_request(parse_form(req.body), self.max_cache_frames,
                                         self.voice_clone_prompt is not None)
        except BadRequest as err:
            return text_response(400, "Bad Request", f"{err}\n")
        return run(g)

    # -- POST /api/generate ----------------------------------------------------------------
    def _generate(self, g: GenerationRequest) -> Response:
        o = g.options
        t0 = time.perf_counter()
        if g.use_voice_clone:
            codes = self.engine.generate_voice_clone_codes(g.text, self.voice_clone_prompt, o)
        else:
            codes = self.engine.generate_codes(g.text, o)
        generation_seconds = time.perf_counter() - t0
        t1 = time.perf_counter()
        samples = self.engine.decode_codes(codes.codes)
        decode_seconds = time.perf_counter() - t1
        t2 = time.perf_counter()
        speech = GeneratedSpeech(g.text, codes.frames, codes.ended_by_eos, codes.codes,
                                 np.asarray(samples, np.float32), SAMPLE_RATE)
        wav = wav_bytes(speech.samples, SAMPLE_RATE, g.wav_gain)
        wav_seconds = time.perf_counter() - t2
        first_audio = time.perf_counter() - t0
        audio_seconds = speech.audio_seconds()
        inference = generation_seconds + decode_seconds
        self.log(f"generated: voice_clone={_bool(g.use_voice_clone)}, frames={speech.frames}, "
                 f"samples={speech.samples.size}, ended_by_eos={_bool(speech.ended_by_eos)}, "
                 f"time_to_first_audio_seconds={first_audio:.6f}, generation_seconds={generation_seconds:.6f}, "
                 f"decode_seconds={decode_seconds:.6f}, wav_seconds={wav_seconds:.6f}, "
                 f"audio_seconds={audio_seconds:.6f}, inference_rtf={rtf(inference, audio_seconds):.6f}")
        headers = [
            ("Content-Type", "audio/wav"),
            ("Cache-Control", "no-store"),
            ("X-TTS-Load-Seconds", format_seconds(self.load_seconds)),
            ("X-TTS-Generation-Seconds", format_seconds(generation_seconds)),
            ("X-TTS-Decode-Seconds", format_seconds(decode_seconds)),
            ("X-TTS-Wav-Seconds", format_seconds(wav_seconds)),
            ("X-TTS-Time-To-First-Audio-Seconds", format_seconds(first_audio)),
            ("X-TTS-Inference-Seconds", format_seconds(inference)),
            ("X-TTS-Audio-Seconds", format_seconds(audio_seconds)),
            ("X-TTS-Generation-RTF", format_seconds(rtf(generation_seconds, audio_seconds))),
            ("X-TTS-Decode-RTF", format_seconds(rtf(decode_seconds, audio_seconds))),
            ("X-TTS-Inference-RTF", format_seconds(rtf(inference, audio_seconds))),
            ("X-TTS-Frames", str(speech.frames)),
            ("X-TTS-Samples", str(speech.samples.size)),
            ("X-TTS-Ended-By-EOS", _bool(speech.ended_by_eos)),
            ("X-TTS-Voice-Clone", _bool(g.use_voice_clone)),
            ("X-TTS-Repetition-Penalty", format_seconds(o.repetition_penalty)),
            ("X-TTS-Do-Sample", _bool(o.do_sample)),
            ("X-TTS-Top-K", str(o.top_k)),
            ("X-TTS-Top-P", format_seconds(o.top_p)),
            ("X-TTS-Temperature", format_seconds(o.temperature)),
            ("X-TTS-Subtalker-Do-Sample", _bool(o.subtalker_dosample)),
            ("X-TTS-Subtalker-Top-K", str(o.subtalker_top_k)),
            ("X-TTS-Subtalker-Top-P", format_seconds(o.subtalker_top_p)),
            ("X-TTS-Subtalker-Temperature", format_seconds(o.subtalker_temperature)),
            ("X-TTS-Seed", str(o.seed)),
        ]
        return Response(200, "OK", headers, wav)

    # -- POST /api/stream ------------------------------------------------------------------
    def _stream(self, g: GenerationRequest) -> Response:
        t0 = time.perf_counter()
        if g.use_voice_clone:
            st = self.engine.start_voice_clone_stream(g.text, self.voice_clone_prompt, g.options, g.stream_options)
        else:
            st = self.engine.start_stream(g.text, g.options, g.stream_options)
        stats = {"samples": 0, "frames": 0, "eos": False, "first": None}

        def pcm() -> Iterator[bytes]:
            try:
                while True:
                    chunk = st.next_audio_chunk(g.stream_chunk_frames)
                    if chunk is None:
                        return
                    if stats["first"] is None and chunk.samples.size:
                        stats["first"] = time.perf_counter() - t0
                    stats["samples"] += int(chunk.samples.size)
                    stats["frames"] = int(chunk.total_frames)
                    stats["eos"] = bool(chunk.ended_by_eos)
                    yield pcm_s16le(chunk.samples, g.wav_gain)
            finally:
                st.close()

        def done() -> None:
            seconds = time.perf_counter() - t0
            audio = stats["samples"] / SAMPLE_RATE
            first = "n/a" if stats["first"] is None else format_seconds(stats["first"])
            self.log(f"streamed: voice_clone={_bool(g.use_voice_clone)}, frames={stats['frames']}, "
                     f"samples={stats['samples']}, ended_by_eos={_bool(stats['eos'])}, "
                     f"time_to_first_audio_seconds={first}, seconds={seconds:.6f}, audio_seconds={audio:.6f}, "
                     f"rtf={rtf(seconds, audio):.6f}")

        headers = [
            ("Content-Type", "application/octet-stream"),
            ("Cache-Control", "no-store"),
            ("X-TTS-Sample-Rate", str(SAMPLE_RATE)),
            ("X-TTS-Sample-Format", "s16le"),
            ("X-TTS-Chunk-Frames", str(g.stream_chunk_frames)),
            ("X-TTS-Text-Lookahead-Tokens", str(g.stream_options.text_lookahead_tokens)),
            ("X-TTS-Left-Context-Frames", str(g.stream_options.left_context_frames)),
            ("X-TTS-Voice-Clone", _bool(g.use_voice_clone)),
        ]
        return Response(200, "OK", headers, chunks=_StreamChunks(pcm(), st), on_done=done)

    # -- GET / -----------------------------------------------------------------------------
    def index_html(self) -> str:
        """A form over both POST routes; the stream route's PCM is played as it arrives."""
        vc = self.voice_clone_prompt is not None
        return _INDEX.format(load=f"{self.load_seconds:.3f}", cap=self.max_cache_frames, rate=SAMPLE_RATE,
                             vc="loaded" if vc else "none", vc_disabled="" if vc else " disabled",
                             chunk=DEFAULT_STREAM_CHUNK_FRAMES, lookahead=DEFAULT_TEXT_LOOKAHEAD_TOKENS,
                             left=DEFAULT_STREAM_LEFT_CONTEXT_FRAMES, text=html.escape(DEFAULT_TEXT))

    # -- sockets ---------------------------------------------------------------------------
    def serve_connection(self, conn: socket.socket) -> None:
        """Read one request, write its response, close (``Connection: close``)."""
        with conn:
            try:
                req = parse_request_bytes(lambda: conn.recv(4096))
            except BadRequest as err:  # the reference answers an unreadable request with a 500
                self.log(f"request failed: {err}")
                _send_all(conn, response_head(text_response(500, "Internal Server Error", str(err))) +
                          str(err).encode("utf-8"))
                return
            resp = self.handle(req)
            if resp.chunks is None:
                _send_all(conn, response_head(resp) + resp.body)
                return
            try:
                conn.sendall(response_head(resp))
                for data in resp.chunks:
                    if data:
                        conn.sendall(chunk_frame(data))
                conn.sendall(CHUNKED_END)
            except Exception as err:  # headers already sent: the connection just ends
                self.log(f"request failed: {err}")
                return
            finally:
                # A client that went away leaves the generator suspended mid-stream: close it
                # here, so its engine stream (and the slot it holds) is released now rather
                # than whenever the generator is garbage-collected.
                close = getattr(resp.chunks, "close", None)
                if close is not None:
                    close()
            if resp.on_done:
                resp.on_done()

    def serve_forever(self, listener: socket.socket, max_requests: Optional[int] = None) -> None:
        """Accept and serve connections one at a time (``max_requests``: stop after that many)."""
        served = 0
        while max_requests is None or served < max_requests:
            try:
                conn, _ = listener.accept()
            except OSError as err:
                if listener.fileno() < 0:
                    return
                self.log(f"accept failed: {err}")
                continue
            self.serve_connection(conn)
            served += 1


class _StreamChunks:
    """The PCM chunks of an engine stream.  ``close()`` ends the generator and closes the
    stream even when the generator never started (the response head could not be sent):
    the stream was started before the head, so its slot must not wait for the garbage
    collector."""

    def __init__(self, gen: Iterator[bytes], stream) -> None:
        self._gen, self._stream = gen, stream

    def __iter__(self) -> Iterator[bytes]:
        return self._gen

    def close(self) -> None:
        try:
            self._gen.close()
        finally:
            self._stream.close()


def _send_all(conn: socket.socket, data: bytes) -> None:
    try:
        conn.sendall(data)
    except OSError:
        pass


def listen(bind: str) -> socket.socket:
    host, _, port = bind.rpartition(":")
    sock = socket.socket(socket.AF_INET6 if ":" in host.strip("[]") else socket.AF_INET, socket.SOCK_STREAM)
    sock.setsockopt(socket.SOL_SOCKET, socket.SO_REUSEADDR, 1)
    sock.bind((host.strip("[]"), int(port)))
    sock.listen(16)
    return sock


def main(argv: Sequence[str]) -> int:
    """``tts-server`` main (tts-server.rs:43-102)."""
    from .engine import HipTtsEngine
    from .voice_clone import VoiceClonePrompt

    if not argv:
        print("usage: python -m q3t.server <model_dir> [bind_addr] [max_cache_frames] [voice_clone_prompt_json]",
              file=sys.stderr)
        return 2
    model_dir = argv[0]
    bind = argv[1] if len(argv) > 1 else DEFAULT_BIND
    max_frames = parse_uint(argv[2], "max_cache_frames") if len(argv) > 2 else DEFAULT_MAX_CACHE_FRAMES
    if max_frames == 0:
        print("max_cache_frames must be non-zero", file=sys.stderr)
        return 2
    prompt_path = argv[3] if len(argv) > 3 else None
    prompt = VoiceClonePrompt.from_json(prompt_path) if prompt_path else None
    t0 = time.perf_counter()
    engine = HipTtsEngine.load_with_max_frames(model_dir, 0, max_frames)
    engine.synchronize()
    load_seconds = time.perf_counter() - t0
    server = TtsServer(engine, max_frames, prompt, load_seconds)
    listener = listen(bind)
    print(f"TTS server listening on http://{bind}/, model_dir={model_dir}, load_seconds={load_seconds:.6f}, "
          f"max_cache_frames={max_frames}, voice_clone_prompt={prompt_path or 'none'}", flush=True)
    try:
        server.serve_forever(listener)
    finally:
        listener.close()
        engine.close()
    return 0


_INDEX = """<!doctype html>
<html lang="en"><head><meta charset="utf-8"><title>q3t TTS server</title>
<style>
body {{ font-family: sans-serif; max-width: 48rem; margin: 2rem auto; padding: 0 1rem; }}
fieldset {{ display: flex; flex-wrap: wrap; gap: .75rem; border: 1px solid #bbb; }}
label {{ display: flex; flex-direction: column; font-size: .85rem; }}
textarea {{ width: 100%; min-height: 5rem; }}
pre {{ background: #f4f4f4; padding: .75rem; overflow-x: auto; }}
</style></head><body>
<h1>q3t TTS server</h1>
<p>Model load {load} s &middot; max frames {cap} &middot; {rate} Hz &middot; voice clone prompt: {vc}</p>
<form id="f">
<textarea name="text">{text}</textarea>
<fieldset><legend>Generation</legend>
<label>Route<select id="route"><option value="generate">WAV (/api/generate)</option>
<option value="stream">PCM stream (/api/stream)</option></select></label>
<label>Frames<input name="max_frames" type="number" min="1" max="{cap}" value="120"></label>
<label>Speaker<input name="speaker" value="Ryan"></label>
<label>Language<input name="language" value="English"></label>
<label>Voice<select name="use_voice_clone"><option value="false">speaker</option>
<option value="true"{vc_disabled}>voice clone prompt</option></select></label>
<label>Gain<input name="wav_gain" type="number" step="0.1" value="1.0"></label>
<label>Seed<input name="seed" type="number" min="0" value="0"></label>
</fieldset>
<fieldset><legend>Sampling (semantic / acoustic)</legend>
<label>Sample<select name="do_sample"><option>true</option><option>false</option></select></label>
<label>Top k<input name="top_k" type="number" min="0" value="50"></label>
<label>Top p<input name="top_p" type="number" step="0.01" value="1.0"></label>
<label>Temperature<input name="temperature" type="number" step="0.01" value="0.9"></label>
<label>Repetition penalty<input name="repetition_penalty" type="number" step="0.01" value="1.05"></label>
<label>Sample<select name="subtalker_dosample"><option>true</option><option>false</option></select></label>
<label>Top k<input name="subtalker_top_k" type="number" min="0" value="50"></label>
<label>Top p<input name="subtalker_top_p" type="number" step="0.01" value="1.0"></label>
<label>Temperature<input name="subtalker_temperature" type="number" step="0.01" value="0.9"></label>
</fieldset>
<fieldset><legend>Streaming</legend>
<label>Chunk frames<input name="stream_chunk_frames" type="number" min="1" value="{chunk}"></label>
<label>Text lookahead<input name="text_lookahead_tokens" type="number" min="1" value="{lookahead}"></label>
<label>Left context frames<input name="left_context_frames" type="number" min="0" value="{left}"></label>
</fieldset>
<p><button>Run</button></p></form>
<audio id="a" controls></audio><pre id="s"></pre>
<script>
const f = document.getElementById('f'), out = document.getElementById('s');
f.addEventListener('submit', async (ev) => {{
  ev.preventDefault();
  const route = document.getElementById('route').value, t0 = performance.now();
  const r = await fetch('/api/' + route, {{ method: 'POST', body: new URLSearchParams(new FormData(f)),
    headers: {{ 'Content-Type': 'application/x-www-form-urlencoded' }} }});
  if (!r.ok) {{ out.textContent = await r.text(); return; }}
  if (route === 'generate') {{
    document.getElementById('a').src = URL.createObjectURL(await r.blob());
    const h = {{}}; r.headers.forEach((v, k) => {{ if (k.startsWith('x-tts-')) h[k] = v; }});
    out.textContent = JSON.stringify(h, null, 1);
    return;
  }}
  const ctx = new AudioContext(), rd = r.body.getReader();
  let carry = new Uint8Array(0), at = ctx.currentTime + 0.05, n = 0;
  for (;;) {{
    const {{ done, value }} = await rd.read();
    if (done) break;
    const b = new Uint8Array(carry.length + value.length); b.set(carry); b.set(value, carry.length);
    const m = b.length >> 1; carry = b.slice(2 * m);
    if (!m) continue;
    const dv = new DataView(b.buffer, 0, 2 * m), x = new Float32Array(m);
    for (let i = 0; i < m; i++) x[i] = dv.getInt16(2 * i, true) / 32768;
    const buf = ctx.createBuffer(1, m, {rate}); buf.copyToChannel(x, 0);
    const src = ctx.createBufferSource(); src.buffer = buf; src.connect(ctx.destination);
    at = Math.max(at, ctx.currentTime + 0.02); src.start(at); at += buf.duration; n += m;
    out.textContent = 'samples ' + n + ', first audio after ' + ((performance.now() - t0) / 1000).toFixed(3) + ' s';
  }}
}});
</script></body></html>
"""

if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
