"""Python mirror of the reference crate's engine API, over the q3t C ABI (include/q3t.h).

Names, defaults, argument meaning and error behaviour follow src/generation.rs of
piedshag/qwen3-tts-hip:

=========================================  =============================================
reference (Rust)                            here
=========================================  =============================================
``HipTtsEngine::load`` / ``load_with_max_   ``HipTtsEngine.load`` / ``load_with_max_frames``
frames`` / ``load_with_options`` (255-315)  / ``load_with_options``
``generate_codes`` (356-371)                ``HipTtsEngine.generate_codes``
``start_stream`` (421-440)                  ``HipTtsEngine.start_stream``
``generate_voice_clone[_codes]`` (334-393)  ``HipTtsEngine.generate_voice_clone[_codes]``
``start_voice_clone_stream`` (442-462)      ``HipTtsEngine.start_voice_clone_stream``
``start_[voice_clone_]text_stream[_polling]`` ``HipTtsEngine.start_[voice_clone_]text_stream[_polling]``
(463-511), ``PollingTextStream``,           (:mod:`q3t.text_stream`)
``HipTextStream``, ``TextStreamInput``
``HipTtsStream::next_codes_chunk`` (876-)   ``HipTtsStream.next_codes_chunk``
``HipTtsStream::finish_codes`` (991-997)    ``HipTtsStream.finish_codes``
``GenerateOptions`` / ``StreamOptions``     same names, same defaults (40-92)
``Error::InvalidInput`` / ``Error::Hip``    ``InvalidInputError`` / ``HipError``
=========================================  =============================================

The generation calls take text (tokenized with the model directory's tokenizer files, as
the reference does), a sequence of content token ids (prepared on the device, or by a
:class:`q3t.textprep.TextPrep` given to the engine), or a
:class:`q3t.textprep.PreparedInputs` (the reference's ``TtsPreparedInputs``).

There is no CPU fallback: if ``libq3t.so`` is missing or the GPU call fails, the call
raises.
"""
from __future__ import annotations

import ctypes
import dataclasses
import os
from typing import List, Optional, Sequence, Union

import numpy as np

from .textprep import PreparedInputs, TextPrep
from .voice_clone import VoiceClonePrompt

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libq3t.so")

DEFAULT_MAX_CACHE_STEPS = 512          # generation.rs:20
DEFAULT_PREFILL_HEADROOM = 256         # generation.rs:21
DEFAULT_STREAM_LEFT_CONTEXT_FRAMES = 25
DEFAULT_TEXT_LOOKAHEAD_TOKENS = 8
SAMPLE_RATE = 24_000
SAMPLES_PER_FRAME = 1920               # 80 ms per codec frame

Q3T_OK, Q3T_ERR_INVALID, Q3T_ERR_HIP, Q3T_ERR_CAPACITY, Q3T_ERR_NOT_FOUND, Q3T_ERR_BUSY = range(6)

SPEAKERS = ["serena", "vivian", "uncle_fu", "ryan", "aiden", "ono_anna", "sohee", "eric", "dylan"]
LANGUAGES = ["chinese", "english", "japanese", "korean", "german", "french", "russian",
             "portuguese", "spanish", "italian"]
_SPEAKER_ALIASES = {"unclefu": "uncle_fu", "onoanna": "ono_anna"}
_LANGUAGE_ALIASES = {"zh": "chinese", "en": "english", "ja": "japanese", "ko": "korean", "de": "german",
                     "fr": "french", "ru": "russian", "pt": "portuguese", "es": "spanish", "it": "italian"}


def parse_speaker(value: str) -> int:
    """``Speaker::from_str`` (text.rs:137-153): case-insensitive name -> the enum ordinal."""
    v = str(value).lower()
    v = _SPEAKER_ALIASES.get(v, v)
    if v not in SPEAKERS:
        raise InvalidInputError(Q3T_ERR_INVALID, f"unknown speaker {value}")
    return SPEAKERS.index(v)


def parse_language(value: str) -> int:
    """``Language::from_str`` (text.rs:75-93): case-insensitive name or ISO code -> ordinal."""
    v = str(value).lower()
    v = _LANGUAGE_ALIASES.get(v, v)
    if v not in LANGUAGES:
        raise InvalidInputError(Q3T_ERR_INVALID, f"unknown language {value}")
    return LANGUAGES.index(v)


class Q3tError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class InvalidInputError(Q3tError, ValueError):
    pass


class HipError(Q3tError):
    pass


class CapacityError(InvalidInputError):
    pass


class NotFoundError(InvalidInputError):
    pass


class BusyError(Q3tError):
    pass


_ERRORS = {Q3T_ERR_INVALID: InvalidInputError, Q3T_ERR_HIP: HipError, Q3T_ERR_CAPACITY: CapacityError,
           Q3T_ERR_NOT_FOUND: NotFoundError, Q3T_ERR_BUSY: BusyError}


class _EngineOptions(ctypes.Structure):
    _fields_ = [("model_dir", ctypes.c_char_p), ("device", ctypes.c_int32),
                ("max_cache_steps", ctypes.c_int32), ("max_streams", ctypes.c_int32),
                ("use_graph", ctypes.c_int32), ("kv_dtype", ctypes.c_int32)]


class _GenerateOptions(ctypes.Structure):
    _fields_ = [("speaker", ctypes.c_int32), ("language", ctypes.c_int32),
                ("max_frames", ctypes.c_int32), ("decode_audio", ctypes.c_int32),
                ("do_sample", ctypes.c_int32), ("top_k", ctypes.c_int32),
                ("top_p", ctypes.c_float), ("temperature", ctypes.c_float),
                ("repetition_penalty", ctypes.c_float), ("subtalker_dosample", ctypes.c_int32),
                ("subtalker_top_k", ctypes.c_int32), ("subtalker_top_p", ctypes.c_float),
                ("subtalker_temperature", ctypes.c_float), ("seed", ctypes.c_uint64),
                ("repetition_penalty_per_occurrence", ctypes.c_int32)]


class _EngineInfo(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "talker_hidden", "talker_intermediate", "talker_layers", "talker_vocab",
        "cp_hidden", "cp_intermediate", "cp_layers", "cp_vocab",
        "q_heads", "kv_heads", "head_dim", "num_code_groups",
        "codec_eos", "max_cache_steps", "max_streams")] + [("device_bytes", ctypes.c_int64),
                                                             ("text_vocab", ctypes.c_int32),
                                                             ("text_hidden", ctypes.c_int32),
                                                             ("samples_per_frame", ctypes.c_int32)]


class _ChunkInfo(ctypes.Structure):
    _fields_ = [("frames", ctypes.c_int32), ("total_frames", ctypes.c_int32),
                ("ended_by_eos", ctypes.c_int32)]


class _Profile(ctypes.Structure):
    _fields_ = [("upload_seconds", ctypes.c_double), ("prefill_seconds", ctypes.c_double),
                ("code_predictor_seconds", ctypes.c_double), ("talker_decode_seconds", ctypes.c_double)]


class _StreamInput(ctypes.Structure):
    _fields_ = [("prefill", ctypes.POINTER(ctypes.c_float)), ("prefill_steps", ctypes.c_int32),
                ("trailing", ctypes.POINTER(ctypes.c_float)), ("trailing_steps", ctypes.c_int32),
                ("tts_pad", ctypes.POINTER(ctypes.c_float))]


_lib = None


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libq3t.so (built by ``__graft_entry__.build()``); raise if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(f"{path} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
    lib = ctypes.CDLL(path)
    P = ctypes.POINTER
    f32p, i32p = P(ctypes.c_float), P(ctypes.c_int32)
    sigs = {
        "q3t_generate_options_default": (None, [P(_GenerateOptions)]),
        "q3t_generate_options_validate": (ctypes.c_int, [P(_GenerateOptions)]),
        "q3t_engine_create": (ctypes.c_int, [P(_EngineOptions), P(ctypes.c_void_p)]),
        "q3t_engine_destroy": (ctypes.c_int, [ctypes.c_void_p]),
        "q3t_engine_get_info": (ctypes.c_int, [ctypes.c_void_p, P(_EngineInfo)]),
        "q3t_engine_set_trace": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32]),
        "q3t_engine_set_fused_attention_rows": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32]),
        "q3t_stream_start": (ctypes.c_int, [ctypes.c_void_p, f32p, ctypes.c_int32, f32p, ctypes.c_int32,
                                            f32p, P(_GenerateOptions), P(ctypes.c_void_p)]),
        "q3t_stream_next_codes": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, i32p, P(_ChunkInfo)]),
        "q3t_stream_destroy": (ctypes.c_int, [ctypes.c_void_p]),
        "q3t_stream_start_profiled": (ctypes.c_int, [ctypes.c_void_p, f32p, ctypes.c_int32, f32p, ctypes.c_int32,
                                                     f32p, P(_GenerateOptions), P(ctypes.c_void_p), P(_Profile)]),
        "q3t_stream_next_codes_profiled": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, i32p, P(_ChunkInfo),
                                                          P(_Profile)]),
        "q3t_debug_phase_times": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, i32p, P(_ChunkInfo), f32p, f32p,
                                                 i32p]),
        "q3t_decode_codes": (ctypes.c_int, [ctypes.c_void_p, i32p, ctypes.c_int32, f32p]),
        "q3t_stream_next_audio": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, i32p, f32p, i32p,
                                                 P(_ChunkInfo)]),
        "q3t_prepare_text": (ctypes.c_int, [ctypes.c_void_p, i32p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                            ctypes.c_int32, f32p, i32p, f32p, i32p, f32p]),
        "q3t_prepare_text_noalloc": (ctypes.c_int, [ctypes.c_void_p, i32p, ctypes.c_int32, ctypes.c_int32,
                                                    ctypes.c_int32, ctypes.c_int32, f32p, i32p, f32p, i32p, f32p]),
        "q3t_stream_start_text": (ctypes.c_int, [ctypes.c_void_p, i32p, ctypes.c_int32, ctypes.c_int32,
                                                 P(_GenerateOptions), P(ctypes.c_void_p)]),
        "q3t_prepare_text_voice_clone": (ctypes.c_int, [ctypes.c_void_p, i32p, ctypes.c_int32, f32p, ctypes.c_int32,
                                                        ctypes.c_int32, ctypes.c_int32, f32p, i32p, f32p, i32p,
                                                        f32p]),
        "q3t_stream_start_voice_clone": (ctypes.c_int, [ctypes.c_void_p, i32p, ctypes.c_int32, f32p,
                                                        ctypes.c_int32, ctypes.c_int32, P(_GenerateOptions),
                                                        P(ctypes.c_void_p)]),
        "q3t_text_stream_start": (ctypes.c_int, [ctypes.c_void_p, i32p, ctypes.c_int32, f32p, ctypes.c_int32,
                                                 P(_GenerateOptions), P(ctypes.c_void_p)]),
        "q3t_text_stream_push": (ctypes.c_int, [ctypes.c_void_p, i32p, ctypes.c_int32]),
        "q3t_text_stream_finish": (ctypes.c_int, [ctypes.c_void_p]),
        "q3t_streams_start": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, P(_StreamInput), P(_GenerateOptions),
                                             P(ctypes.c_void_p)]),
        "q3t_streams_next_codes": (ctypes.c_int, [ctypes.c_void_p, P(ctypes.c_void_p), ctypes.c_int32,
                                                  ctypes.c_int32, i32p, P(_ChunkInfo)]),
        "q3t_generate_codes": (ctypes.c_int, [ctypes.c_void_p, f32p, ctypes.c_int32, f32p, ctypes.c_int32,
                                              f32p, P(_GenerateOptions), i32p, i32p, i32p]),
        "q3t_stream_read_talker_logits": (ctypes.c_int, [ctypes.c_void_p, f32p, ctypes.c_int32, i32p]),
        "q3t_stream_read_cp_logits": (ctypes.c_int, [ctypes.c_void_p, f32p, ctypes.c_int32, i32p]),
        "q3t_sampler_draw": (ctypes.c_int, [ctypes.c_void_p, f32p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                            ctypes.c_float, ctypes.c_float, ctypes.c_uint64, ctypes.c_int32,
                                            ctypes.c_int32, i32p]),
        "q3t_engine_synchronize": (ctypes.c_int, [ctypes.c_void_p]),
        "q3t_bench_kernel": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                                            P(ctypes.c_double), P(ctypes.c_double)]),
        "q3t_bench_kernel_timed": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                                            P(ctypes.c_double), P(ctypes.c_double)]),
        "q3t_debug_gemm": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, f32p, ctypes.c_int32, ctypes.c_int32,
                                          P(ctypes.c_uint16), ctypes.c_int32, f32p, ctypes.c_float, f32p, f32p,
                                          f32p]),
        "q3t_debug_talker_prefill": (ctypes.c_int, [ctypes.c_void_p, f32p, ctypes.c_int32, f32p, f32p, i32p]),
        "q3t_debug_talker_step": (ctypes.c_int, [ctypes.c_void_p, f32p, ctypes.c_int32, f32p, f32p, i32p]),
        "q3t_debug_code_predictor": (ctypes.c_int, [ctypes.c_void_p, f32p, f32p, i32p, f32p]),
        "q3t_last_error": (ctypes.c_char_p, []),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _check(rc: int) -> None:
    if rc != Q3T_OK:
        msg = _lib.q3t_last_error().decode(errors="replace")
        raise _ERRORS.get(rc, Q3tError)(rc, msg)


def _f32(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _fptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _iptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))


@dataclasses.dataclass
class EngineOptions:
    """``EngineOptions`` (generation.rs:25-38) + stream slots and graph replay."""
    device: int = 0
    max_cache_steps: int = DEFAULT_MAX_CACHE_STEPS
    max_streams: int = 1
    use_graph: bool = True
    kv_bf16: bool = False   # KV cache in bf16 instead of fp32


@dataclasses.dataclass
class GenerateOptions:
    """``GenerateOptions`` (generation.rs:40-77), same defaults."""
    speaker: str = "ryan"
    language: str = "english"
    max_frames: int = 240
    decode_audio: bool = True
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
    # Not in the crate's GenerateOptions: False counts each distinct earlier semantic token
    # once (HF, the Python reference); True compounds per occurrence, as the crate's GPU kernel
    # does (src/gpu/kernels.rs:408-426).
    repetition_penalty_per_occurrence: bool = False

    @classmethod
    def greedy(cls, max_frames: int = 240, **kw) -> "GenerateOptions":
        """The reference's parity setting (scripts/qwen3-hip-parity.sh:51-70)."""
        base = dict(max_frames=max_frames, do_sample=False, repetition_penalty=1.0,
                    subtalker_dosample=False, decode_audio=False)
        base.update(kw)
        return cls(**base)

    def _c(self) -> _GenerateOptions:
        o = _GenerateOptions()
        o.speaker = parse_speaker(self.speaker)
        o.language = parse_language(self.language)
        o.max_frames = int(self.max_frames)
        o.decode_audio = int(bool(self.decode_audio))
        o.do_sample = int(bool(self.do_sample))
        o.top_k = int(self.top_k)
        o.top_p = float(self.top_p)
        o.temperature = float(self.temperature)
        o.repetition_penalty = float(self.repetition_penalty)
        o.subtalker_dosample = int(bool(self.subtalker_dosample))
        o.subtalker_top_k = int(self.subtalker_top_k)
        o.subtalker_top_p = float(self.subtalker_top_p)
        o.subtalker_temperature = float(self.subtalker_temperature)
        o.seed = int(self.seed) & 0xFFFFFFFFFFFFFFFF
        o.repetition_penalty_per_occurrence = int(bool(self.repetition_penalty_per_occurrence))
        return o

    def validate(self) -> None:
        """``validate_generate_options`` (generation.rs:569-583), through the C ABI."""
        load_library()
        o = self._c()
        _check(_lib.q3t_generate_options_validate(ctypes.byref(o)))


@dataclasses.dataclass
class StreamOptions:
    """``StreamOptions`` (generation.rs:79-92)."""
    text_lookahead_tokens: int = DEFAULT_TEXT_LOOKAHEAD_TOKENS
    left_context_frames: int = DEFAULT_STREAM_LEFT_CONTEXT_FRAMES

    def validate(self) -> None:
        if self.text_lookahead_tokens == 0:
            raise InvalidInputError(Q3T_ERR_INVALID, "text_lookahead_tokens must be non-zero")


@dataclasses.dataclass
class GeneratedAudioChunk:
    """``GeneratedAudioChunk`` (generation.rs:165-172)."""
    samples: np.ndarray      # float32, 24 kHz
    sample_rate: int
    frames: int
    total_frames: int
    ended_by_eos: bool


@dataclasses.dataclass
class GeneratedSpeech:
    """``GeneratedSpeech`` (generation.rs:94-103, 1521-1553)."""
    text: str
    frames: int
    ended_by_eos: bool
    codes: np.ndarray
    samples: np.ndarray
    sample_rate: int

    def audio_seconds(self) -> float:
        return self.samples.size / float(self.sample_rate)

    def to_wav_bytes(self, gain: float = 1.0) -> bytes:
        from .wav import wav_bytes
        return wav_bytes(self.samples, self.sample_rate, gain)

    def write_wav(self, path, gain: float = 1.0) -> None:
        from .wav import write_wav
        write_wav(path, self.samples, self.sample_rate, gain)


@dataclasses.dataclass
class GenerationProfile:
    """``GenerationProfile`` (generation.rs:104-125).  prepare_text_seconds is host time; the
    rest is GPU time between events.  The CodePredictor prefix (prepare_prefix) is built by
    the Talker's token selection and the next Talker input (build_step_input) by the last
    CodePredictor selection, so their time is inside talker_decode_seconds and
    code_predictor_seconds and those two fields stay 0."""
    prepare_text_seconds: float = 0.0
    upload_seconds: float = 0.0
    prefill_seconds: float = 0.0
    prepare_prefix_seconds: float = 0.0
    code_predictor_seconds: float = 0.0
    build_step_input_seconds: float = 0.0
    talker_decode_seconds: float = 0.0

    def total_seconds(self) -> float:
        return (self.prepare_text_seconds + self.upload_seconds + self.prefill_seconds + self.prepare_prefix_seconds
                + self.code_predictor_seconds + self.build_step_input_seconds + self.talker_decode_seconds)


@dataclasses.dataclass
class ProfiledGeneratedCodes:
    """``ProfiledGeneratedCodes`` (generation.rs:127-131)."""
    codes: "GeneratedCodes"
    profile: GenerationProfile


@dataclasses.dataclass
class GeneratedCodes:
    codes: np.ndarray        # [frames, num_code_groups] int32
    frames: int
    ended_by_eos: bool


@dataclasses.dataclass
class GeneratedCodesChunk:
    codes: np.ndarray        # [frames, num_code_groups] int32
    frames: int
    total_frames: int
    ended_by_eos: bool


# A prompt: prepared rows, content token ids, or text (tokenized with the model directory's
# tokenizer files).
Inputs = Union[PreparedInputs, Sequence[int], str]


class HipTtsEngine:
    def __init__(self, model_dir: str, options: EngineOptions = EngineOptions(),
                 text_prep: Optional[TextPrep] = None):
        load_library()
        o = _EngineOptions(model_dir.encode(), options.device, options.max_cache_steps,
                           options.max_streams, int(options.use_graph), int(options.kv_bf16))
        handle = ctypes.c_void_p()
        _check(_lib.q3t_engine_create(ctypes.byref(o), ctypes.byref(handle)))
        self._h = handle
        info = _EngineInfo()
        _check(_lib.q3t_engine_get_info(self._h, ctypes.byref(info)))
        self.info = {n: getattr(info, n) for n, _ in _EngineInfo._fields_}
        self.code_groups = info.num_code_groups
        self.codec_eos_token = info.codec_eos
        self.max_cache_steps = info.max_cache_steps
        self.hidden = info.talker_hidden
        self.text_prep = text_prep
        self._streams = 0
        # TextTokenizer::from_pretrained (text.rs:161-182) when the directory has its files.
        self.tokenizer = None
        if any(os.path.exists(os.path.join(model_dir, f)) for f in ("tokenizer.json", "vocab.json")):
            from .tokenizer import TextTokenizer
            self.tokenizer = TextTokenizer.from_pretrained(model_dir)

    # -- constructors (generation.rs:255-315) ------------------------------------------
    @classmethod
    def load(cls, model_dir: str, device: int = 0, **kw) -> "HipTtsEngine":
        return cls(model_dir, EngineOptions(device=device), **kw)

    @classmethod
    def load_with_max_frames(cls, model_dir: str, device: int, max_frames: int, **kw) -> "HipTtsEngine":
        return cls(model_dir, EngineOptions(device=device,
                                            max_cache_steps=DEFAULT_PREFILL_HEADROOM + max_frames), **kw)

    @classmethod
    def load_with_options(cls, model_dir: str, options: EngineOptions, **kw) -> "HipTtsEngine":
        return cls(model_dir, options, **kw)

    def close(self) -> None:
        if getattr(self, "_h", None):
            _check(_lib.q3t_engine_destroy(self._h))
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_trace(self, enabled: bool) -> None:
        """Record raw logits of every step (parity checks)."""
        _check(_lib.q3t_engine_set_trace(self._h, int(bool(enabled))))

    def set_fused_attention_rows(self, rows: int) -> None:
        """Talker positions below `rows` run the fused attention + O kernel (default 192 with
        an fp32 KV cache, 256 with bf16), later ones the split attention and the merging O
        projection."""
        _check(_lib.q3t_engine_set_fused_attention_rows(self._h, int(rows)))

    def synchronize(self) -> None:
        _check(_lib.q3t_engine_synchronize(self._h))

    KERNELS = {0: "gemv_qkv_rmsnorm", 1: "gemv_o_residual", 2: "gemv_gate_up_swiglu", 3: "gemv_down_residual",
               4: "attention_decode_full_cache", 5: "attention_codepredictor", 6: "select_cp_greedy",
               7: "attention_talker_half_cache", 8: "gemv_lm_head", 9: "attention_oproj_codepredictor",
               10: "attention_oproj_talker_half_cache"}

    def bench_kernel(self, kernel: int, iters: int = 1030):
        """(average launch microseconds, algorithmic bytes per launch) of one kernel class."""
        us, b = ctypes.c_double(), ctypes.c_double()
        _check(_lib.q3t_bench_kernel(self._h, int(kernel), int(iters), ctypes.byref(us), ctypes.byref(b)))
        return us.value, b.value

    def bench_kernel_timed(self, kernel: int, iters: int = 1030):
        """(average kernel duration in microseconds without the launch gap, algorithmic bytes per
        launch) of one kernel class, eager launches timed by their own dispatch events."""
        us, b = ctypes.c_double(), ctypes.c_double()
        _check(_lib.q3t_bench_kernel_timed(self._h, int(kernel), int(iters), ctypes.byref(us), ctypes.byref(b)))
        return us.value, b.value

    def dominant_kernel_roofline(self, peak_gbps: float, kernel: int = 2, iters: int = 1030,
                                 graph: bool = True) -> dict:
        """Roofline entry for the kernel class that dominates a frame's time (the gate/up GEMV).

        ``achieved`` divides the algorithmic bytes of a launch by the kernel's own duration: the
        1030 launches of one frame order are issued eagerly, each timed by its dispatch's start
        and stop events (the per-dispatch duration rocprofv3's kernel trace reports for the same
        command).  ``graph_us_per_launch`` is the same sequence replayed as one graph, timed as a
        whole (the dependent-launch gap included): the cost a frame sees.  ``graph=False``
        captures no graph at all (commands run under a kernel tracer): that leg is then null."""
        self.bench_kernel_timed(kernel, 103)   # warm
        us, b = self.bench_kernel_timed(kernel, iters)
        gus = None
        if graph:
            self.bench_kernel(kernel, 103)
            gus, _ = self.bench_kernel(kernel, iters)
        achieved = b / (us * 1e-6) / 1e9
        return {"kernel": self.KERNELS[kernel], "bound": "hbm", "achieved": round(achieved, 1),
                "peak": peak_gbps, "unit": "GB/s", "frac": round(achieved / peak_gbps, 4), "traffic": None,
                "avg_launch_us": round(us, 3), "timing": "eager launches, per-dispatch start/stop events",
                "graph_us_per_launch": round(gus, 3) if gus is not None else None,
                "graph_frac_gap_included": (round(b / (gus * 1e-6) / 1e9 / peak_gbps, 4)
                                            if gus is not None else None),
                "algorithmic_bytes_per_launch": int(b), "launches_timed": iters}

    def debug_gemm(self, epi: int, X: np.ndarray, W_bits: np.ndarray, N: int, gamma=None, eps: float = 1e-6,
                   res=None, bias=None) -> np.ndarray:
        """The matrix-core GEMM on host arrays (test hook)."""
        X = _f32(X)
        M, K = X.shape
        Wb = np.ascontiguousarray(W_bits, dtype=np.uint16)
        Y = np.zeros((M, N), dtype=np.float32)
        opt = lambda a: _fptr(_f32(a)) if a is not None else None
        keep = [_f32(a) for a in (gamma, res, bias) if a is not None]  # noqa: F841 (lifetime)
        g = _f32(gamma) if gamma is not None else None
        r = _f32(res) if res is not None else None
        b = _f32(bias) if bias is not None else None
        _check(_lib.q3t_debug_gemm(self._h, int(epi), _fptr(X), M, K,
                                   Wb.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), int(N),
                                   _fptr(g) if g is not None else None, float(eps),
                                   _fptr(r) if r is not None else None, _fptr(b) if b is not None else None,
                                   _fptr(Y)))
        return Y

    # -- parity hooks (the reference's prefill_from_host / decode_step_from_host /
    #    generate_from_host seams) --------------------------------------------------------
    def debug_talker_prefill(self, prefill: np.ndarray):
        """(normed hidden [H], raw logits [V], greedy token) after a Talker prefill on slot 0."""
        x = _f32(prefill)
        hidden = np.zeros(self.info["talker_hidden"], np.float32)
        logits = np.zeros(self.info["talker_vocab"], np.float32)
        tok = ctypes.c_int32()
        _check(_lib.q3t_debug_talker_prefill(self._h, _fptr(x), x.shape[0], _fptr(hidden), _fptr(logits),
                                             ctypes.byref(tok)))
        return hidden, logits, tok.value

    def debug_talker_step(self, step_input: np.ndarray, offset: int):
        """One Talker step at `offset` over slot 0's cache: (normed hidden, raw logits, greedy token)."""
        x = _f32(step_input)
        hidden = np.zeros(self.info["talker_hidden"], np.float32)
        logits = np.zeros(self.info["talker_vocab"], np.float32)
        tok = ctypes.c_int32()
        _check(_lib.q3t_debug_talker_step(self._h, _fptr(x), int(offset), _fptr(hidden), _fptr(logits),
                                          ctypes.byref(tok)))
        return hidden, logits, tok.value

    def debug_code_predictor(self, talker_hidden: np.ndarray, semantic_embed: np.ndarray):
        """Greedy CodePredictor over [talker_hidden; semantic_embed]: (tokens [groups-1], embedding_sum)."""
        th, se = _f32(talker_hidden), _f32(semantic_embed)
        tokens = np.zeros(self.code_groups - 1, np.int32)
        emb = np.zeros(self.info["talker_hidden"], np.float32)
        _check(_lib.q3t_debug_code_predictor(self._h, _fptr(th), _fptr(se), _iptr(tokens), _fptr(emb)))
        return tokens, emb

    def sampler_draw(self, logits: np.ndarray, n: int, do_sample: bool = True, top_k: int = 50,
                     top_p: float = 1.0, temperature: float = 0.9, seed: int = 0, kind: int = 0) -> np.ndarray:
        """n draws of the fused sampler from one logit row (draw i uses Philox counter (i, kind))."""
        l = _f32(logits)
        out = np.zeros(n, dtype=np.int32)
        _check(_lib.q3t_sampler_draw(self._h, _fptr(l), l.shape[0], int(bool(do_sample)), int(top_k),
                                     float(top_p), float(temperature), int(seed) & 0xFFFFFFFFFFFFFFFF,
                                     int(kind), int(n), _iptr(out)))
        return out

    # -- generation ----------------------------------------------------------------------
    def content_ids(self, text: str) -> List[int]:
        """``content_ids_for_text`` (text.rs:384-395) with the model directory's tokenizer."""
        if self.tokenizer is None:
            raise InvalidInputError(Q3T_ERR_INVALID, "the model directory has no tokenizer.json or "
                                                     "vocab.json + merges.txt")
        return self.tokenizer.content_ids(text)

    def _on_device(self, inputs: Inputs) -> Optional[List[int]]:
        """Content ids to prepare on the device, or None for host-prepared inputs: text, or ids
        with no host TextPrep given."""
        if isinstance(inputs, PreparedInputs):
            return None
        if isinstance(inputs, str):
            return self.content_ids(inputs)
        return None if self.text_prep is not None else [int(i) for i in inputs]

    def _prepare(self, inputs: Inputs, options: GenerateOptions, lookahead: int) -> PreparedInputs:
        if isinstance(inputs, PreparedInputs):
            return inputs
        if isinstance(inputs, str) or self.text_prep is None:
            ids = self._on_device(inputs)
            return self.prepare_text(ids, options.speaker, options.language, lookahead)
        return self.text_prep.prepare(inputs, options.speaker, options.language, lookahead)

    def generate_codes(self, inputs: Inputs, options: GenerateOptions = GenerateOptions()) -> GeneratedCodes:
        """``generate_codes`` (generation.rs:356-371): all text in the prefill, then the rollout."""
        ids = self._on_device(inputs)
        if ids is not None:  # prompt rows built on the device, then drained as one chunk
            with self.start_stream_text(ids, options, StreamOptions(text_lookahead_tokens=0x7FFFFFFF)) as st:
                chunk = st.next_codes_chunk(max(options.max_frames, 1))
                codes = chunk.codes if chunk else np.zeros((0, self.code_groups), np.int32)
                return GeneratedCodes(codes, int(codes.shape[0]), st.ended_by_eos)
        inp = self._prepare(inputs, options, 1 << 30)
        o = options._c()
        pre, trail, pad = _f32(inp.prefill), _f32(inp.trailing_text), _f32(inp.tts_pad_embed)
        codes = np.zeros((max(options.max_frames, 0), self.code_groups), dtype=np.int32)
        frames, eos = ctypes.c_int32(), ctypes.c_int32()
        _check(_lib.q3t_generate_codes(self._h, _fptr(pre), pre.shape[0], _fptr(trail), trail.shape[0],
                                       _fptr(pad), ctypes.byref(o), _iptr(codes), ctypes.byref(frames),
                                       ctypes.byref(eos)))
        return GeneratedCodes(codes[:frames.value].copy(), frames.value, bool(eos.value))

    def generate_codes_profiled(self, inputs: Inputs,
                                options: GenerateOptions = GenerateOptions()) -> ProfiledGeneratedCodes:
        """``generate_codes_profiled`` (generation.rs:395-419): generate_codes with the time of
        each phase.  Frames run one at a time without the frame graph."""
        import time
        options.validate()
        t0 = time.perf_counter()
        inp = self._prepare(inputs, options, 1 << 30)
        prof = GenerationProfile(prepare_text_seconds=time.perf_counter() - t0)
        p = _Profile()
        o = options._c()
        pre, trail, pad = _f32(inp.prefill), _f32(inp.trailing_text), _f32(inp.tts_pad_embed)
        handle = ctypes.c_void_p()
        _check(_lib.q3t_stream_start_profiled(self._h, _fptr(pre), pre.shape[0], _fptr(trail), trail.shape[0],
                                              _fptr(pad), ctypes.byref(o), ctypes.byref(handle), ctypes.byref(p)))
        try:
            n = max(options.max_frames, 1)
            codes = np.zeros((n, self.code_groups), dtype=np.int32)
            info = _ChunkInfo()
            _check(_lib.q3t_stream_next_codes_profiled(handle, n, _iptr(codes), ctypes.byref(info), ctypes.byref(p)))
        finally:
            _check(_lib.q3t_stream_destroy(handle))
        prof.upload_seconds, prof.prefill_seconds = p.upload_seconds, p.prefill_seconds
        prof.code_predictor_seconds, prof.talker_decode_seconds = p.code_predictor_seconds, p.talker_decode_seconds
        g = GeneratedCodes(codes[:info.frames].copy(), int(info.frames), bool(info.ended_by_eos))
        return ProfiledGeneratedCodes(g, prof)

    def start_stream(self, inputs: Inputs, options: GenerateOptions = GenerateOptions(),
                     stream_options: StreamOptions = StreamOptions()) -> "HipTtsStream":
        """``start_stream`` (generation.rs:421-440)."""
        stream_options.validate()
        ids = self._on_device(inputs)
        if ids is not None:
            return self.start_stream_text(ids, options, stream_options)
        inp = self._prepare(inputs, options, stream_options.text_lookahead_tokens)
        return HipTtsStream(self, inp, options, stream_options)

    # -- codec decoder ----------------------------------------------------------------------
    @property
    def has_codec(self) -> bool:
        """The model directory holds speech_tokenizer/model.safetensors (decode_codes works)."""
        return self.info.get("samples_per_frame", 0) > 0

    def decode_codes(self, codes: np.ndarray) -> np.ndarray:
        """``decode_codes`` (generation.rs:619-647): codes [frames, 16] -> float32 samples at 24 kHz."""
        c = np.ascontiguousarray(np.asarray(codes, dtype=np.int32))
        if c.size % self.code_groups:
            raise InvalidInputError(Q3T_ERR_INVALID, f"code length {c.size} is not divisible by {self.code_groups}")
        frames = c.size // self.code_groups
        out = np.zeros(frames * max(self.info["samples_per_frame"], 1), dtype=np.float32)
        _check(_lib.q3t_decode_codes(self._h, _iptr(c), frames, _fptr(out)))
        return out if frames else np.zeros(0, np.float32)

    def generate(self, inputs: Inputs, options: GenerateOptions = GenerateOptions()) -> "GeneratedSpeech":
        """``generate`` (generation.rs:317-332): codes, then audio when ``decode_audio``."""
        g = self.generate_codes(inputs, options)
        samples = (self.decode_codes(g.codes) if options.decode_audio and g.frames
                   else np.zeros(0, np.float32))
        return GeneratedSpeech(inputs if isinstance(inputs, str) else "", g.frames, g.ended_by_eos, g.codes,
                               samples, SAMPLE_RATE)

    # -- prompt preparation on the device --------------------------------------------------
    @property
    def has_device_text_prep(self) -> bool:
        """The checkpoint holds the text-embedding table (q3t_prepare_text works)."""
        return self.info.get("text_vocab", 0) > 0

    def prepare_text(self, content_ids: Sequence[int], speaker: str = "ryan", language: str = "english",
                     text_lookahead_tokens: int = 1 << 30, no_alloc: bool = False) -> PreparedInputs:
        """``TtsTextPrep::prepare_custom_voice_with_lookahead`` (text.rs:340-382) on the device
        (``q3t_prepare_text``): content ids -> prefill rows, trailing text rows, tts_pad row.
        ``no_alloc`` runs ``q3t_prepare_text_noalloc`` instead: the same rows with no device
        allocation (a bounded prompt length; calls on one GPU must not overlap)."""
        ids = np.ascontiguousarray(np.asarray(content_ids, dtype=np.int64).astype(np.int32))
        n, H = int(ids.size), self.info["talker_hidden"]
        opts = GenerateOptions(speaker=speaker, language=language)._c()
        pre = np.zeros((9 + n, H), np.float32)
        trail = np.zeros((n + 1, H), np.float32)
        pad = np.zeros(H, np.float32)
        P, T = ctypes.c_int32(), ctypes.c_int32()
        lookahead = min(int(text_lookahead_tokens), 0x7FFFFFFF)
        fn = _lib.q3t_prepare_text_noalloc if no_alloc else _lib.q3t_prepare_text
        _check(fn(self._h, _iptr(ids), n, opts.speaker, opts.language, lookahead, _fptr(pre),
                  ctypes.byref(P), _fptr(trail), ctypes.byref(T), _fptr(pad)))
        return PreparedInputs(content_ids=ids.astype(np.int64), prefill=pre[:P.value].copy(),
                              trailing_text=trail[:T.value].copy(), tts_pad_embed=pad)

    def start_stream_text(self, content_ids: Sequence[int], options: GenerateOptions = GenerateOptions(),
                          stream_options: StreamOptions = StreamOptions()) -> "HipTtsStream":
        """``start_stream`` (generation.rs:421-440) with the prompt rows built on the device
        straight into the stream's slot (``q3t_stream_start_text``)."""
        stream_options.validate()
        ids = np.ascontiguousarray(np.asarray(content_ids, dtype=np.int64).astype(np.int32))
        o = options._c()
        handle = ctypes.c_void_p()
        lookahead = min(int(stream_options.text_lookahead_tokens), 0x7FFFFFFF)
        _check(_lib.q3t_stream_start_text(self._h, _iptr(ids), int(ids.size), lookahead, ctypes.byref(o),
                                          ctypes.byref(handle)))
        n = int(ids.size)
        steps = 9 + (0 if n == 0 else max(1, min(lookahead, n)))
        return HipTtsStream(self, None, options, stream_options, handle=handle, prefill_steps=steps)

    # -- voice clone (x-vector prompts) ----------------------------------------------------
    def _voice_clone_args(self, inputs: Union[str, Sequence[int]], prompt: VoiceClonePrompt):
        if isinstance(inputs, PreparedInputs):
            raise InvalidInputError(Q3T_ERR_INVALID, "voice clone calls take text or content token ids")
        prompt.check_x_vector_only()
        ids = self.content_ids(inputs) if isinstance(inputs, str) else [int(i) for i in inputs]
        ids = np.ascontiguousarray(np.asarray(ids, dtype=np.int64).astype(np.int32))
        emb = np.ascontiguousarray(np.asarray(prompt.speaker_embedding, dtype=np.float32).reshape(-1))
        return ids, emb

    def prepare_voice_clone_text(self, inputs: Union[str, Sequence[int]], prompt: VoiceClonePrompt,
                                 language: str = "english", text_lookahead_tokens: int = 1 << 30) -> PreparedInputs:
        """``TtsTextPrep::prepare_voice_clone_xvector_with_lookahead`` (text.rs:432-490) on the
        device (``q3t_prepare_text_voice_clone``)."""
        ids, emb = self._voice_clone_args(inputs, prompt)
        n, H = int(ids.size), self.info["talker_hidden"]
        lang = GenerateOptions(language=language)._c().language
        pre = np.zeros((9 + n, H), np.float32)
        trail = np.zeros((n + 1, H), np.float32)
        pad = np.zeros(H, np.float32)
        P, T = ctypes.c_int32(), ctypes.c_int32()
        lookahead = min(int(text_lookahead_tokens), 0x7FFFFFFF)
        _check(_lib.q3t_prepare_text_voice_clone(self._h, _iptr(ids), n, _fptr(emb), int(emb.size), lang, lookahead,
                                                 _fptr(pre), ctypes.byref(P), _fptr(trail), ctypes.byref(T),
                                                 _fptr(pad)))
        return PreparedInputs(content_ids=ids.astype(np.int64), prefill=pre[:P.value].copy(),
                              trailing_text=trail[:T.value].copy(), tts_pad_embed=pad)

    def start_voice_clone_stream(self, inputs: Union[str, Sequence[int]], prompt: VoiceClonePrompt,
                                 options: GenerateOptions = GenerateOptions(),
                                 stream_options: StreamOptions = StreamOptions()) -> "HipTtsStream":
        """``start_voice_clone_stream`` (generation.rs:442-462): the prompt rows with the
        prompt's speaker embedding, built on the device into the stream's slot
        (``q3t_stream_start_voice_clone``).  ``options.speaker`` is not used."""
        options.validate()  # generation.rs:450-451: options, stream options, then the prompt
        stream_options.validate()
        ids, emb = self._voice_clone_args(inputs, prompt)
        o = options._c()
        handle = ctypes.c_void_p()
        lookahead = min(int(stream_options.text_lookahead_tokens), 0x7FFFFFFF)
        _check(_lib.q3t_stream_start_voice_clone(self._h, _iptr(ids), int(ids.size), _fptr(emb), int(emb.size),
                                                 lookahead, ctypes.byref(o), ctypes.byref(handle)))
        n = int(ids.size)
        steps = 9 + (0 if n == 0 else max(1, min(lookahead, n)))
        return HipTtsStream(self, None, options, stream_options, handle=handle, prefill_steps=steps)

    def generate_voice_clone_codes(self, inputs: Union[str, Sequence[int]], prompt: VoiceClonePrompt,
                                   options: GenerateOptions = GenerateOptions()) -> GeneratedCodes:
        """``generate_voice_clone_codes`` (generation.rs:373-393): all text in the prefill, then
        the rollout."""
        with self.start_voice_clone_stream(inputs, prompt, options,
                                           StreamOptions(text_lookahead_tokens=0x7FFFFFFF)) as st:
            chunk = st.next_codes_chunk(max(options.max_frames, 1))
            codes = chunk.codes if chunk else np.zeros((0, self.code_groups), np.int32)
            return GeneratedCodes(codes, int(codes.shape[0]), st.ended_by_eos)

    def generate_voice_clone(self, inputs: Union[str, Sequence[int]], prompt: VoiceClonePrompt,
                             options: GenerateOptions = GenerateOptions()) -> "GeneratedSpeech":
        """``generate_voice_clone`` (generation.rs:334-354): codes, then audio when ``decode_audio``."""
        g = self.generate_voice_clone_codes(inputs, prompt, options)
        samples = (self.decode_codes(g.codes) if options.decode_audio and g.frames
                   else np.zeros(0, np.float32))
        return GeneratedSpeech(inputs if isinstance(inputs, str) else "", g.frames, g.ended_by_eos, g.codes,
                               samples, SAMPLE_RATE)

    # -- text streams (text pushed while audio is produced) ---------------------------------
    def start_text_stream_polling(self, options: GenerateOptions = GenerateOptions(), stream_options=None):
        """``start_text_stream_polling`` (generation.rs:475-483)."""
        from .text_stream import PollingTextStream, TextStreamOptions
        return PollingTextStream(self, options, stream_options or TextStreamOptions())

    def start_text_stream(self, options: GenerateOptions = GenerateOptions(), stream_options=None):
        """``start_text_stream`` (generation.rs:463-473): (TextStreamInput, HipTextStream)."""
        from .text_stream import HipTextStream
        st = HipTextStream(self.start_text_stream_polling(options, stream_options))
        return st._input(), st

    def start_voice_clone_text_stream_polling(self, prompt: VoiceClonePrompt,
                                              options: GenerateOptions = GenerateOptions(), stream_options=None):
        """``start_voice_clone_text_stream_polling`` (generation.rs:496-511)."""
        from .text_stream import PollingTextStream, TextStreamOptions
        return PollingTextStream(self, options, stream_options or TextStreamOptions(), prompt)

    def start_voice_clone_text_stream(self, prompt: VoiceClonePrompt, options: GenerateOptions = GenerateOptions(),
                                      stream_options=None):
        """``start_voice_clone_text_stream`` (generation.rs:485-494)."""
        from .text_stream import HipTextStream
        st = HipTextStream(self.start_voice_clone_text_stream_polling(prompt, options, stream_options))
        return st._input(), st

    # -- several streams at once (no counterpart in the reference: one stream per engine) --
    def start_streams(self, inputs: List[Inputs], options: List[GenerateOptions],
                      stream_options: StreamOptions = StreamOptions()) -> List["HipTtsStream"]:
        """``q3t_streams_start``: n ``start_stream`` calls with one prefill over all prompts."""
        if len(inputs) != len(options) or not inputs:
            raise InvalidInputError(Q3T_ERR_INVALID, "need one GenerateOptions per input")
        stream_options.validate()
        n = len(inputs)
        prepared = [self._prepare(i, o, stream_options.text_lookahead_tokens) for i, o in zip(inputs, options)]
        keep = []
        ins = (_StreamInput * n)()
        opts = (_GenerateOptions * n)()
        for j, (inp, o) in enumerate(zip(prepared, options)):
            pre, trail, pad = _f32(inp.prefill), _f32(inp.trailing_text), _f32(inp.tts_pad_embed)
            keep += [pre, trail, pad]
            ins[j] = _StreamInput(_fptr(pre), pre.shape[0], _fptr(trail), trail.shape[0], _fptr(pad))
            opts[j] = o._c()
        handles = (ctypes.c_void_p * n)()
        _check(_lib.q3t_streams_start(self._h, n, ins, opts, handles))
        return [HipTtsStream(self, inp, o, stream_options, handle=ctypes.c_void_p(h))
                for inp, o, h in zip(prepared, options, handles)]

    def next_codes_chunks(self, streams: List["HipTtsStream"],
                          max_chunk_frames: int) -> List[Optional[GeneratedCodesChunk]]:
        """``q3t_streams_next_codes``: ``next_codes_chunk`` of every listed stream, run as one
        batch (one pass over the weights per frame for all of them)."""
        if max_chunk_frames <= 0:
            raise InvalidInputError(Q3T_ERR_INVALID, "max_chunk_frames must be non-zero")
        n = len(streams)
        handles = (ctypes.c_void_p * n)(*[s._h.value if s._h else None for s in streams])
        buf = np.zeros((n, max_chunk_frames, self.code_groups), dtype=np.int32)
        infos = (_ChunkInfo * n)()
        _check(_lib.q3t_streams_next_codes(self._h, handles, n, max_chunk_frames, _iptr(buf), infos))
        return [s._accept(buf[j], infos[j]) for j, s in enumerate(streams)]

    def generate_codes_batch(self, inputs: List[Inputs], options: List[GenerateOptions],
                             chunk_frames: int = 6) -> List[GeneratedCodes]:
        """Start every stream together and pull chunks for all of them until each has ended."""
        streams = self.start_streams(inputs, options, StreamOptions(text_lookahead_tokens=1 << 30))
        try:
            live = list(streams)
            while live:
                chunks = self.next_codes_chunks(live, chunk_frames)
                live = [s for s, c in zip(live, chunks) if c is not None]
            return [s.finish_codes() for s in streams]
        finally:
            for s in streams:
                s.close()


class HipTtsStream:
    """``HipTtsStream`` (generation.rs:145-163, 876-997).  Must not outlive its engine."""

    def __init__(self, engine: HipTtsEngine, inputs: Optional[PreparedInputs], options: GenerateOptions,
                 stream_options: StreamOptions, handle: Optional[ctypes.c_void_p] = None,
                 prefill_steps: Optional[int] = None):
        self.engine = engine
        self.inputs = inputs
        self.options = options
        self.stream_options = stream_options
        if handle is None:
            o = options._c()
            pre, trail, pad = _f32(inputs.prefill), _f32(inputs.trailing_text), _f32(inputs.tts_pad_embed)
            handle = ctypes.c_void_p()
            _check(_lib.q3t_stream_start(engine._h, _fptr(pre), pre.shape[0], _fptr(trail), trail.shape[0],
                                         _fptr(pad), ctypes.byref(o), ctypes.byref(handle)))
        self._h = handle
        self.prefill_steps = inputs.prefill_steps if prefill_steps is None else prefill_steps
        self._codes = []
        self.frame = 0
        self.ended_by_eos = False

    def next_codes_chunk(self, max_chunk_frames: int) -> Optional[GeneratedCodesChunk]:
        if max_chunk_frames <= 0:
            raise InvalidInputError(Q3T_ERR_INVALID, "max_chunk_frames must be non-zero")
        buf = np.zeros((max_chunk_frames, self.engine.code_groups), dtype=np.int32)
        info = _ChunkInfo()
        _check(_lib.q3t_stream_next_codes(self._h, max_chunk_frames, _iptr(buf), ctypes.byref(info)))
        return self._accept(buf, info)

    def next_codes_chunk_timed(self, max_chunk_frames: int):
        """``next_codes_chunk`` with each frame's phases timed on the GPU (``q3t_debug_phase_times``):
        (chunk or None, CodePredictor microseconds per frame, Talker-step microseconds per frame)."""
        if max_chunk_frames <= 0:
            raise InvalidInputError(Q3T_ERR_INVALID, "max_chunk_frames must be non-zero")
        buf = np.zeros((max_chunk_frames, self.engine.code_groups), dtype=np.int32)
        cp = np.zeros(max_chunk_frames, np.float32)
        tk = np.zeros(max_chunk_frames, np.float32)
        info = _ChunkInfo()
        n = ctypes.c_int32()
        _check(_lib.q3t_debug_phase_times(self._h, max_chunk_frames, _iptr(buf), ctypes.byref(info), _fptr(cp),
                                          _fptr(tk), ctypes.byref(n)))
        return self._accept(buf, info), cp[:n.value].copy(), tk[:n.value].copy()

    def next_audio_chunk(self, max_chunk_frames: int) -> Optional[GeneratedAudioChunk]:
        """``next_audio_chunk`` (generation.rs:965-989): the next codes chunk, decoded with up
        to ``stream_options.left_context_frames`` earlier frames as context."""
        if max_chunk_frames <= 0:
            raise InvalidInputError(Q3T_ERR_INVALID, "max_chunk_frames must be non-zero")
        buf = np.zeros((max_chunk_frames, self.engine.code_groups), dtype=np.int32)
        samples = np.zeros(max_chunk_frames * max(self.engine.info["samples_per_frame"], 1), dtype=np.float32)
        n = ctypes.c_int32()
        info = _ChunkInfo()
        _check(_lib.q3t_stream_next_audio(self._h, max_chunk_frames, int(self.stream_options.left_context_frames),
                                          _iptr(buf), _fptr(samples), ctypes.byref(n), ctypes.byref(info)))
        chunk = self._accept(buf, info)
        if chunk is None:
            return None
        return GeneratedAudioChunk(samples[:n.value].copy(), SAMPLE_RATE, chunk.frames, chunk.total_frames,
                                   chunk.ended_by_eos)

    def _accept(self, buf: np.ndarray, info: _ChunkInfo) -> Optional[GeneratedCodesChunk]:
        self.frame = info.total_frames
        self.ended_by_eos = bool(info.ended_by_eos)
        if info.frames == 0:
            return None
        codes = buf[:info.frames].copy()
        self._codes.append(codes)
        return GeneratedCodesChunk(codes, info.frames, info.total_frames, bool(info.ended_by_eos))

    def finish_codes(self) -> GeneratedCodes:
        codes = (np.concatenate(self._codes) if self._codes
                 else np.zeros((0, self.engine.code_groups), dtype=np.int32))
        self.close()
        return GeneratedCodes(codes, int(codes.shape[0]), self.ended_by_eos)

    def talker_logits(self) -> np.ndarray:
        """Raw Talker logits of every Talker evaluation so far ([rows, V])."""
        V = self.engine.info["talker_vocab"]
        cap = self.frame + 1
        out = np.zeros((cap, V), dtype=np.float32)
        rows = ctypes.c_int32()
        _check(_lib.q3t_stream_read_talker_logits(self._h, _fptr(out), cap, ctypes.byref(rows)))
        return out[:rows.value]

    def cp_logits(self) -> np.ndarray:
        """CodePredictor logits of the frames so far ([frames, groups - 1, V_cp])."""
        e = self.engine.info
        out = np.zeros((max(self.frame, 1), e["num_code_groups"] - 1, e["cp_vocab"]), dtype=np.float32)
        n = ctypes.c_int32()
        _check(_lib.q3t_stream_read_cp_logits(self._h, _fptr(out), self.frame, ctypes.byref(n)))
        return out[:n.value]

    def close(self) -> None:
        if getattr(self, "_h", None):
            _check(_lib.q3t_stream_destroy(self._h))
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
