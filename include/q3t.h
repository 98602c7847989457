/*
 * q3t — MI355X-native Qwen3-TTS token loop (Talker decode step + 15-group CodePredictor).
 *
 * C ABI.  Plain pointers and sizes; no C++ or torch types cross this boundary.
 * Each entry point replaces one piece of the reference crate's public API
 * (piedshag/qwen3-tts-hip, src/generation.rs) and is cited below.
 *
 * Conventions (mirroring the reference's Result<T, Error>, src/error.rs:3-44):
 *   - every call returns an int status: Q3T_OK (0) or one of the Q3T_ERR_* codes;
 *   - the message of the last failure on the calling thread is q3t_last_error();
 *   - the engine owns all device memory; the caller owns host arrays and nothing is
 *     retained after a call returns;
 *   - one host thread drives an engine (the reference engine is neither Send nor Sync);
 *     a stream must not outlive its engine.
 */
#ifndef Q3T_H
#define Q3T_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q3T_OK 0
#define Q3T_ERR_INVALID 1   /* Error::InvalidInput (src/error.rs) */
#define Q3T_ERR_HIP 2       /* Error::Hip{call,status,message} */
#define Q3T_ERR_CAPACITY 3  /* P + max_frames exceeds max_cache_steps (generation.rs:608-617) */
#define Q3T_ERR_NOT_FOUND 4 /* missing file / tensor (Error::InvalidInput in the reference loader) */
#define Q3T_ERR_BUSY 5      /* every stream slot of the engine is in use */

typedef struct q3t_engine q3t_engine;
typedef struct q3t_stream q3t_stream;

/* EngineOptions (generation.rs:25-38) plus the model directory the reference passes to
 * HipTtsEngine::load_with_options (generation.rs:255-315).  max_streams is new: the
 * reference engine owns a single Talker KV cache. */
typedef struct {
  const char *model_dir;   /* holds config.json + model.safetensors */
  int32_t device;          /* HIP device ordinal */
  int32_t max_cache_steps; /* Talker KV capacity per stream (default 512, at most 8192) */
  int32_t max_streams;     /* stream slots (KV caches) to allocate (default 1, at most 16) */
  int32_t use_graph;       /* 1 = replay each frame as one captured hipGraph (default) */
  int32_t kv_dtype;        /* KV cache element: 0 = fp32 (default, as the reference),
                              1 = bf16 (half the KV bytes, rounded once at the store) */
} q3t_engine_options;

/* GenerateOptions (generation.rs:40-77), field for field.  speaker / language (the Speaker /
 * Language ordinals) choose the codec rows of a prompt that q3t_stream_start_text prepares; with
 * prepared rows they are already encoded in them.  decode_audio is the caller's: audio comes
 * from q3t_decode_codes / q3t_stream_next_audio. */
typedef struct {
  int32_t speaker;
  int32_t language;
  int32_t max_frames;
  int32_t decode_audio;
  int32_t do_sample;
  int32_t top_k;
  float top_p;
  float temperature;
  float repetition_penalty;
  int32_t subtalker_dosample;
  int32_t subtalker_top_k;
  float subtalker_top_p;
  float subtalker_temperature;
  uint64_t seed;
  /* No counterpart in GenerateOptions: how repetition_penalty counts the history.  0 (default):
   * once per distinct earlier semantic token, as HF's processor in the Python reference does.
   * 1: once per occurrence, compounding, as the crate's GPU kernel apply_repetition_penalty_f32
   * does over the full semantic_history (src/gpu/kernels.rs:408-426, generation.rs:717-727). */
  int32_t repetition_penalty_per_occurrence;
} q3t_generate_options;

/* Shapes read from config.json (src/model/config.rs:8-43). */
typedef struct {
  int32_t talker_hidden, talker_intermediate, talker_layers, talker_vocab;
  int32_t cp_hidden, cp_intermediate, cp_layers, cp_vocab;
  int32_t q_heads, kv_heads, head_dim, num_code_groups;
  int32_t codec_eos, max_cache_steps, max_streams;
  int64_t device_bytes; /* device memory held by the engine */
  int32_t text_vocab;   /* text-embedding rows on the device (0: no device text preparation) */
  int32_t text_hidden;
  int32_t samples_per_frame; /* codec samples per frame (1920 at 24 kHz), 0: no codec decoder */
} q3t_engine_info;

/* GeneratedCodesChunk (generation.rs:876-963). */
typedef struct {
  int32_t frames;       /* frames in this chunk (0 = the stream had nothing left: None) */
  int32_t total_frames; /* frames produced by the stream so far */
  int32_t ended_by_eos;
} q3t_chunk_info;

/* Fills *opts with the reference defaults (GenerateOptions::default, generation.rs:60-77). */
void q3t_generate_options_default(q3t_generate_options *opts);

/* HipTtsEngine::validate_generate_options (generation.rs:569-583) and
 * SamplingConfig::validate (src/model/sampling.rs:11-26): max_frames > 0,
 * repetition_penalty > 0, top_p in (0, 1], temperature > 0, top_k >= 0, for both the Talker
 * and the subtalker.  q3t_stream_start applies the same checks. */
int q3t_generate_options_validate(const q3t_generate_options *opts);

/* HipTtsEngine::load_with_options (generation.rs:255-315). */
int q3t_engine_create(const q3t_engine_options *opts, q3t_engine **out);
int q3t_engine_destroy(q3t_engine *engine);
/* The loaded shapes (q3t_engine_info) and the engine's capacity, memory and codec figures. */
int q3t_engine_get_info(const q3t_engine *engine, q3t_engine_info *out);

/* HipTtsEngine::start_stream_with_inputs (generation.rs:513-567): validates options
 * (generation.rs:569-606), checks P + max_frames <= max_cache_steps, uploads the prefill
 * [P, H], trailing text rows [T, H] and tts_pad [H], runs the Talker prefill and draws the
 * first semantic token.  Host arrays are float32 row-major. */
int q3t_stream_start(q3t_engine *engine, const float *prefill, int32_t prefill_steps,
                     const float *trailing, int32_t trailing_steps, const float *tts_pad,
                     const q3t_generate_options *opts, q3t_stream **out);

/* HipTtsStream::next_codes_chunk (generation.rs:876-963): runs up to max_chunk_frames
 * frames and copies their codes ([frames, num_code_groups] int32, frame-major
 * [semantic, a1..a15]) into codes, which must hold max_chunk_frames * num_code_groups. */
int q3t_stream_next_codes(q3t_stream *stream, int32_t max_chunk_frames, int32_t *codes,
                          q3t_chunk_info *info);

/* One stream's inputs for q3t_streams_start: the arrays q3t_stream_start takes
 * (TtsTextPrep::prepare_custom_voice_with_lookahead, text.rs:340-382). */
typedef struct {
  const float *prefill;   /* [prefill_steps, H] */
  int32_t prefill_steps;
  const float *trailing;  /* [trailing_steps, H] */
  int32_t trailing_steps;
  const float *tts_pad;   /* [H] */
} q3t_stream_input;

/* Multi-stream start (new; the reference serves one stream per engine): n independent
 * start_stream_with_inputs calls (generation.rs:513-567) in one.  Same validation and
 * capacity check per stream; takes n free slots; runs one Talker prefill over the prompt
 * rows of all n streams (each stream attends only to its own rows and cache) and draws each
 * stream's first semantic token.  opts and out have n entries.  Q3T_ERR_BUSY when fewer
 * than n slots are free.  Each stream's codes equal what q3t_stream_start would produce. */
int q3t_streams_start(q3t_engine *engine, int32_t n, const q3t_stream_input *inputs,
                      const q3t_generate_options *opts, q3t_stream **out);

/* Batched HipTtsStream::next_codes_chunk (generation.rs:876-963) over n streams of one
 * engine: every frame advances all listed streams that have frames left with one pass over
 * the weights (ragged positions, per-stream KV caches and options), until each has produced
 * max_chunk_frames frames or ended.  Stream j's codes go to codes + j * max_chunk_frames *
 * num_code_groups and its chunk to info[j] (frames = 0: nothing left, the reference's None).
 * Streams not listed are untouched.  When exactly one listed stream has frames left it runs
 * the single-stream frame (q3t_stream_next_codes), which is faster for one row; both compute
 * the same frame to float32 rounding. */
int q3t_streams_next_codes(q3t_engine *engine, q3t_stream *const *streams, int32_t n,
                           int32_t max_chunk_frames, int32_t *codes, q3t_chunk_info *info);

/* TtsTextPrep::prepare_custom_voice_with_lookahead (text.rs:340-382) from content token ids,
 * on the device: the tokenizer's ids between the chat-template prefix and suffix (text.rs:361)
 * -> text-embedding rows -> text_projection (fc1, SiLU, fc2) -> plus the codec embedding rows
 * of the role / think / language / speaker / pad / bos layout (text.rs:516-603).  speaker and
 * language are the q3t_generate_options enums, resolved through config.json's spk_id and
 * codec_language_id maps (text.rs:642-653).  The model directory must hold
 * talker.model.text_embedding.weight (Q3T_ERR_NOT_FOUND otherwise).  prefill must hold
 * (9 + n_ids) * H floats, trailing (n_ids + 1) * H, tts_pad H; *prefill_steps = 9 + lookahead
 * rows and *trailing_steps = n_ids - lookahead + 1 (the rest of the content, then tts_eos),
 * lookahead = min(max(text_lookahead_tokens, 1), n_ids) (0 without content). */
int q3t_prepare_text(q3t_engine *engine, const int32_t *content_ids, int32_t n_ids, int32_t speaker,
                     int32_t language, int32_t text_lookahead_tokens, float *prefill, int32_t *prefill_steps,
                     float *trailing, int32_t *trailing_steps, float *tts_pad);

/* q3t_prepare_text without any device allocation.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, rows and errors as q3t_prepare_text; its workspace and staging
 * rows live in a statically sized per-GPU array of 16 MiB (the GEMMs' K-split partials stay in
 * the engine's own workspace, allocated at q3t_engine_create), which bounds the prompt: about
 * 650 content ids at Talker hidden 1024 and 500 at 2048 (text_hidden 2048), Q3T_ERR_INVALID
 * beyond.  Every call on one GPU shares that array, from any engine: calls that overlap on one
 * GPU (another thread) race and must be serialised by the caller. */
int q3t_prepare_text_noalloc(q3t_engine *engine, const int32_t *content_ids, int32_t n_ids, int32_t speaker,
                             int32_t language, int32_t text_lookahead_tokens, float *prefill,
                             int32_t *prefill_steps, float *trailing, int32_t *trailing_steps, float *tts_pad);

/* HipTtsEngine::start_stream (generation.rs:421-440) from content token ids: the rows
 * q3t_prepare_text describes are built on the device straight into the stream's slot (no
 * host round trip), then as q3t_stream_start.  The speaker and language come from opts. */
int q3t_stream_start_text(q3t_engine *engine, const int32_t *content_ids, int32_t n_ids,
                          int32_t text_lookahead_tokens, const q3t_generate_options *opts, q3t_stream **out);

/* TtsTextPrep::prepare_voice_clone_xvector_with_lookahead (text.rs:432-490, 507-514): as
 * q3t_prepare_text with the speaker's codec row replaced by a voice-clone prompt's speaker
 * embedding (VoiceClonePrompt::speaker_embedding, src/model/voice_clone.rs), embedding_len
 * floats in host memory; embedding_len must equal the Talker hidden size (Q3T_ERR_INVALID
 * "speaker embedding length ... does not match model hidden ...", text.rs:445-451).  Only
 * x-vector prompts exist here; rejecting ICL prompts (text.rs:439-443) is the caller's, who
 * holds the prompt. */
int q3t_prepare_text_voice_clone(q3t_engine *engine, const int32_t *content_ids, int32_t n_ids,
                                 const float *speaker_embedding, int32_t embedding_len, int32_t language,
                                 int32_t text_lookahead_tokens, float *prefill, int32_t *prefill_steps,
                                 float *trailing, int32_t *trailing_steps, float *tts_pad);

/* HipTtsEngine::start_voice_clone_stream (generation.rs:442-462) from content token ids: the
 * rows q3t_prepare_text_voice_clone describes, built on the device into the stream's slot,
 * then as q3t_stream_start.  opts->speaker is not used; opts->language is. */
int q3t_stream_start_voice_clone(q3t_engine *engine, const int32_t *content_ids, int32_t n_ids,
                                 const float *speaker_embedding, int32_t embedding_len,
                                 int32_t text_lookahead_tokens, const q3t_generate_options *opts,
                                 q3t_stream **out);

/* Text streams: text that arrives while audio is produced (PollingTextStream,
 * generation.rs:176-211, 1093-1437).  The caller keeps the reference's token queue and its
 * start / resume / flush rules (TextStreamOptions, generation.rs:212-228); the device holds the
 * prompt rows and the trailing text rows.
 *
 * q3t_text_stream_start: try_start_generation (generation.rs:1280-1358) once enough content ids
 * are queued: the prefill of custom_voice_prefill_from_content_tokens (text.rs:397-404) with every
 * one of the n_ids >= 1 ids in it (codec bos on the last), or, with a non-null
 * speaker_embedding of embedding_len floats, voice_clone_xvector_prefill_from_content_tokens
 * (text.rs:406-418); then the Talker prefill and the first semantic token.  The stream's
 * trailing text starts empty and open: q3t_stream_next_codes / q3t_stream_next_audio run frame
 * f (f + 1 < max_frames) only once trailing row f has been pushed, and return frames = 0 with
 * ended_by_eos = 0 and total_frames < max_frames when the next frame waits for text (the
 * reference's IncrementalAudio::NeedMoreText).  Open streams are not accepted by
 * q3t_streams_next_codes. */
int q3t_text_stream_start(q3t_engine *engine, const int32_t *content_ids, int32_t n_ids,
                          const float *speaker_embedding, int32_t embedding_len,
                          const q3t_generate_options *opts, q3t_stream **out);

/* The next n content ids popped from the caller's queue, in order: each becomes the next
 * trailing text row, projected on the device (next_trailing_buffer, generation.rs:1367-1369).
 * Q3T_ERR_INVALID "cannot push text after finish_text" once the text is finished
 * (generation.rs:1108-1116). */
int q3t_text_stream_push(q3t_stream *stream, const int32_t *content_ids, int32_t n);

/* finish_text (generation.rs:1118-1129): the tts_eos row follows the last pushed row, then every
 * later frame reads tts_pad (generation.rs:1371-1386), and the frames no longer wait for text.
 * A second call does nothing. */
int q3t_text_stream_finish(q3t_stream *stream);

/* HipTtsEngine::decode_codes (generation.rs:619-647): codec frames [frames][num_code_groups]
 * int32 (frame-major, as the codes calls return them) -> frames * samples_per_frame samples at
 * 24 kHz in [-1, 1], through the speech tokenizer's decoder (src/audio/codec_hip.rs: RVQ,
 * pre-conv, 8-layer pre-transformer, two ConvNeXt upsampling stages, four Snake / transposed-
 * conv decoder blocks).  The model directory must hold speech_tokenizer/model.safetensors
 * (Q3T_ERR_NOT_FOUND otherwise).  frames = 0 decodes nothing. */
int q3t_decode_codes(q3t_engine *engine, const int32_t *codes, int32_t frames, float *samples);

/* HipTtsStream::next_audio_chunk (generation.rs:965-989): q3t_stream_next_codes into codes
 * (max_chunk_frames * num_code_groups), then the chunk's frames decoded together with up to
 * left_context_frames earlier frames of the stream (StreamOptions::left_context_frames,
 * default 25), keeping the chunk's own info->frames * samples_per_frame samples in samples
 * (*n_samples of them).  info->frames = 0: the stream had nothing left. */
int q3t_stream_next_audio(q3t_stream *stream, int32_t max_chunk_frames, int32_t left_context_frames,
                          int32_t *codes, float *samples, int32_t *n_samples, q3t_chunk_info *info);

/* GenerationProfile (generation.rs:104-125) as the device measures it, in seconds of GPU time
 * between hipEvents: the upload of the prompt rows, the Talker prefill with the first token,
 * the CodePredictor passes (its token selection and the next Talker input, the reference's
 * build_step_input, included) and the Talker decode steps (codec head, token selection and the
 * CodePredictor prefix, the reference's prepare_code_predictor_prefix, included). */
typedef struct {
  double upload_seconds, prefill_seconds, code_predictor_seconds, talker_decode_seconds;
} q3t_profile;

/* generate_codes_profiled's rollout (generation.rs:395-419, 751-874): q3t_stream_start and
 * q3t_stream_next_codes that also add their phases' GPU time to *profile.  Frames run one at
 * a time without the frame graph (events between the phases), so they are slower than
 * q3t_stream_next_codes; the codes are the same. */
int q3t_stream_start_profiled(q3t_engine *engine, const float *prefill, int32_t prefill_steps,
                              const float *trailing, int32_t trailing_steps, const float *tts_pad,
                              const q3t_generate_options *opts, q3t_stream **out, q3t_profile *profile);
int q3t_stream_next_codes_profiled(q3t_stream *stream, int32_t max_chunk_frames, int32_t *codes,
                                   q3t_chunk_info *info, q3t_profile *profile);

/* Drops the stream and frees its slot (HipTtsStream's Drop). */
int q3t_stream_destroy(q3t_stream *stream);

/* HipTtsEngine::generate_codes (generation.rs:356-371, rollout 657-749): start + drain.
 * codes must hold max_frames * num_code_groups int32. */
int q3t_generate_codes(q3t_engine *engine, const float *prefill, int32_t prefill_steps,
                       const float *trailing, int32_t trailing_steps, const float *tts_pad,
                       const q3t_generate_options *opts, int32_t *codes, int32_t *frames,
                       int32_t *ended_by_eos);

/* Parity hook (the reference's fixture dump, python-reference/qwen3_tts_reference.py:487-523):
 * raw Talker logits of every Talker evaluation so far ([rows, talker_vocab]: row 0 is the
 * prefill, row f+1 follows frame f).  Recording is on when the stream was started after
 * q3t_engine_set_trace(engine, 1).  *rows receives the number of rows written. */
int q3t_engine_set_trace(q3t_engine *engine, int32_t enabled);
int q3t_stream_read_talker_logits(q3t_stream *stream, float *out, int32_t capacity_rows,
                                  int32_t *rows);
/* CodePredictor logits of the frames so far ([frames, num_code_groups - 1, cp_vocab]). */
int q3t_stream_read_cp_logits(q3t_stream *stream, float *out, int32_t capacity_frames,
                              int32_t *frames);

/* Parity hooks on the reference's own seams (all run greedy on stream slot 0, which must not
 * hold a stream; ERR_BUSY otherwise):
 *   q3t_debug_talker_prefill  HipTalker::prefill_from_host (talker.rs:140-205): the Talker
 *     prefill of `steps` rows [steps, H]; hidden = final RMSNorm of the last row [H], logits =
 *     raw codec-head logits [talker_vocab], token = argmax of the suppressed logits.  Slot 0's
 *     KV cache keeps the prefill for q3t_debug_talker_step.
 *   q3t_debug_talker_step     HipTalker::decode_step_from_host (talker.rs:235-295): one
 *     Talker step of input [H] at position `offset` over slot 0's cache rows 0..offset-1;
 *     same outputs.
 *   q3t_debug_code_predictor  HipCodePredictor::generate_from_host (code_predictor.rs:277-302):
 *     the greedy CodePredictor over the prefix [talker_hidden; semantic_embed] (each
 *     talker-hidden wide); tokens [num_code_groups - 1], embedding_sum [talker_hidden]. */
int q3t_debug_talker_prefill(q3t_engine *engine, const float *prefill, int32_t steps, float *hidden,
                             float *logits, int32_t *token);
int q3t_debug_talker_step(q3t_engine *engine, const float *input, int32_t offset, float *hidden,
                          float *logits, int32_t *token);
int q3t_debug_code_predictor(q3t_engine *engine, const float *talker_hidden,
                             const float *semantic_embed, int32_t *tokens, float *embedding_sum);

/* Talker positions below `rows` (default 192 with an fp32 KV cache, 256 with bf16) run the
 * 0.6B Talker's fused attention + O projection kernel, later positions the split attention and
 * the O projection that merges its partials (the fused kernel's workgroups each read their
 * head's whole cache, which costs more than the extra launch from ~190 fp32 / ~265 bf16 rows
 * on).  0 never fuses; a value at or above the KV capacity
 * always does.  Both compute the same step to float32 rounding.  Takes effect from the next
 * call that runs frames.  No counterpart in the reference (a tuning and test hook). */
int q3t_engine_set_fused_attention_rows(q3t_engine *engine, int32_t rows);

/* Waits until every stream slot of the engine is idle. */
int q3t_engine_synchronize(q3t_engine *engine);

/* Kernel timing for the roofline report (no counterpart in the reference, whose profiler is
 * external rocprofv3 + ROCTx ranges, src/gpu/profile.rs:20-72).  Captures `iters` kernels of
 * one class, in the order a frame issues them (Talker layers, then the CodePredictor layers of
 * its 15 passes), as one hipGraph on stream slot 0's stream -- the way frames run -- and times
 * one replay with hipEvents.  Returns the average time per launch (us; the gap between
 * dependent launches included) and the algorithmic bytes one launch moves.
 *   kernel 0: QKV GEMV (+ input RMSNorm)    1: O GEMV (+ residual)
 *          2: gate/up GEMV (+ RMSNorm, SwiGLU)    3: down GEMV (+ residual)
 *          4: Talker attention over a full cache  5: CodePredictor attention (positions 0..15)
 *          6: greedy CodePredictor selection     7: Talker attention at half the cache
 *          8: CodePredictor LM-head GEMV
 *          9: CodePredictor attention with the O projection fused (when the model has it)
 *         10: Talker attention at half the cache with the O projection fused (when the model
 *             has it: the 0.6B Talker)
 * Class 1 is the O GEMV merging split-attention partials (Talker layers); a Talker with
 * the fused attention + O projection (the 0.6B's) runs class 10 in frames instead.  Class 2
 * (gate/up) sums the per-head shares of the Talker's and the CodePredictor's fused
 * projections as frames do. Slot 0 must not hold a stream.  An engine created with
 * use_graph = 0 captures no graph anywhere: there this call fails with Q3T_ERR_INVALID (the
 * timed variant below launches eagerly). */
int q3t_bench_kernel(q3t_engine *engine, int32_t kernel, int32_t iters, double *avg_us,
                     double *bytes_per_launch);

/* q3t_bench_kernel with every launch issued eagerly and bracketed by its own dispatch's
 * start / stop timestamps (hipExtLaunchKernelGGL events): *avg_us is the kernel's duration
 * without the dependent-launch gap, the per-dispatch duration a kernel trace reports for the
 * same launches.  Kernel class 6 is not available here.  Bench hook, no counterpart in the
 * reference. */
int q3t_bench_kernel_timed(q3t_engine *engine, int32_t kernel, int32_t iters, double *avg_us,
                           double *bytes_per_launch);

/* q3t_stream_next_codes with the GPU time of each frame's two phases: the CodePredictor's 15
 * groups (cp_us[i]) and the Talker step with its token selection (talker_us[i]), each phase
 * replayed as its own graph (eager launches without use_graph) with events between them and
 * a synchronisation after every frame.  *timed = the frames timed (<= max_chunk_frames).  Bench
 * hook for per-step rooflines (the reference's GenerationProfile splits the same phases,
 * generation.rs:104-131). */
int q3t_debug_phase_times(q3t_stream *stream, int32_t max_chunk_frames, int32_t *codes, q3t_chunk_info *info,
                          float *cp_us, float *talker_us, int32_t *timed);

/* The fused token sampler on its own: n draws from one logit row [V] (host array), draw i
 * using Philox4x32-10 counter (i, kind, 0, 0) and key seed.  This is the code path of the
 * frame loop's select kernels, exposed the way the reference exposes its sample_topk_f32
 * kernel (src/gpu/kernels.rs:265-334) for statistical checks.  do_sample = 0 returns the
 * argmax (ties to the lowest index, kernels.rs:176-221). */
int q3t_sampler_draw(q3t_engine *engine, const float *logits, int32_t vocab, int32_t do_sample,
                     int32_t top_k, float top_p, float temperature, uint64_t seed, int32_t kind,
                     int32_t n, int32_t *tokens);

/* The matrix-core GEMM on its own (test hook; no counterpart in the reference, whose
 * rocblas_sgemm call sites this kernel replaces, src/gpu/blas.rs:99-154):
 * Y[M][N] = f(X[M][K]) . W[N][K]^T with epilogue epi (0 store, 1 + res[M][N], 2 SwiGLU with
 * W = [gate rows; up rows] ([2N][K]), 3 + bias[N]).  gamma != NULL applies RMSNorm(eps) with
 * gain gamma[K] to each row of X first.  W is bf16 bits; X, Y, res, bias fp32 host arrays.
 * M <= 16 with K = 512 * {1,2,3,4,6,8,12} runs the batched-decode (skinny) kernel, other
 * shapes the prefill kernel.  epi 4 is epi 1 in the batched frame's K-split form (M <= 16,
 * K = 1024 * {1,2,3,4,6}, N % 32 == 0, no gamma): two K halves summed by fp32 atomic adds. */
int q3t_debug_gemm(q3t_engine *engine, int32_t epi, const float *X, int32_t M, int32_t K,
                   const uint16_t *W, int32_t N, const float *gamma, float eps, const float *res,
                   const float *bias, float *Y);

const char *q3t_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* Q3T_H */
