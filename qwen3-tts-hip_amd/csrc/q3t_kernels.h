// Host-side launchers for the gfx950 kernels in q3t_kernels.hip.
#pragma once

#include "q3t_device.h"

namespace q3t {

// Optional hardware timestamps of one launch (hipExtLaunchKernelGGL start/stop events).
struct LaunchTiming {
  hipEvent_t start = nullptr, stop = nullptr;
};

// y = W x (optionally x := RMSNorm(x) * gamma first) with the epilogue `epi`.  `streaming`
// selects non-temporal weight loads.  Requires K = 512 * c for c in {1, 2, 3, 4, 6, 8, 12};
// returns hipErrorInvalidValue otherwise.  a.rows = 2 (ordinary loads, K <= 3072) runs two
// input rows against one pass over the weights.
hipError_t launch_gemv(int epi, bool norm, bool streaming, const GemvArgs &a, hipStream_t stream,
                       const LaunchTiming *timing = nullptr);
bool gemv_supports_k(int K);
// Workgroups of a store (or bias) GEMV launch of N outputs over K with cache-resident (not
// streamed) weights: the number of order keys a hand-off producer writes.
int gemv_grid_for(int N, int K);

// Most stream rows one batched launch covers (skinny GEMM rows, select workgroups).
constexpr int kMaxRows = 16;

// Fused q/k head RMSNorm + RoPE + KV-cache write + GQA decode attention, split over key
// positions in chunks (one workgroup per (KV head, chunk, stream row)).  With partial_out
// the chunks' partials are merged by the consumer (the O-projection GEMV, or
// launch_attn_merge for stream rows).
hipError_t launch_attn_decode(const AttnArgs &a, int head_dim, hipStream_t stream,
                              const LaunchTiming *timing = nullptr, int rows = 1);
hipError_t launch_attn_merge(const AttnMergeArgs &a, int rows, hipStream_t stream);
// The same attention for one stream and one chunk (cap <= 32, chunk attn_chunk_len(cap),
// position from the launch), with the output projection fused in: a.opart[h][r] = KV head h's share of
// (a.wo * attn)[r] for r < a.wo_rows (a multiple of 32).  The gate/up GEMV adds the shares
// to the residual (GemvArgs::parts, hidden 512 or 1024).  Requires at most 8 KV heads and 1
// or 2 query heads per KV head.
hipError_t launch_attn_oproj(const AttnArgs &a, int head_dim, hipStream_t stream,
                             const LaunchTiming *timing = nullptr);
// The Talker's decode attention (one stream) and its O projection in one launch, with the
// projection's K split by KV head: a.opart[h][r] = KV head h's share of (a.wo * attn)[r] for
// r < a.wo_rows, the shares the gate/up GEMV adds to the residual (GemvArgs::parts).  Every
// workgroup runs its head's whole attention (no partials): a.cap <= 1024, position from the
// stream state (POS_TALKER_FRAME) or the launch; a.wo_rows a multiple of
// attn_oproj_full_rows(q_heads, kv_heads); at most 8 KV heads and 1 or 2 query heads per KV
// head; a.kcache / a.vcache are the layer's caches of one stream.
hipError_t launch_attn_oproj_full(const AttnArgs &a, int head_dim, hipStream_t stream,
                                  const LaunchTiming *timing = nullptr);
int attn_oproj_full_rows(int q_heads, int kv_heads);
// Most attention chunks the O-projection GEMV merges itself (caches up to 8 x 128 rows); the
// partials of a longer cache are merged by launch_attn_merge first.
constexpr int kAttnGemvMergeChunks = 8;
// Most chunk partials launch_attn_merge merges per (KV head, stream row).
constexpr int kAttnMergeMaxChunks = 64;
int attn_max_cache_steps(int q_heads, int kv_heads);
// Key rows per attention workgroup for a cache of `cap` rows, and the resulting number of
// chunks (partials the workspace must hold per head).
int attn_chunk_len(int cap);
int attn_chunks(int cap);
// Key rows per workgroup of the stream-row (batched) attention, whose partials
// launch_attn_merge merges: 32 up to a 2,048-row cache, then 64 and 128.
int attn_rows_chunk_len(int cap);

// Matrix-core GEMM (bf16 weights, fp32 activations split into three bf16 terms, fp32 accumulate)
// for many rows: prompt prefill and batched decode.  Requires K % 32 == 0.
hipError_t launch_gemm(int epi, const GemmArgs &a, hipStream_t stream);
// The same product for M <= 16 rows (batched decode); norm = fused RMSNorm of the rows with
// gain gamma (row_scale must be null).  Requires K = 512 * c, c in {1, 2, 3, 4, 6, 8, 12}
// (K <= 2048 with norm).
bool gemm_skinny_supports(int M, int K, bool norm);
// GemmArgs::split2 (EPI_RESIDUAL, T16 X and Y): K = 1024 * c, c in {1, 2, 3, 4, 6}.
bool gemm_skinny_split2_supports(int K);
hipError_t launch_gemm_skinny(int epi, bool norm, const GemmArgs &a, hipStream_t stream);
// dst = src [rows][K] bf16 in the skinny GEMM's packed layout (GemmArgs::w_packed).
// Requires rows % 16 == 0 and K % 32 == 0.
hipError_t launch_pack_weights(const uint16_t *src, uint16_t *dst, int rows, int K, hipStream_t stream);
// inv_rms[m] = 1 / sqrt(mean(X[m]^2) + eps).
hipError_t launch_row_rms(const float *X, int ldx, int M, int K, float eps, float *inv_rms, hipStream_t stream);

// Prompt preparation: X[m] = fp32(table[ids[m]]) ([M][width]); x = silu(x) in place; and row m
// of Y ([M][H], + codec_emb[codec[m]] where codec[m] >= 0) to dst[m] = (kind << 24) | row with
// kind 0 prefill row, 1 trailing row, 2 the tts_pad row, 3 dropped.  The host validates ids.
hipError_t launch_text_gather(const uint16_t *table, int width, const int32_t *ids, int M, float *X, hipStream_t stream);
hipError_t launch_silu(float *x, size_t n, hipStream_t stream);
// codec[m] value that adds the H-float row `xvec` (a voice-clone speaker embedding) instead of
// a codec embedding row.
constexpr int32_t kTextSpeakerRow = -2;
hipError_t launch_text_assemble(const float *Y, int H, int M, const int32_t *codec, const uint16_t *codec_emb,
                                const float *xvec, const int32_t *dst, float *prefill, float *trailing, float *pad,
                                hipStream_t stream);

// dst[i] = src[i] (bf16 -> fp32, exact).
hipError_t launch_bf16_to_f32(const uint16_t *src, float *dst, size_t n, hipStream_t stream);

// Prefill attention: q/k norm + RoPE + KV store for P rows, then causal attention.
hipError_t launch_prefill_attention(const PrefillBatchArgs &a, hipStream_t stream);
// The same for P = 2 rows at positions 0 and 1 (the CodePredictor's prefix) in one launch.
// With a.wo set, the output projection is fused in as in launch_attn_oproj: row p's per-KV-head
// shares go to a.opart + p * a.opart_row (a.out unused).
hipError_t launch_prefix_attention(const PrefillAttnArgs &a, hipStream_t stream);
// The same prefix for stream rows 0 .. rows - 1 (PrefillAttnArgs::ld_pos, kv_row, st, row_on),
// output in T16 blocks, one per position; no fused projection.
hipError_t launch_prefix_attention_rows(const PrefillAttnArgs &a, int rows, hipStream_t stream);

// Token selection, one workgroup per stream row (rows > 1 needs row_on and the row strides).
hipError_t launch_select_talker(const SelectTalkerArgs &a, hipStream_t stream, int rows = 1);
hipError_t launch_select_cp(const SelectCpArgs &a, hipStream_t stream, int rows = 1);
// n independent draws from one logit row (draw i uses Philox counter (i, kind, 0, 0)).
hipError_t launch_sample_draws(const float *logits, int V, const SamplingParams &sp, uint64_t seed, int kind, int n,
                               int32_t *out, hipStream_t stream);

// Largest vocabulary the select kernels hold in LDS.
constexpr int kMaxVocab = 4096;

// Device scratch of the entry points that allocate nothing (q3t_prepare_text_noalloc): one
// statically sized array per GPU, shared by every call on that GPU (calls that overlap on one
// GPU race).  noalloc_scratch_setup resolves the array's address on the current device (once
// per device; call it with that device current); noalloc_scratch returns it (nullptr before
// a successful setup).
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
hipError_t noalloc_scratch_setup(int device);
void *noalloc_scratch(int device);

}  // namespace q3t
