// Types shared by the host engine and the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q3t {

// Per-stream loop state, resident in device memory so that one captured frame graph can
// be replayed frame after frame without host round trips.  Written only by the kernels
// that end a frame (the Talker's token selection) and by the host at stream start.
struct SlotState {
  int32_t frame;          // frames completed so far
  int32_t semantic;       // semantic token that starts the next frame
  int32_t done;           // 0 running, 1 ended by codec_eos, 2 reached max_frames
  int32_t prefill_steps;  // P: the Talker decodes frame f at position P + f
  int32_t max_frames;
  int32_t trailing_rows;  // trailing text rows held on device (the next row is tts_pad)
  int32_t pad0, pad1;
};

struct SamplingParams {
  int32_t do_sample;
  int32_t top_k;       // 0 keeps every finite candidate
  float top_p;
  float temperature;
};

// Per-stream options, also device resident (read by the select kernels).
struct SlotParams {
  SamplingParams talker;
  SamplingParams cp;
  float repetition_penalty;
  int32_t use_history;  // repetition penalty applies (penalty != 1 or talker sampling on)
  uint32_t seed_lo, seed_hi;
  int32_t trace;        // record raw logits
  int32_t codec_eos;
  int32_t penalty_per_occurrence;  // repetition penalty compounds per history occurrence
  int32_t pad1;
};

enum SkipMode : int32_t {
  SKIP_NEVER = 0,   // host-driven work (prefill)
  SKIP_DONE = 1,    // frame work: skipped once the stream has ended
  SKIP_TALKER = 2,  // the Talker step that follows a frame: also skipped after the last frame
};

enum PosMode : int32_t {
  POS_CONST = 0,        // position given by the launch
  POS_TALKER_FRAME = 1, // position = prefill_steps + frame
};

enum Epilogue : int32_t {
  EPI_STORE = 0,     // out[n] = acc
  EPI_RESIDUAL = 1,  // out[n] = res[n] + acc
  EPI_SWIGLU = 2,    // out[j] = silu(acc_gate_j) * acc_up_j; W holds gate rows then up rows
  EPI_BIAS = 3,      // out[n] = acc + bias[n]
  // matrix-core GEMMs only (the codec decoder):
  EPI_AFFINE_RES = 4,  // out[n] = res[n] + (acc + bias[n]) * scale[n] (bias, scale optional)
  EPI_BIAS_GELU = 5,   // out[n] = gelu(acc + bias[n]), erf form
};

// Greedy token hand-off into a CodePredictor group (one stream): the group's input token is
// the one whose order key is the largest of keys[0 .. n_keys) (the previous group's LM head
// writes them).  Workgroup 0 of the consuming kernel also stores the group's input row to cur
// (row tok of cur_table when set, else the embedding row emb[tok]), adds emb[tok] to sum
// (first: assigns it) and writes the token to codes[frame][code] (first: also the frame's
// semantic token to codes[frame][0]); codes rows are `groups` wide.
struct TokenHandoff {
  const uint64_t *keys;
  int32_t n_keys;
  const uint16_t *emb;     // [V][emb_width] bf16
  int32_t emb_width;
  const float *cur_table;  // [V][cur_width] or null
  int32_t cur_width;
  float *cur, *sum;
  int32_t *codes;
  int32_t first, code, groups;
  // Stream rows (grid z of the attention): row r reads keys + r * keys_row and stores to
  // sum + r * sum_row, cur + r * cur_row, codes + r * codes_row (all 0 for one stream).
  int64_t keys_row, sum_row, cur_row, codes_row;
  // One stream, token chosen by a selection kernel (sampled groups): the token is read from
  // tok_in instead of reduced from keys.  With emb null the selection kernel has done the
  // stores above (only the table row is taken); with emb set (and cur, sum, codes, first,
  // code, groups) workgroup (0, 0) does them, as for keys.
  const int32_t *tok_in;
};

struct GemvArgs {
  const uint16_t *W;  // [rows, K] bf16, row-major (the checkpoint's [out, in] layout)
  const float *x;     // [K]
  const float *gamma; // RMSNorm gain over x (prologue variants)
  const float *res;   // residual (EPI_RESIDUAL)
  const float *bias;  // bias (EPI_BIAS)
  float *out;
  int32_t N;          // outputs (EPI_SWIGLU: I, with 2I weight rows)
  int32_t K;
  float eps;
  int32_t skip;
  const SlotState *st;
  // Input = merge of attention partials (O projection after split attention), when set.
  const float *attn_part;
  int32_t attn_part_chunks, attn_chunk, attn_pos_mode, attn_pos_const, attn_q_heads, attn_kv_heads;
  // rows = 2: a second input row x + ldx_r (res + ldr_r, out + ldo_r) against the same weights
  int32_t rows, ldx_r, ldr_r, ldo_r;
  // Greedy token hand-off producer (one stream; EPI_STORE), replacing a token selection
  // kernel: workgroup b also stores to keys_out[b] the order key (order_key) of its largest
  // output, and the outputs to trace + st->frame * trace_frame when trace is set.
  uint64_t *keys_out;
  float *trace;
  int64_t trace_frame;
  // Input = x + parts[0] + parts[1] + ... + parts[n_parts - 1] (in that order), each part at
  // parts + p * ld_parts, when parts is set (a head-split O projection's per-head shares;
  // gate/up with RMSNorm only, K of 512 or 1024).  Workgroup 0 also stores that sum to
  // x_store.
  const float *parts;
  int32_t n_parts, ld_parts;
  float *x_store;
  // rows = 2 with parts: row 1's parts at parts + ldp_r, its sum stored at x_store + ldxs_r
  int32_t ldp_r, ldxs_r;
  // Input = the next Talker input, assembled from the last CodePredictor group's greedy
  // hand-off when tin.keys is set (one stream; EPI_STORE with RMSNorm, streamed weights,
  // K = tin.emb_width): tok = the token of the largest of tin.keys[0 .. n_keys), e =
  // tin.emb[tok], s = tin.sum + e and x = (tin_codec_emb[st->semantic] + s) +
  // tin_trailing[min(st->frame, st->trailing_rows)], what the selection kernel would store.
  // Workgroup 0 stores x to tin_x and tok to tin.codes[st->frame * tin.groups + tin.code]
  // unless the stream has ended, before the launch's own skip check.  tin.sum and tin.cur
  // are not written (nothing reads them after the last group).
  TokenHandoff tin;
  const uint16_t *tin_codec_emb;  // [V][K] bf16
  const float *tin_trailing;      // [rows][K]
  float *tin_x;                   // [K]
};

// Most workgroups a hand-off producer may have (keys per group).
constexpr int kHandoffKeys = 256;

struct AttnArgs {
  const float *qkv;     // [q_heads*d + 2*kv_heads*d] raw projections
  const float *gq;      // [d] q_norm gain
  const float *gk;      // [d] k_norm gain
  const float2 *rope;   // [cap][d/2] (cos, sin)
  void *kcache;         // [kv_heads][cap][d], fp32 or bf16 (kv_bf16)
  void *vcache;         // [kv_heads][cap][d]
  float *out;           // [q_heads*d]
  int32_t q_heads, kv_heads, cap;
  float eps, scale;
  int32_t pos_mode, pos_const;
  int32_t skip;
  int32_t kv_bf16;
  const SlotState *st;
  float *part;          // [kv_heads][part_chunks][G][2 + d] per-chunk (max, sum, P.V)
  int32_t part_chunks;
  int32_t chunk;        // key rows per workgroup (attn_chunk_len(cap))
  int32_t partial_out;  // 1: write partials for the O projection to merge; 0: write `out`
  // Stream rows (grid z): row r reads qkv + r * ld_qkv, state st + r, caches + r * kv_row
  // elements, and writes out + r * ld_out / part + r * part_row.  row_on (null for one
  // stream) masks rows that are not part of the launch.
  int32_t ld_qkv, ld_out;
  int64_t kv_row, part_row;
  const int32_t *row_on;
  int32_t out_t16;      // direct output in T16 (rows <= 16) instead of out + r * ld_out
  // Greedy hand-off (one chunk; one stream or stream rows): the raw q/k/v row is
  // qkv_table + tok * ld_table instead of qkv, tok as TokenHandoff defines it (h.keys set).
  TokenHandoff h;
  const float *qkv_table;
  int64_t ld_table;
  // Fused output projection (launch_attn_oproj): wo [wo_rows][q_heads*d] bf16; opart
  // [kv_heads][wo_rows] receives each KV head's share of wo * attn.
  const uint16_t *wo;
  int32_t wo_rows;
  float *opart;
};

// Merge of split-attention partials into attention outputs, one workgroup per stream row.
struct AttnMergeArgs {
  const float *part;    // [rows][kv_heads][part_chunks][G][2 + d]
  float *out;           // [rows][ld_out]
  int32_t q_heads, kv_heads, part_chunks, chunk, pos_mode, pos_const, skip, ld_out;
  int64_t part_row;
  const SlotState *st;  // [rows]
  const int32_t *row_on;
  int32_t out_t16;      // output in T16 instead of out + r * ld_out
};

// Tiled 16-row activation layout ("T16") used between the skinny GEMMs of the batched frame:
// element (m, k) of a [16][K] block sits at t16_index(m, k).  Each 32-wide k step is one
// contiguous 2 KiB block in the order the matrix cores take their A operand (lane
// m + 16 * ((k % 32) / 8) holds k % 8 = 0..7), so a wave loads it with unit-stride 32-byte
// reads instead of touching 16 rows per instruction.
__host__ __device__ inline size_t t16_index(int m, int k) {
  return ((size_t)(k >> 5) * 64 + ((k >> 3) & 3) * 16 + m) * 8 + (k & 7);
}

// Y[M][N] = X[M][K] . W[N][K]^T with the GEMV epilogues (matrix-core path for many rows).
struct GemmArgs {
  const float *X;          // [M][ldx] fp32
  const float *row_scale;  // [M] per-row multiplier on X (RMSNorm 1/rms) or null
  const float *gamma;      // [K] per-column multiplier on X (RMSNorm gain) or null
  const uint16_t *W;       // [N][K] bf16 (EPI_SWIGLU: [2N][K], gate rows then up rows)
  float *Y;                // [M][ldy]
  const float *res;        // EPI_RESIDUAL: [M][ldr]
  const float *bias;       // EPI_BIAS: [N]
  const float *scale;      // EPI_AFFINE_RES: [N] or null
  int32_t M, N, K, ldx, ldy, ldr;
  // Segmented X rows (matrix-core GEMMs; a dilated convolution's taps): with xseg_len > 0,
  // element k of row m is X[m * ldx + (k / xseg_len) * xseg_stride + k % xseg_len].
  int32_t xseg_len, xseg_stride;
  float eps;               // skinny GEMM with a fused RMSNorm
  const int32_t *row_on;   // skinny GEMM: row m is stored only where row_on[m] (null: all rows)
  // skinny GEMM layouts: X / Y / res in T16 (ld ignored) instead of row-major.  Its W must be
  // packed (w_packed = 1) as [N/16][K/32][64 lanes][8] (each k step of a 16-column tile is
  // 1 KiB contiguous).
  int32_t x_t16, y_t16, r_t16, w_packed;
  // skinny GEMM, EPI_STORE: instead of Y, each workgroup (16 columns) stores every row's
  // largest order key (value, lowest column) at keys_out[m * keys_row + blockIdx.x].
  uint64_t *keys_out;
  int64_t keys_row;
  // matrix-core GEMMs: a launch of few workgroups may split K over grid z, each split storing
  // its raw sums to split_ws[z][M][N] (SwiGLU: [z][M][2N], the up sums at N + n; split_cap
  // floats available); a second kernel adds the splits in order and applies the epilogue.
  // Null: never split.
  float *split_ws;
  int64_t split_cap;
  // skinny GEMM, EPI_RESIDUAL, T16 Y: K split in two halves over grid y.  Each half adds its
  // sums to Y with an fp32 atomic add, so Y must hold zeros; two adds onto zero commute, so
  // the result does not depend on their order.  The first half also adds the residual, and
  // then stores zero to res_zero (T16, may be res itself) at the same element: the buffer
  // the next split GEMM of the chain accumulates into.
  int32_t split2;
  float *res_zero;
  // skinny GEMM: mb = 2 runs two 16-row blocks (two positions of the same stream rows, row m
  // of either block masked by row_on[m]) against one pass over W.  Block 1 of a T16 operand
  // starts 16 * K (X) or 16 * N (Y, res, res_zero) elements after block 0; of a row-major one,
  // x_blk / r_blk / y_blk elements after.
  int32_t mb;
  int64_t x_blk, r_blk, y_blk;
  // skinny GEMM: weights read with non-temporal loads (weights read once per step, e.g. the
  // Talker's, so that they do not displace weights that are reread from the last-level cache).
  int32_t w_nt;
};

// Prompt prefill attention over rows at positions pos0 .. pos0 + P - 1.
struct PrefillAttnArgs {
  float *qkv;           // [P][ldq] raw projections (q normalised + rotated in place)
  const float *gq, *gk; // q_norm / k_norm gains
  const float2 *rope;   // [cap][d/2]
  void *kcache, *vcache;// [kv_heads][cap][d]
  float *out;           // [P][ldo] attention output
  int32_t P, pos0, ldq, ldo, q_heads, kv_heads, cap;
  float eps, scale;
  int32_t kv_bf16;
  // launch_prefix_attention with the output projection fused (wo set): wo [wo_rows][q_heads*d]
  // bf16; row p's per-KV-head shares at opart + p * opart_row + h * wo_rows.
  const uint16_t *wo;
  int32_t wo_rows;
  float *opart;
  int64_t opart_row;
  // launch_prefix_attention_rows (stream rows, grid z = row r, no fused projection): row r
  // reads position p's projections at qkv + r * ldq + p * ld_pos, its caches at kcache /
  // vcache + r * kv_row elements and its state at st + r (nothing is done for an ended or
  // masked row), and writes T16 blocks: position p at out + p * 16 * ldo (ldo = q_heads * d).
  int64_t ld_pos, kv_row;
  const SlotState *st;
  const int32_t *row_on;
};

// The prompt prefill attention of several streams in one launch (segment s = one stream's
// P[s] prompt rows, rows row0[s] .. row0[s] + P[s] - 1 of qkv / out, positions 0 .. P[s] - 1
// of its caches).  unit0[s] = first attention unit of segment s (units per segment:
// ceil(P / 16) * q_heads), unit0[nseg] = all units.
constexpr int kMaxPrefillSegs = 16;
struct PrefillBatchArgs {
  float *qkv;            // [M][ldq] raw projections (q normalised + rotated in place)
  const float *gq, *gk;  // q_norm / k_norm gains
  const float2 *rope;    // [cap][d/2]
  float *out;            // [M][ldo] attention output
  int32_t M, ldq, ldo, q_heads, kv_heads, cap, nseg, kv_bf16;
  float eps, scale;
  int32_t row0[kMaxPrefillSegs], P[kMaxPrefillSegs], unit0[kMaxPrefillSegs + 1];
  void *kcache[kMaxPrefillSegs], *vcache[kMaxPrefillSegs];  // [kv_heads][cap][d] of the layer
};

struct SelectTalkerArgs {
  const float *logits;      // [V] raw codec-head logits
  const float *x;           // [H] Talker output before the final norm
  const float *gamma;       // [H] talker.model.norm
  const uint16_t *codec_emb;// [V][H] bf16
  float *cp_prefix;         // [2][H]: normed hidden ; codec_emb[token]
  int32_t *codes;           // [max_frames][groups]
  float *trace;             // [max_frames + 1][V] or null
  SlotState *st;
  const SlotParams *prm;
  int32_t V, H, groups;
  float eps;
  int32_t after_frame;      // 0: token drawn after the prefill; 1: after the current frame
  // Stream rows (grid x): row r uses logits + r * V, x + r * H, cp_prefix + r * 2H,
  // codes + r * codes_row, trace + r * trace_row, st + r, prm + r; rows where row_on is 0
  // are skipped (row_on null: one stream).
  int64_t codes_row, trace_row;
  const int32_t *row_on;
  int32_t x_t16;            // x is a T16 block (row r = stream row r) instead of x + r * H
  int32_t end_frame;        // also end the frame: advance the counter by after_frame, EOS / max_frames
};

struct SelectCpArgs {
  const float *logits;        // [Vc]
  const uint16_t *emb;        // [Vc][Ht] codec_embedding.g (bf16)
  float *cur;                 // [Ht] embedding of the chosen token (next CP input)
  float *emb_sum;             // [Ht]
  int32_t *codes;
  float *trace;               // [max_frames][groups-1][Vc] or null
  // last group only: next Talker input = (codec_emb[semantic] + emb_sum) + trailing row
  float *talker_in;
  const uint16_t *codec_emb;  // [Vt][Ht]
  const float *trailing;      // [trailing_rows + 1][Ht], last row = tts_pad
  SlotState *st;
  const SlotParams *prm;
  int32_t Vc, Ht, groups, group;
  // Stream rows (grid x): logits + r * Vc; cur, emb_sum, talker_in + r * Ht; codes, trace,
  // trailing + r * their row strides; st + r, prm + r.
  int64_t codes_row, trace_row, trailing_row;
  const int32_t *row_on;
  int32_t *tok_out;           // one stream: the chosen token is also stored here (or null)
  // tok_out set, not the last group: only the token and its code are stored; the next
  // group's hand-off attention (TokenHandoff::tok_in with emb) stores cur and emb_sum.
  int32_t token_only;
};

}  // namespace q3t
