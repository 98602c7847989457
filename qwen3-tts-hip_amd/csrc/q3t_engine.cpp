// Host engine behind the C ABI in include/q3t.h.
//
// Mirrors the reference crate's engine (piedshag/qwen3-tts-hip src/generation.rs,
// src/model/{talker,code_predictor,decode}.rs) with a MI355X-first execution model:
//   * bf16 weights kept in the checkpoint's [out, in] layout (rows contiguous along K),
//     packed per layer as [q | k | v], [o], [gate | up], [down];
//   * per-stream slots, each with its own bf16 KV caches, workspace and loop state;
//   * the whole frame (15 CodePredictor groups + the next Talker step + token selection)
//     enqueued as one sequence of kernels whose varying inputs (frame index, position,
//     tokens, EOS) live in device memory, so it is captured once as a hipGraph and
//     replayed; the host synchronises once per chunk.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstddef>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "../../include/q3t.h"
#include "q3t_codec.h"
#include "q3t_device.h"
#include "q3t_host.h"
#include "q3t_json.h"
#include "q3t_kernels.h"

namespace q3t {
namespace {

thread_local std::string g_last_error;

template <typename F>
int guarded(F &&f) {
  try {
    f();
    return Q3T_OK;
  } catch (const Failure &e) {
    g_last_error = e.msg;
    return e.code;
  } catch (const std::exception &e) {
    g_last_error = e.what();
    return Q3T_ERR_INVALID;
  }
}

// ------------------------------------------------------------------------------------
// model
// ------------------------------------------------------------------------------------
struct Dims {
  int hidden, intermediate, layers, q_heads, kv_heads, head_dim, vocab;
  float eps, theta;
  int q_out() const { return q_heads * head_dim; }
  int kv_out() const { return kv_heads * head_dim; }
  int qkv_rows() const { return q_out() + 2 * kv_out(); }
  size_t layer_elems() const {
    return (size_t)qkv_rows() * hidden + (size_t)hidden * q_out() + 2 * (size_t)intermediate * hidden +
           (size_t)hidden * intermediate;
  }
};

Dims dims_from(const json::Value &c) {
  Dims d;
  d.hidden = (int)c.at("hidden_size").integer();
  d.intermediate = (int)c.at("intermediate_size").integer();
  d.layers = (int)c.at("num_hidden_layers").integer();
  d.q_heads = (int)c.at("num_attention_heads").integer();
  d.kv_heads = (int)c.at("num_key_value_heads").integer();
  d.head_dim = (int)c.at("head_dim").integer();
  d.vocab = (int)c.at("vocab_size").integer();
  d.eps = (float)c.at("rms_norm_eps").number();
  d.theta = (float)c.at("rope_theta").number();
  return d;
}

struct LayerW {
  const uint16_t *qkv, *o, *gu, *down;
  const float *g_in, *g_post, *gq, *gk;
  // The same matrices in the skinny GEMM's packed layout (multi-stream engines only).
  const uint16_t *qkv_p = nullptr, *o_p = nullptr, *gu_p = nullptr, *down_p = nullptr;
};

struct StackW {
  Dims d;
  std::vector<LayerW> layers;
  uint16_t *mats = nullptr;
  uint16_t *mats_p = nullptr;  // packed copy, same offsets
  float *gains = nullptr;
  float2 *rope = nullptr;  // [cap][head_dim / 2]
  int cap = 0;
};

void load_stack(const SafeTensors &st, const std::string &prefix, const Dims &d, int cap, StackW &w,
                int64_t &tally) {
  w.d = d;
  w.cap = cap;
  std::vector<uint16_t> mats;
  mats.reserve(d.layer_elems() * d.layers);
  std::vector<float> gains;
  const int64_t H = d.hidden, I = d.intermediate, Q = d.q_out(), KV = d.kv_out(), D = d.head_dim;
  struct Off {
    size_t qkv, o, gu, down, g_in, g_post, gq, gk;
  };
  std::vector<Off> offs;
  for (int l = 0; l < d.layers; ++l) {
    const std::string p = prefix + ".layers." + std::to_string(l);
    Off o;
    o.qkv = mats.size();
    st.append_bf16(p + ".self_attn.q_proj.weight", {Q, H}, mats);
    st.append_bf16(p + ".self_attn.k_proj.weight", {KV, H}, mats);
    st.append_bf16(p + ".self_attn.v_proj.weight", {KV, H}, mats);
    o.o = mats.size();
    st.append_bf16(p + ".self_attn.o_proj.weight", {H, Q}, mats);
    o.gu = mats.size();
    st.append_bf16(p + ".mlp.gate_proj.weight", {I, H}, mats);
    st.append_bf16(p + ".mlp.up_proj.weight", {I, H}, mats);
    o.down = mats.size();
    st.append_bf16(p + ".mlp.down_proj.weight", {H, I}, mats);
    auto add = [&](const std::string &n, int64_t len) {
      const size_t at = gains.size();
      auto v = st.f32(n, {len});
      gains.insert(gains.end(), v.begin(), v.end());
      return at;
    };
    o.g_in = add(p + ".input_layernorm.weight", H);
    o.g_post = add(p + ".post_attention_layernorm.weight", H);
    o.gq = add(p + ".self_attn.q_norm.weight", D);
    o.gk = add(p + ".self_attn.k_norm.weight", D);
    offs.push_back(o);
  }
  w.mats = dev_alloc<uint16_t>(mats.size(), tally);
  HIPC(hipMemcpy(w.mats, mats.data(), mats.size() * 2, hipMemcpyHostToDevice));
  w.gains = dev_alloc<float>(gains.size(), tally);
  HIPC(hipMemcpy(w.gains, gains.data(), gains.size() * 4, hipMemcpyHostToDevice));
  for (auto &o : offs)
    w.layers.push_back(LayerW{w.mats + o.qkv, w.mats + o.o, w.mats + o.gu, w.mats + o.down, w.gains + o.g_in,
                              w.gains + o.g_post, w.gains + o.gq, w.gains + o.gk});
  // RoPE table: angle = pos * theta^(-2i/d), evaluated in double and stored as float.
  const int half = d.head_dim / 2;
  std::vector<float2> rope((size_t)cap * half);
  for (int p = 0; p < cap; ++p)
    for (int i = 0; i < half; ++i) {
      const double inv = std::pow((double)d.theta, -(2.0 * i) / (double)d.head_dim);
      const double ang = (double)p * inv;
      rope[(size_t)p * half + i] = make_float2((float)std::cos(ang), (float)std::sin(ang));
    }
  w.rope = dev_alloc<float2>(rope.size(), tally);
  HIPC(hipMemcpy(w.rope, rope.data(), rope.size() * sizeof(float2), hipMemcpyHostToDevice));
}

struct Slot {
  bool in_use = false;
  // Views into the engine's pools (row `index` of each).
  char *t_k = nullptr, *t_v = nullptr, *c_k = nullptr, *c_v = nullptr;  // KV caches (fp32 or bf16)
  float *x_t, *t_in, *qkv, *attn, *act, *logits_t, *logits_c, *x_c, *cp_prefix, *cp_in, *cur, *emb_sum;
  float *trailing;
  float *attn_part;      // attention partials [kv_heads][chunks][G][2 + head_dim]
  int attn_part_chunks = 0;
  // Head-split O projections (the CodePredictor's fused into its attention, the 0.6B
  // Talker's after its split attention): per-KV-head shares of the projection
  // [kv_heads][hidden], and the residual row they sum to (stored by the gate/up GEMV).
  float *opart = nullptr, *x_mid = nullptr;
  int32_t *codes;
  SlotState *st;
  SlotParams *prm;
  float *trace_t = nullptr, *trace_c = nullptr;
  hipStream_t stream = nullptr;
  hipGraphExec_t graph = nullptr;
  hipGraphExec_t graph_long = nullptr;  // the same frame with the split Talker attention
  bool graph_traced = false;
  bool graph_cp_greedy = false;
  // The frame as separate graphs (q3t_debug_phase_times), keyed like `graph`: the
  // CodePredictor, the Talker step, and the Talker step with the split attention.
  hipGraphExec_t phase_graph[3] = {nullptr, nullptr, nullptr};
  bool phase_traced = false, phase_cp_greedy = false;
  SlotState *h_state = nullptr;  // pinned host mirror
  // Greedy CodePredictor (the stream's subtalker does not sample): each LM head hands its
  // argmax to the next group's first GEMV through cp_keys ([groups - 1][kHandoffKeys] order
  // keys) instead of a token selection kernel.
  uint64_t *cp_keys = nullptr;
  bool cp_greedy = false;
  int32_t *tok_cur = nullptr;  // the token the last CodePredictor selection kernel chose
};

// Per-stream device buffers for all slots, laid out as rows: slot i's buffer is
// base + i * (its row stride), so a batched kernel addresses stream row r directly and a
// single-stream launch is the one-row case.  The prefill workspace is shared: one prefill
// (of one or several streams) runs at a time.
struct Pools {
  int n = 0;
  size_t t_kv_row = 0, c_kv_row = 0;  // KV elements per slot (K or V, all layers)
  int s_qkv = 0, s_attn = 0, s_act = 0;
  int part_chunks = 0;
  // The batched frame splits the Talker's attention into shorter chunks (more workgroups,
  // fewer bytes each) than one stream can: its partials are merged by k_attn_merge
  // (attn_rows_chunk_len: 32 rows up to a 2,048-row cache, longer chunks beyond).
  int rows_part_chunks = 0;
  int64_t part_row = 0, trailing_row = 0, codes_row = 0, trace_t_row = 0, trace_c_row = 0, s_opart = 0;
  char *t_k = nullptr, *t_v = nullptr, *c_k = nullptr, *c_v = nullptr;
  float *x_t = nullptr, *t_in = nullptr, *qkv = nullptr, *attn = nullptr, *act = nullptr, *logits_t = nullptr,
        *logits_c = nullptr, *x_c = nullptr, *cp_prefix = nullptr, *cp_in = nullptr, *cur = nullptr,
        *emb_sum = nullptr, *trailing = nullptr, *attn_part = nullptr, *trace_t = nullptr, *trace_c = nullptr,
        *opart = nullptr, *x_mid = nullptr;
  int32_t *codes = nullptr;
  uint64_t *cp_keys = nullptr;                          // [n][groups - 1][kHandoffKeys]
  int32_t *tok_cur = nullptr;                           // [n]
  SlotState *st = nullptr;
  SlotParams *prm = nullptr;
  int32_t *row_on = nullptr;                            // [n] rows a batched launch covers
  int prefill_rows = 0;                                 // n * cap
  float *px = nullptr, *pqkv = nullptr, *pattn = nullptr, *pact = nullptr, *pinv = nullptr;
  SlotState *h_states = nullptr;                        // pinned [n]
  int32_t *h_codes = nullptr;                           // pinned [n][codes_row], mirrors codes
  int32_t *h_row_on = nullptr;                          // pinned [n]
  hipStream_t stream = nullptr;                         // batched work
  // The batched frame's graphs, one per (rows, fused), all captured with the trace setting
  // graphs_traced: a ragged batch changes its row count as streams end, and each count keeps
  // its graph instead of capturing again in every generation.
  hipGraphExec_t graphs[kMaxRows + 1][2] = {};
  bool graphs_traced = false;
  void drop_graphs() {
    for (auto &byrows : graphs)
      for (hipGraphExec_t &g : byrows)
        if (g) {
          (void)hipGraphExecDestroy(g);
          g = nullptr;
        }
  }
};

// One stream's rows in a (possibly multi-stream) prompt prefill.
struct PrefillSeg {
  int slot, row0, P;
};

}  // namespace

struct Engine {
  int device = 0;
  int cap = 512;
  int use_graph = 1;
  int kv_bf16 = 0;
  int trace = 0;
  int groups = 16;
  int codec_eos = 2150;
  Dims td{}, cd{};
  int talker_hidden = 0;
  bool has_proj = false;
  StackW talker, cp;
  uint16_t *codec_head = nullptr, *codec_emb = nullptr;  // [Vt][Ht]
  float *t_norm = nullptr, *c_norm = nullptr;
  uint16_t *lm_heads = nullptr;  // [groups-1][Vc][Hc]
  uint16_t *cp_emb = nullptr;    // [groups-1][Vc][Ht]
  uint16_t *proj_w = nullptr;    // [Hc][Ht]
  float *proj_b = nullptr;
  // Greedy hand-off tables (built at load): for CodePredictor groups 1 .. groups-2, the layer-0
  // raw q/k/v row of every input token, [groups-2][Vc][qkv_rows], and (projection only) the
  // projected input row, [groups-2][Vc][Hc].
  float *cp_qkv_table = nullptr, *cp_in_table = nullptr;
  // K-split partial sums of prompt-prefill and text-projection GEMMs over few rows
  static constexpr int64_t kSplitFloats = (int64_t)4 << 20;
  float *split_ws = nullptr;
  // result of resolving the device's no-allocation scratch at creation
  hipError_t scratch_status = hipErrorNotInitialized;
  // Prompt preparation on the device (text.rs:516-603), when the checkpoint holds
  // talker.model.text_embedding.weight: the table [text_vocab][text_hidden] and the text
  // projection fc1 [tp_inter][text_hidden] + bias, fc2 [H][tp_inter] + bias.
  uint16_t *text_emb = nullptr, *tp_fc1 = nullptr, *tp_fc2 = nullptr;
  float *tp_b1 = nullptr, *tp_b2 = nullptr;
  int text_vocab = 0, text_hidden = 0, tp_inter = 0;
  // Special ids (config.rs:30-44).
  int tok_im_start = 0, tok_assistant = 0, tok_tts_pad = 0, tok_tts_bos = 0, tok_tts_eos = 0;
  int codec_pad = 0, codec_bos = 0, codec_think = 0, codec_think_bos = 0, codec_think_eos = 0;
  std::map<std::string, int> speaker_ids, language_ids;
  // Codec decoder (speech_tokenizer/model.safetensors under the model directory), or null.
  Codec *codec = nullptr;
  // Packed copies for the batched frame's skinny GEMMs (multi-stream engines only).
  uint16_t *codec_head_p = nullptr, *lm_heads_p = nullptr, *proj_w_p = nullptr;
  // Batched-frame activations in T16 (16 stream rows): residual streams, attention output,
  // MLP activation, projected CodePredictor inputs.
  float *bx_t = nullptr, *bx_c = nullptr, *battn = nullptr, *bact = nullptr, *bcp_in = nullptr;
  // The mid-layer residual (after attention) of the K-split O / down GEMMs: all zeros
  // except between a layer's O GEMM, which accumulates into it, and its down GEMM, which
  // reads it as the residual and zeroes it again.
  float *bmid = nullptr;
  size_t bmid_floats = 0;
  // Set when batched frames stopped with an error, possibly between a split O GEMM and its
  // down GEMM (bmid then holds partial sums): the next batched call zeroes bmid first.
  bool bmid_dirty = false;
  // The two-block prefix pass's q/k/v rows: [2 positions][16 rows][qkv_rows] (row-major).
  float *bqkv2 = nullptr;
  std::vector<Slot> slots;
  Pools pools;
  bool rows_ok = false;  // the batched frame's fused-norm GEMMs support both hidden sizes
  // Talker positions below this run the fused attention + O kernel (talker_heads_o), from it
  // the split attention and the merging O GEMV: each fused workgroup reads its head's whole
  // cache.  Whole 0.6B frames (ms, every frame split / fused), fp32 cache: positions 16-255
  // 1.720 / 1.691, 129-248 1.729 / 1.731, 256-375 1.841 / 1.899, 509-628 1.934 / 2.088, so
  // they cross near 190 rows (config 2 at limits 256 / 224 / 192 / 160: 589.5 / 590.7 /
  // 590.8 / 590.5 frames/s); bf16 cache (half the bytes per row): 1.703 / 1.655, 1.709 /
  // 1.678, 1.733 / 1.753, 1.820 / 1.918, crossing near 265.  Set at engine creation by the
  // cache's type; q3t_engine_set_fused_attention_rows changes it.
  static constexpr int kFusedAttnRowsF32 = 192, kFusedAttnRowsBf16 = 256;
  int fused_attn_rows = kFusedAttnRowsF32;
  int64_t device_bytes = 0;

  // nt: stream the weights with non-temporal loads (Talker weights are read once per frame).
  void gemv(int epi, bool norm, const uint16_t *W, const float *x, const float *gamma, float eps,
            const float *res, const float *bias, float *out, int N, int K, int skip, const SlotState *st,
            hipStream_t s, bool nt = false, const LaunchTiming *timing = nullptr) {
    GemvArgs a{W, x, gamma, res, bias, out, N, K, eps, skip, st};
    hip_check(launch_gemv(epi, norm, nt, a, s, timing), "launch_gemv");
  }

  // The CodePredictor's attention fits one chunk (16 rows), so its O projection can be fused
  // into the attention kernel (launch_attn_oproj) with the residual summed by the gate/up
  // GEMV: one launch fewer per layer.
  bool oproj_ok(const StackW &w) const {
    const Dims &d = w.d;
    return &w == &cp && w.cap <= 32 && d.kv_heads <= 8 &&
           (d.hidden == 512 || d.hidden == 1024);
  }

  // The Talker's attention runs with its O projection fused in, split by KV head
  // (launch_attn_oproj_full), the shares summed into the residual by the gate/up GEMV, when
  // its hidden size takes the partial-sum GEMV (512 or 1024: the 0.6B Talker) and the cache
  // fits the fused kernel (33 .. 1024 rows).  Otherwise the split attention's partials are
  // merged by the O GEMV.
  bool talker_heads_o(const StackW &w) const {
    const Dims &d = w.d;
    const int rows = attn_oproj_full_rows(d.q_heads, d.kv_heads);
    return &w == &talker && attn_chunks(w.cap) > 1 && attn_chunks(w.cap) <= kAttnGemvMergeChunks &&
           d.kv_heads <= 8 && (d.hidden == 512 || d.hidden == 1024) && rows > 0 && d.hidden % rows == 0;
  }

  // One decoder-stack step for one position (decode.rs:951-1001 / 1300-1475).
  // handoff: layer 0 takes its raw q/k/v row from qkv_table (row = the handed-off token) in its
  // attention kernel and runs no QKV GEMV; `in` is then the row that kernel stores
  // (handoff->cur).
  // tin (the Talker after a greedy CodePredictor): layer 0's QKV GEMV assembles its input from
  // the last group's hand-off (GemvArgs::tin) and stores it to `in`.
  void stack_step(const StackW &w, char *kc, char *vc, const float *in, float *x, Slot &sl, int pos_mode,
                  int pos_const, int skip, hipStream_t s, const TokenHandoff *handoff = nullptr,
                  const float *qkv_table = nullptr, const GemvArgs *tin = nullptr, bool split_attn = false) {
    const Dims &d = w.d;
    const bool nt = &w == &talker;
    const bool fuse_o = oproj_ok(w);
    const size_t cache_layer = (size_t)d.kv_heads * w.cap * d.head_dim * (kv_bf16 ? 2 : 4);
    for (int l = 0; l < d.layers; ++l) {
      const LayerW &L = w.layers[l];
      const float *src = l == 0 ? in : x;
      const bool table = l == 0 && handoff;
      if (l == 0 && tin) {
        GemvArgs a = *tin;
        a.W = L.qkv; a.x = nullptr; a.gamma = L.g_in; a.out = sl.qkv; a.N = d.qkv_rows(); a.K = d.hidden;
        a.eps = d.eps; a.skip = skip; a.st = sl.st; a.tin_x = const_cast<float *>(in);
        hip_check(launch_gemv(EPI_STORE, true, nt, a, s), "launch_gemv(qkv, Talker input hand-off)");
      } else if (!table)
        gemv(EPI_STORE, true, L.qkv, src, L.g_in, d.eps, nullptr, nullptr, sl.qkv, d.qkv_rows(), d.hidden, skip,
             sl.st, s, nt);
      if (fuse_o) {
        // Attention and the O projection in one kernel (K split by KV head), the residual
        // sum in the gate/up GEMV, which also stores it (x_mid) for the down GEMV.
        AttnArgs aa{sl.qkv,   L.gq,      L.gk,       w.rope,  kc + l * cache_layer, vc + l * cache_layer,
                    nullptr,  d.q_heads, d.kv_heads, w.cap,   d.eps, 1.0f / std::sqrt((float)d.head_dim),
                    pos_mode, pos_const, skip,       kv_bf16, sl.st, nullptr, 0, attn_chunk_len(w.cap), 0};
        if (table) {
          aa.h = *handoff;
          aa.qkv_table = qkv_table;
          aa.ld_table = d.qkv_rows();
        }
        aa.wo = L.o;
        aa.wo_rows = d.hidden;
        aa.opart = sl.opart;
        hip_check(launch_attn_oproj(aa, d.head_dim, s), "launch_attn_oproj");
        GemvArgs gu{L.gu, src, L.g_post, nullptr, nullptr, sl.act, d.intermediate, d.hidden, d.eps, skip, sl.st};
        gu.parts = sl.opart;
        gu.n_parts = d.kv_heads;
        gu.ld_parts = d.hidden;
        gu.x_store = sl.x_mid;
        hip_check(launch_gemv(EPI_SWIGLU, true, false, gu, s), "launch_gemv(gate/up, partial sum)");
        gemv(EPI_RESIDUAL, false, L.down, sl.act, nullptr, 0.f, sl.x_mid, nullptr, x, d.hidden, d.intermediate, skip,
             sl.st, s, nt);
        continue;
      }
      if (!split_attn && talker_heads_o(w)) {
        // Attention and the O projection (K split by KV head) in one launch; the gate/up GEMV
        // sums the residual and the per-head shares, and stores that sum (x_mid) for down.
        AttnArgs aa{sl.qkv,   L.gq,      L.gk,       w.rope,  kc + l * cache_layer, vc + l * cache_layer,
                    nullptr,  d.q_heads, d.kv_heads, w.cap,   d.eps, 1.0f / std::sqrt((float)d.head_dim),
                    pos_mode, pos_const, skip,       kv_bf16, sl.st, nullptr, 0, attn_chunk_len(w.cap), 0};
        aa.wo = L.o;
        aa.wo_rows = d.hidden;
        aa.opart = sl.opart;
        hip_check(launch_attn_oproj_full(aa, d.head_dim, s), "launch_attn_oproj_full");
        GemvArgs gu{L.gu, src, L.g_post, nullptr, nullptr, sl.act, d.intermediate, d.hidden, d.eps, skip, sl.st};
        gu.parts = sl.opart;
        gu.n_parts = d.kv_heads;
        gu.ld_parts = d.hidden;
        gu.x_store = sl.x_mid;
        hip_check(launch_gemv(EPI_SWIGLU, true, nt, gu, s), "launch_gemv(gate/up, partial sum)");
        gemv(EPI_RESIDUAL, false, L.down, sl.act, nullptr, 0.f, sl.x_mid, nullptr, x, d.hidden, d.intermediate, skip,
             sl.st, s, nt);
        continue;
      }
      // The Talker's attention spans many chunks: partials, merged by the O projection.  The
      // CodePredictor's 16-row cache is one chunk: direct output.
      const int partial = attn_chunks(w.cap) > 1 ? 1 : 0;
      AttnArgs aa{sl.qkv,   L.gq,    L.gk,     w.rope,  kc + l * cache_layer, vc + l * cache_layer,
                  sl.attn,  d.q_heads, d.kv_heads, w.cap, d.eps, 1.0f / std::sqrt((float)d.head_dim),
                  pos_mode, pos_const, skip,    kv_bf16, sl.st,  sl.attn_part, sl.attn_part_chunks,
                  attn_chunk_len(w.cap), partial};
      if (table) {
        aa.h = *handoff;
        aa.qkv_table = qkv_table;
        aa.ld_table = d.qkv_rows();
      }
      hip_check(launch_attn_decode(aa, d.head_dim, s), "launch_attn_decode");
      // Up to kAttnGemvMergeChunks partials are merged inside the O projection; more (caches
      // past 1024 rows) by the merge kernel first.
      const bool merge_in_o = partial && attn_chunks(w.cap) <= kAttnGemvMergeChunks;
      if (partial && !merge_in_o) {
        AttnMergeArgs ma{sl.attn_part, sl.attn, d.q_heads, d.kv_heads, sl.attn_part_chunks, attn_chunk_len(w.cap),
                         pos_mode, pos_const, skip, d.q_out(), 0, sl.st, nullptr, 0};
        hip_check(launch_attn_merge(ma, 1, s), "launch_attn_merge");
      }
      GemvArgs og{L.o, sl.attn, nullptr, src, nullptr, x, d.hidden, d.q_out(), 0.f, skip, sl.st};
      if (merge_in_o) {
        og.x = nullptr;
        og.attn_part = sl.attn_part;
        og.attn_part_chunks = sl.attn_part_chunks;
        og.attn_chunk = attn_chunk_len(w.cap);
        og.attn_pos_mode = pos_mode;
        og.attn_pos_const = pos_const;
        og.attn_q_heads = d.q_heads;
        og.attn_kv_heads = d.kv_heads;
      }
      hip_check(launch_gemv(EPI_RESIDUAL, false, nt, og, s), "launch_gemv");
      gemv(EPI_SWIGLU, true, L.gu, x, L.g_post, d.eps, nullptr, nullptr, sl.act, d.intermediate, d.hidden, skip,
           sl.st, s, nt);
      gemv(EPI_RESIDUAL, false, L.down, sl.act, nullptr, 0.f, x, nullptr, x, d.hidden, d.intermediate, skip, sl.st,
           s, nt);
    }
  }

  // Talker prompt prefill on the matrix cores: every layer runs over the prompt rows of all
  // segments at once (decode.rs:845-880, 1077-1298), and so does attention, each segment
  // against its stream's own cache.  The prompt rows are in pools.px; each segment's last
  // row's output lands in its slot's x_t.
  void prefill_segments(const std::vector<PrefillSeg> &segs, int M, hipStream_t s) {
    const Dims &d = td;
    Pools &p = pools;
    const int H = d.hidden, Q = d.qkv_rows(), O = d.q_out(), I = d.intermediate;
    if (M <= 0 || M > p.prefill_rows) fail(Q3T_ERR_CAPACITY, "prefill of %d rows exceeds the workspace", M);
    const size_t esz = kv_bf16 ? 2 : 4;
    const size_t cache_layer = (size_t)d.kv_heads * talker.cap * d.head_dim * esz;
    for (int l = 0; l < d.layers; ++l) {
      const LayerW &L = talker.layers[l];
      hip_check(launch_row_rms(p.px, H, M, H, d.eps, p.pinv, s), "launch_row_rms");
      GemmArgs g{};
      g.X = p.px; g.ldx = H; g.row_scale = p.pinv; g.gamma = L.g_in;
      g.W = L.qkv; g.Y = p.pqkv; g.ldy = Q; g.M = M; g.N = Q; g.K = H;
      g.split_ws = split_ws; g.split_cap = kSplitFloats;
      hip_check(launch_gemm(EPI_STORE, g, s), "launch_gemm(qkv)");
      PrefillBatchArgs pa{};
      pa.qkv = p.pqkv; pa.gq = L.gq; pa.gk = L.gk; pa.rope = talker.rope; pa.out = p.pattn;
      pa.M = M; pa.ldq = Q; pa.ldo = O; pa.q_heads = d.q_heads; pa.kv_heads = d.kv_heads; pa.cap = talker.cap;
      pa.nseg = (int)segs.size(); pa.kv_bf16 = kv_bf16; pa.eps = d.eps;
      pa.scale = 1.0f / std::sqrt((float)d.head_dim);
      for (int i = 0; i < pa.nseg; ++i) {
        const Slot &sl = slots[segs[i].slot];
        pa.row0[i] = segs[i].row0;
        pa.P[i] = segs[i].P;
        pa.unit0[i + 1] = pa.unit0[i] + (segs[i].P + 15) / 16 * d.q_heads;
        pa.kcache[i] = sl.t_k + l * cache_layer;
        pa.vcache[i] = sl.t_v + l * cache_layer;
      }
      hip_check(launch_prefill_attention(pa, s), "launch_prefill_attention");
      g = GemmArgs{};
      g.X = p.pattn; g.ldx = O; g.W = L.o; g.res = p.px; g.ldr = H; g.Y = p.px; g.ldy = H;
      g.M = M; g.N = H; g.K = O;
      g.split_ws = split_ws; g.split_cap = kSplitFloats;
      hip_check(launch_gemm(EPI_RESIDUAL, g, s), "launch_gemm(o)");
      hip_check(launch_row_rms(p.px, H, M, H, d.eps, p.pinv, s), "launch_row_rms");
      g = GemmArgs{};
      g.X = p.px; g.ldx = H; g.row_scale = p.pinv; g.gamma = L.g_post;
      g.W = L.gu; g.Y = p.pact; g.ldy = I; g.M = M; g.N = I; g.K = H;
      g.split_ws = split_ws; g.split_cap = kSplitFloats;
      hip_check(launch_gemm(EPI_SWIGLU, g, s), "launch_gemm(gate_up)");
      g = GemmArgs{};
      g.X = p.pact; g.ldx = I; g.W = L.down; g.res = p.px; g.ldr = H; g.Y = p.px; g.ldy = H;
      g.M = M; g.N = H; g.K = I;
      g.split_ws = split_ws; g.split_cap = kSplitFloats;
      hip_check(launch_gemm(EPI_RESIDUAL, g, s), "launch_gemm(down)");
    }
    for (const PrefillSeg &sg : segs)
      HIPC(hipMemcpyAsync(slots[sg.slot].x_t, p.px + (size_t)(sg.row0 + sg.P - 1) * H, (size_t)H * 4,
                          hipMemcpyDeviceToDevice, s));
  }

  // Talker token selection; end_frame = also the frame bookkeeping (counter, EOS, max_frames).
  void select_talker(Slot &sl, int after_frame, hipStream_t s, bool end_frame = true) {
    SelectTalkerArgs a{sl.logits_t, sl.x_t, t_norm, codec_emb, sl.cp_prefix, sl.codes,
                       trace ? sl.trace_t : nullptr, sl.st, sl.prm, td.vocab, td.hidden, groups, td.eps,
                       after_frame};
    a.end_frame = end_frame ? 1 : 0;
    hip_check(launch_select_talker(a, s), "launch_select_talker");
  }

  // Everything one frame does after its semantic token is known (generation.rs:697-741):
  // CodePredictor groups 0..14, the next Talker step, token selection, frame bookkeeping.
  void enqueue_frame(Slot &sl, hipStream_t s, bool split_attn = false) {
    const bool fold = fold_last_group(sl);
    enqueue_code_predictor(sl, s, fold);
    enqueue_talker_decode(sl, s, fold, split_attn);
  }

  // A greedy CodePredictor hands its last group's token to the Talker step that follows
  // (the Talker's layer-0 QKV GEMV assembles its own input: GemvArgs::tin) instead of
  // running a selection kernel.  Both halves of the frame must agree on it.
  bool fold_last_group(const Slot &sl) const {
    return sl.cp_greedy && cp_qkv_table &&
           (talker_hidden == 512 || talker_hidden == 1024 || talker_hidden == 2048);
  }

  void enqueue_talker_decode(Slot &sl, hipStream_t s, bool fold = false, bool split_attn = false) {
    if (fold) {
      const int Vc = cd.vocab, nac = groups - 1;
      GemvArgs tin{};
      tin.tin.keys = sl.cp_keys + (size_t)(nac - 1) * kHandoffKeys;
      tin.tin.n_keys = gemv_grid_for(Vc, cd.hidden);
      tin.tin.emb = cp_emb + (size_t)(nac - 1) * Vc * talker_hidden;
      tin.tin.emb_width = talker_hidden;
      tin.tin.sum = sl.emb_sum;
      tin.tin.codes = sl.codes;
      tin.tin.code = groups - 1;
      tin.tin.groups = groups;
      tin.tin_codec_emb = codec_emb;
      tin.tin_trailing = sl.trailing;
      stack_step(talker, sl.t_k, sl.t_v, sl.t_in, sl.x_t, sl, POS_TALKER_FRAME, 0, SKIP_TALKER, s, nullptr, nullptr,
                 &tin, split_attn);
    } else {
      stack_step(talker, sl.t_k, sl.t_v, sl.t_in, sl.x_t, sl, POS_TALKER_FRAME, 0, SKIP_TALKER, s, nullptr, nullptr,
                 nullptr, split_attn);
    }
    gemv(EPI_STORE, true, codec_head, sl.x_t, t_norm, td.eps, nullptr, nullptr, sl.logits_t, td.vocab, td.hidden,
         SKIP_TALKER, sl.st, s, true);
    select_talker(sl, 1, s);  // + frame bookkeeping
  }

  // The frame's CodePredictor (code_predictor.rs:366-471): prefix rows cp_prefix, then the 15
  // acoustic groups; codes[frame], emb_sum and the next Talker input t_in are its outputs.
  // A GEMV over two input rows (x, x + ldx_r) -> (out, out + ldo_r), one pass over W.
  void gemv2(int epi, bool norm, const uint16_t *W, const float *x, int ldx_r, const float *gamma, float eps,
             const float *res, int ldr_r, const float *bias, float *out, int ldo_r, int N, int K, const Slot &sl,
             hipStream_t s) {
    GemvArgs a{W, x, gamma, res, bias, out, N, K, eps, SKIP_DONE, sl.st};
    a.rows = 2;
    a.ldx_r = ldx_r;
    a.ldr_r = ldr_r;
    a.ldo_r = ldo_r;
    hip_check(launch_gemv(epi, norm, false, a, s), "launch_gemv(2 rows)");
  }

  // CodePredictor positions 0 and 1 (its 2-row prefix, code_predictor.rs:366-400) in one pass
  // per layer: two-row GEMVs and the prefill attention kernels at P = 2 (rows in the prefill
  // workspace, idle during frames).  Returns the position-1 output row.
  const float *cp_prefix_pass(const float *in, int ldin, Slot &sl, hipStream_t s) {
    const StackW &w = cp;
    const Dims &d = w.d;
    Pools &p = pools;
    const int H = d.hidden, Q = d.qkv_rows(), O = d.q_out(), I = d.intermediate;
    float *x2 = p.px;  // [2][H]
    const size_t cache_layer = (size_t)d.kv_heads * w.cap * d.head_dim * (kv_bf16 ? 2 : 4);
    for (int l = 0; l < d.layers; ++l) {
      const LayerW &L = w.layers[l];
      const float *src = l == 0 ? in : x2;
      const int lds = l == 0 ? ldin : H;
      gemv2(EPI_STORE, true, L.qkv, src, lds, L.g_in, d.eps, nullptr, 0, nullptr, p.pqkv, Q, Q, H, sl, s);
      PrefillAttnArgs pa{p.pqkv, L.gq, L.gk, w.rope, sl.c_k + l * cache_layer, sl.c_v + l * cache_layer, p.pattn,
                         2, 0, Q, O, d.q_heads, d.kv_heads, w.cap, d.eps, 1.0f / std::sqrt((float)d.head_dim),
                         kv_bf16};
      if (oproj_ok(w)) {
        // The O projection fused into the attention (per-head shares of both rows in pattn),
        // the residual sum in the two-row gate/up GEMV, which stores it to px rows 2, 3.
        float *x_mid2 = x2 + 2 * H;
        pa.wo = L.o;
        pa.wo_rows = H;
        pa.opart = p.pattn;
        pa.opart_row = (int64_t)d.kv_heads * H;
        hip_check(launch_prefix_attention(pa, s), "launch_prefix_attention(o projection)");
        GemvArgs gu{L.gu, src, L.g_post, nullptr, nullptr, p.pact, I, H, d.eps, SKIP_DONE, sl.st};
        gu.rows = 2;
        gu.ldx_r = lds;
        gu.ldo_r = I;
        gu.parts = p.pattn;
        gu.n_parts = d.kv_heads;
        gu.ld_parts = H;
        gu.ldp_r = d.kv_heads * H;
        gu.x_store = x_mid2;
        gu.ldxs_r = H;
        hip_check(launch_gemv(EPI_SWIGLU, true, false, gu, s), "launch_gemv(2 rows, partial sum)");
        gemv2(EPI_RESIDUAL, false, L.down, p.pact, I, nullptr, 0.f, x_mid2, H, nullptr, x2, H, H, I, sl, s);
        continue;
      }
      hip_check(launch_prefix_attention(pa, s), "launch_prefix_attention");
      gemv2(EPI_RESIDUAL, false, L.o, p.pattn, O, nullptr, 0.f, src, lds, nullptr, x2, H, H, O, sl, s);
      gemv2(EPI_SWIGLU, true, L.gu, x2, H, L.g_post, d.eps, nullptr, 0, nullptr, p.pact, I, I, H, sl, s);
      gemv2(EPI_RESIDUAL, false, L.down, p.pact, I, nullptr, 0.f, x2, H, nullptr, x2, H, H, I, sl, s);
    }
    return x2 + H;
  }

  // fold (fold_last_group): the last group's LM head stores hand-off keys for the Talker step
  // that follows instead of running a selection kernel; codes[frame][groups - 1] and the next
  // Talker input are then stored by that step.
  void enqueue_code_predictor(Slot &sl, hipStream_t s, bool fold = false) {
    const int Ht = talker_hidden, Hc = cd.hidden, Vc = cd.vocab, nac = groups - 1;
    const float *in = sl.cp_prefix;
    int ldin = Ht;
    if (has_proj) {
      gemv2(EPI_BIAS, false, proj_w, sl.cp_prefix, Ht, nullptr, 0.f, nullptr, 0, proj_b, sl.cp_in, Hc, Hc, Ht, sl, s);
      in = sl.cp_in;
      ldin = Hc;
    }
    const float *x_pos1 = cp_prefix_pass(in, ldin, sl, s);
    // Greedy (tables built): groups 0 .. nac-2 hand their token from the LM head to the next
    // group's layer-0 attention, which reads that token's precomputed q/k/v row; the last
    // group's selection kernel also writes the next Talker input.
    const bool fused = sl.cp_greedy && cp_qkv_table;
    // Sampled groups take the tables too (the token from the selection kernel), when the
    // model has no projection and the attention has the fused O projection.
    const bool sampled_tables = !fused && cp_qkv_table && !has_proj && oproj_ok(cp);
    for (int g = 0; g < nac; ++g) {
      if (g > 0) {
        const float *in = sl.cur;
        if (fused) {
          TokenHandoff t{};
          t.keys = sl.cp_keys + (size_t)(g - 1) * kHandoffKeys;
          t.n_keys = gemv_grid_for(Vc, Hc);
          t.emb = cp_emb + (size_t)(g - 1) * Vc * Ht;
          t.emb_width = Ht;
          t.cur = sl.cur;
          t.sum = sl.emb_sum;
          t.codes = sl.codes;
          t.first = g == 1;
          t.code = g;
          t.groups = groups;
          if (has_proj) {  // layer 0's input is the projected row: from its table, to cp_in row 2
            t.cur_table = cp_in_table + (size_t)(g - 1) * Vc * Hc;
            t.cur_width = Hc;
            t.cur = sl.cp_in + 2 * Hc;
            in = t.cur;
          }
          stack_step(cp, sl.c_k, sl.c_v, in, sl.x_c, sl, POS_CONST, g + 1, SKIP_DONE, s, &t,
                     cp_qkv_table + (size_t)(g - 1) * Vc * cd.qkv_rows());
        } else if (sampled_tables) {
          // the previous group's selection kernel chose the token (tok_cur): layer 0 takes the
          // token's q/k/v table row, and its workgroup (0, 0) stores the token's embedding row
          // (cur, the layer's residual input) and the running sum, off the selection kernel's
          // critical path
          TokenHandoff t{};
          t.tok_in = sl.tok_cur;
          t.emb = cp_emb + (size_t)(g - 1) * Vc * Ht;
          t.emb_width = Ht;
          t.cur = sl.cur;
          t.sum = sl.emb_sum;
          t.codes = sl.codes;
          t.first = g == 1;
          t.code = g;
          t.groups = groups;
          stack_step(cp, sl.c_k, sl.c_v, in, sl.x_c, sl, POS_CONST, g + 1, SKIP_DONE, s, &t,
                     cp_qkv_table + (size_t)(g - 1) * Vc * cd.qkv_rows());
        } else {
          if (has_proj) {
            gemv(EPI_BIAS, false, proj_w, sl.cur, nullptr, 0.f, nullptr, proj_b, sl.cp_in + 2 * Hc, Hc, Ht,
                 SKIP_DONE, sl.st, s);
            in = sl.cp_in + 2 * Hc;
          }
          stack_step(cp, sl.c_k, sl.c_v, in, sl.x_c, sl, POS_CONST, g + 1, SKIP_DONE, s);
        }
      }
      GemvArgs a{lm_heads + (size_t)g * Vc * Hc, g == 0 ? x_pos1 : sl.x_c, c_norm, nullptr, nullptr, sl.logits_c,
                 Vc, Hc, cd.eps, SKIP_DONE, sl.st};
      if (fused && (g < nac - 1 || fold)) {
        a.keys_out = sl.cp_keys + (size_t)g * kHandoffKeys;
        if (trace) {
          a.trace = sl.trace_c + (size_t)g * Vc;
          a.trace_frame = (int64_t)(groups - 1) * Vc;
        }
        hip_check(launch_gemv(EPI_STORE, true, false, a, s), "launch_gemv(lm_head hand-off)");
        continue;
      }
      hip_check(launch_gemv(EPI_STORE, true, false, a, s), "launch_gemv(lm_head)");
      SelectCpArgs sa{sl.logits_c, cp_emb + (size_t)g * Vc * Ht, sl.cur, sl.emb_sum, sl.codes,
                      trace ? sl.trace_c : nullptr, sl.t_in, codec_emb, sl.trailing, sl.st, sl.prm, Vc, Ht, groups,
                      g};
      sa.tok_out = sl.tok_cur;
      sa.token_only = sampled_tables && g < nac - 1;
      hip_check(launch_select_cp(sa, s), "launch_select_cp");
    }
  }

  // The greedy hand-off covers the CodePredictor's shapes: LM heads over K = Hc in 512, 1024
  // or 2048 with at most kHandoffKeys workgroups, embedding rows (Ht) of at most 2048, and
  // table GEMMs the matrix-core prefill path takes (Hc % 32 == 0, q/k/v rows % 128 == 0).
  bool handoff_ok() const {
    auto k_ok = [](int k) { return k == 512 || k == 1024 || k == 2048; };
    return k_ok(cd.hidden) && talker_hidden <= 2048 && talker_hidden % 32 == 0 && cd.qkv_rows() % 128 == 0 &&
           cd.vocab >= 128 && gemv_grid_for(cd.vocab, cd.hidden) <= kHandoffKeys && groups > 2;
  }

  // The batched frame's hand-off: tables built, no Talker -> CodePredictor projection (layer
  // 0's input row would be T16), LM heads of whole 16-column tiles, no logit tracing.
  bool rows_handoff_ok() const {
    return cp_qkv_table && !has_proj && !trace && cd.vocab % 16 == 0 && cd.vocab / 16 <= kHandoffKeys;
  }

  // ----- stream rows: the batched frame over slots 0..rows-1, masked by pools.row_on -----

  // An activation operand of the batched frame: row-major with leading dimension ld, or a
  // T16 block (ld < 0).
  struct Act {
    const float *p;
    int ld;
  };
  static Act t16(const float *p) { return Act{p, -1}; }

  // Set by rows_stack_step while it runs the Talker's layers, whose weights a batched frame
  // reads once: rgemm and rgemm_split2 then load them non-temporally, so that they pass
  // without displacing the CodePredictor's weights, which every group rereads, from the
  // last-level cache.
  bool rows_w_nt = false;
  // The batched frame's O and down GEMMs split K in two (rgemm_split2) when both can.
  bool split2_ok(const Dims &d) const {
    return bmid && gemm_skinny_split2_supports(d.q_out()) && gemm_skinny_split2_supports(d.intermediate);
  }

  // Skinny matrix-core GEMM over the stream rows, packed weights Wp.
  void rgemm(int epi, bool norm, const uint16_t *Wp, Act X, const float *gamma, float eps, Act res,
             const float *bias, Act Y, int N, int K, int rows, hipStream_t s, uint64_t *keys_out = nullptr,
             int64_t keys_row = 0) {
    GemmArgs g{};
    g.X = X.p; g.ldx = X.ld < 0 ? K : X.ld; g.x_t16 = X.ld < 0;
    g.gamma = gamma; g.eps = eps; g.W = Wp; g.w_packed = 1;
    g.res = res.p; g.ldr = res.ld < 0 ? N : res.ld; g.r_t16 = res.ld < 0;
    g.bias = bias;
    g.Y = const_cast<float *>(Y.p); g.ldy = Y.ld < 0 ? N : Y.ld; g.y_t16 = Y.ld < 0;
    g.M = rows; g.N = N; g.K = K; g.row_on = pools.row_on;
    g.keys_out = keys_out; g.keys_row = keys_row;
    g.w_nt = rows_w_nt;
    hip_check(launch_gemm_skinny(epi, norm, g, s), "launch_gemm_skinny");
  }

  // One decoder-stack step of every stream row (each at its own position and cache).  The
  // residual stream x is a T16 block; `in` feeds layer 0.  With a hand-off, layer 0's
  // attention takes each row's q/k/v from qkv_table at its token and stores `in` itself.
  void rows_stack_step(const StackW &w, char *kc, char *vc, size_t kv_row, Act in, float *x, int rows, int pos_mode,
                       int pos_const, int skip, hipStream_t s, const TokenHandoff *handoff = nullptr,
                       const float *qkv_table = nullptr) {
    const Dims &d = w.d;
    Pools &p = pools;
    const int H = d.hidden;
    struct WntScope {
      bool &f;
      WntScope(bool &flag, bool v) : f(flag) { f = v; }
      ~WntScope() { f = false; }
    } wnt_scope(rows_w_nt, &w == &talker);
    const size_t cache_layer = (size_t)d.kv_heads * w.cap * d.head_dim * (kv_bf16 ? 2 : 4);
    const int chunk = attn_rows_chunk_len(w.cap);  // the CodePredictor's short cache: one 16-row chunk
    const int nch = (w.cap + chunk - 1) / chunk;
    const int partial = nch > 1 ? 1 : 0;
    const Act none{nullptr, 0};
    const bool split = split2_ok(d);
    for (int l = 0; l < d.layers; ++l) {
      const LayerW &L = w.layers[l];
      const Act src = l == 0 ? in : t16(x);
      const bool table = l == 0 && handoff;
      if (!table)
        rgemm(EPI_STORE, true, L.qkv_p, src, L.g_in, d.eps, none, nullptr, Act{p.qkv, p.s_qkv}, d.qkv_rows(), H,
              rows, s);
      AttnArgs aa{p.qkv,    L.gq,    L.gk,     w.rope,  kc + l * cache_layer, vc + l * cache_layer,
                  battn,    d.q_heads, d.kv_heads, w.cap, d.eps, 1.0f / std::sqrt((float)d.head_dim),
                  pos_mode, pos_const, skip,    kv_bf16, p.st,   p.attn_part, nch,
                  chunk,    partial};
      aa.ld_qkv = p.s_qkv;
      aa.ld_out = p.s_attn;
      aa.kv_row = (int64_t)kv_row;
      aa.part_row = p.part_row;
      aa.row_on = p.row_on;
      aa.out_t16 = 1;
      if (table) {
        aa.h = *handoff;
        aa.qkv_table = qkv_table;
        aa.ld_table = d.qkv_rows();
      }
      hip_check(launch_attn_decode(aa, d.head_dim, s, nullptr, rows), "launch_attn_decode(rows)");
      if (partial) {
        AttnMergeArgs m{p.attn_part, battn,     d.q_heads, d.kv_heads, nch,        chunk,
                        pos_mode,    pos_const, skip,      p.s_attn,   p.part_row, p.st,
                        p.row_on,    1};
        hip_check(launch_attn_merge(m, rows, s), "launch_attn_merge");
      }
      if (split) {
        // O: bmid (zeros) += src + W_o . attn in two K halves, the first half also zeroing x
        // (which the down GEMM then accumulates into); down: x += bmid + W_d . act, zeroing bmid.
        rgemm_split2(L.o_p, t16(battn), src, x, bmid, H, d.q_out(), rows, s);
        rgemm(EPI_SWIGLU, true, L.gu_p, t16(bmid), L.g_post, d.eps, none, nullptr, t16(bact), d.intermediate, H,
              rows, s);
        rgemm_split2(L.down_p, t16(bact), t16(bmid), bmid, x, H, d.intermediate, rows, s);
        continue;
      }
      rgemm(EPI_RESIDUAL, false, L.o_p, t16(battn), nullptr, 0.f, src, nullptr, t16(x), H, d.q_out(), rows, s);
      rgemm(EPI_SWIGLU, true, L.gu_p, t16(x), L.g_post, d.eps, none, nullptr, t16(bact), d.intermediate, H, rows, s);
      rgemm(EPI_RESIDUAL, false, L.down_p, t16(bact), nullptr, 0.f, t16(x), nullptr, t16(x), H, d.intermediate,
            rows, s);
    }
  }

  // Y (T16, zeros) += res + X . Wp^T over two K halves (GemmArgs::split2); the first half
  // stores zero to res_zero (T16) at each element it adds.
  // mb = 2: two row blocks (the prefix pass); a row-major res has its block 1 res_blk
  // elements after block 0.
  void rgemm_split2(const uint16_t *Wp, Act X, Act res, float *res_zero, float *Y, int N, int K, int rows,
                    hipStream_t s, int mb = 1, int64_t res_blk = 0) {
    GemmArgs g{};
    g.X = X.p; g.ldx = K; g.x_t16 = 1;
    g.W = Wp; g.w_packed = 1;
    g.res = res.p; g.ldr = res.ld < 0 ? N : res.ld; g.r_t16 = res.ld < 0; g.r_blk = res_blk;
    g.Y = Y; g.ldy = N; g.y_t16 = 1;
    g.M = rows; g.N = N; g.K = K; g.row_on = pools.row_on;
    g.split2 = 1; g.res_zero = res_zero; g.mb = mb;
    g.w_nt = mb == 1 && rows_w_nt;
    hip_check(launch_gemm_skinny(EPI_RESIDUAL, false, g, s), "launch_gemm_skinny(split2)");
  }

  // The CodePredictor's two prefix positions of every stream row in one pass per layer: the
  // skinny GEMMs run two 16-row blocks (block p = position p) against one read of each weight,
  // and one prefix-attention launch stores both positions' K/V rows and attends causally.
  // Position p's input is block p of `in` (T16, or row-major with block p in_blk elements
  // after block 0); block p of bx_c receives its output.  Needs prefix2_ok().
  void rows_prefix_pass(Act in, int64_t in_blk, int rows, hipStream_t s) {
    const StackW &w = cp;
    const Dims &d = w.d;
    Pools &p = pools;
    const int H = d.hidden, Q = d.qkv_rows(), O = d.q_out(), I = d.intermediate;
    const size_t cache_layer = (size_t)d.kv_heads * w.cap * d.head_dim * (kv_bf16 ? 2 : 4);
    for (int l = 0; l < d.layers; ++l) {
      const LayerW &L = w.layers[l];
      const Act src = l == 0 ? in : t16(bx_c);
      const int64_t src_blk = l == 0 ? in_blk : 0;
      GemmArgs g{};
      g.X = src.p; g.ldx = src.ld < 0 ? H : src.ld; g.x_t16 = src.ld < 0; g.x_blk = src_blk;
      g.gamma = L.g_in; g.eps = d.eps; g.W = L.qkv_p; g.w_packed = 1;
      g.Y = bqkv2; g.ldy = Q; g.y_blk = (int64_t)16 * Q;
      g.M = rows; g.N = Q; g.K = H; g.row_on = p.row_on; g.mb = 2;
      hip_check(launch_gemm_skinny(EPI_STORE, true, g, s), "launch_gemm_skinny(prefix qkv)");
      PrefillAttnArgs pa{bqkv2, L.gq, L.gk, w.rope, p.c_k + l * cache_layer, p.c_v + l * cache_layer, battn, 2, 0,
                         Q, O, d.q_heads, d.kv_heads, w.cap, d.eps, 1.0f / std::sqrt((float)d.head_dim), kv_bf16};
      pa.ld_pos = (int64_t)16 * Q;
      pa.kv_row = (int64_t)p.c_kv_row;
      pa.st = p.st;
      pa.row_on = p.row_on;
      hip_check(launch_prefix_attention_rows(pa, rows, s), "launch_prefix_attention_rows");
      rgemm_split2(L.o_p, t16(battn), src, bx_c, bmid, H, O, rows, s, 2, src_blk);
      g = GemmArgs{};
      g.X = bmid; g.ldx = H; g.x_t16 = 1;
      g.gamma = L.g_post; g.eps = d.eps; g.W = L.gu_p; g.w_packed = 1;
      g.Y = bact; g.ldy = I; g.y_t16 = 1;
      g.M = rows; g.N = I; g.K = H; g.row_on = p.row_on; g.mb = 2;
      hip_check(launch_gemm_skinny(EPI_SWIGLU, true, g, s), "launch_gemm_skinny(prefix gate/up)");
      rgemm_split2(L.down_p, t16(bact), t16(bmid), bmid, bx_c, H, I, rows, s, 2);
    }
  }

  // The two-block prefix pass applies: the split O / down GEMMs, and K = H within the
  // two-block RMSNorm GEMMs' sizes.
  bool prefix2_ok() const {
    auto k_ok = [](int k) { return k == 512 || k == 1024 || k == 2048; };
    return bqkv2 && split2_ok(cd) && k_ok(cd.hidden) && (!has_proj || k_ok(talker_hidden));
  }

  void select_talker_rows(int rows, int after_frame, Act x, hipStream_t s) {
    Pools &p = pools;
    SelectTalkerArgs a{p.logits_t, x.p, t_norm, codec_emb, p.cp_prefix, p.codes, trace ? p.trace_t : nullptr,
                       p.st, p.prm, td.vocab, td.hidden, groups, td.eps, after_frame};
    a.codes_row = p.codes_row;
    a.trace_row = p.trace_t_row;
    a.row_on = p.row_on;
    a.x_t16 = x.ld < 0;
    a.end_frame = 1;
    hip_check(launch_select_talker(a, s, rows), "launch_select_talker(rows)");
  }

  // enqueue_frame for stream rows 0..rows-1 at once: the weights of every pass are read
  // once for all rows (skinny matrix-core GEMMs); attention, selection and the loop state
  // are per row.  Rows that have ended or are masked out keep their state.
  //
  // fused (every live row greedy in the CodePredictor, rows_handoff_ok()): groups 0 .. nac-2
  // hand their tokens over as the single-stream frame does (per-row argmax keys from the LM
  // head, q/k/v table rows in the next group's layer-0 attention); only the last group runs
  // the selection kernel.
  void enqueue_rows_frame(int rows, bool fused, hipStream_t s) {
    Pools &p = pools;
    const int Ht = talker_hidden, Hc = cd.hidden, Vc = cd.vocab, nac = groups - 1;
    const int64_t keys_row = (int64_t)(groups - 1) * kHandoffKeys;
    const Act none{nullptr, 0};
    const size_t hc16 = (size_t)16 * Hc;
    Act in0{p.cp_prefix, 2 * Ht}, in1{p.cp_prefix + Ht, 2 * Ht};
    // group 0's LM head reads the prefix's position-1 output: block 1 of bx_c after the
    // two-block pass, else bx_c after the second one-position pass
    const float *x_pre = bx_c;
    if (prefix2_ok()) {
      Act in = in0;
      if (has_proj) {
        GemmArgs g{};
        g.X = p.cp_prefix; g.ldx = 2 * Ht; g.x_blk = Ht; g.W = proj_w_p; g.w_packed = 1; g.bias = proj_b;
        g.Y = bcp_in; g.ldy = Hc; g.y_t16 = 1;
        g.M = rows; g.N = Hc; g.K = Ht; g.row_on = p.row_on; g.mb = 2;
        hip_check(launch_gemm_skinny(EPI_BIAS, false, g, s), "launch_gemm_skinny(prefix projection)");
        in = t16(bcp_in);
      }
      rows_prefix_pass(in, has_proj ? 0 : Ht, rows, s);
      x_pre = bx_c + hc16;
    } else {
      if (has_proj) {
        rgemm(EPI_BIAS, false, proj_w_p, in0, nullptr, 0.f, none, proj_b, t16(bcp_in), Hc, Ht, rows, s);
        rgemm(EPI_BIAS, false, proj_w_p, in1, nullptr, 0.f, none, proj_b, t16(bcp_in + hc16), Hc, Ht, rows, s);
        in0 = t16(bcp_in);
        in1 = t16(bcp_in + hc16);
      }
      rows_stack_step(cp, p.c_k, p.c_v, p.c_kv_row, in0, bx_c, rows, POS_CONST, 0, SKIP_DONE, s);
      rows_stack_step(cp, p.c_k, p.c_v, p.c_kv_row, in1, bx_c, rows, POS_CONST, 1, SKIP_DONE, s);
    }
    for (int g = 0; g < nac; ++g) {
      if (g > 0 && fused) {
        TokenHandoff t{};
        t.keys = p.cp_keys + (size_t)(g - 1) * kHandoffKeys;
        t.keys_row = keys_row;
        t.n_keys = (Vc + 15) / 16;
        t.emb = cp_emb + (size_t)(g - 1) * Vc * Ht;
        t.emb_width = Ht;
        t.cur = p.cur;
        t.cur_row = Ht;
        t.sum = p.emb_sum;
        t.sum_row = Ht;
        t.codes = p.codes;
        t.codes_row = p.codes_row;
        t.first = g == 1;
        t.code = g;
        t.groups = groups;
        rows_stack_step(cp, p.c_k, p.c_v, p.c_kv_row, Act{p.cur, Ht}, bx_c, rows, POS_CONST, g + 1, SKIP_DONE, s, &t,
                        cp_qkv_table + (size_t)(g - 1) * Vc * cd.qkv_rows());
      } else if (g > 0) {
        Act in{p.cur, Ht};
        if (has_proj) {
          rgemm(EPI_BIAS, false, proj_w_p, in, nullptr, 0.f, none, proj_b, t16(bcp_in + 2 * hc16), Hc, Ht, rows, s);
          in = t16(bcp_in + 2 * hc16);
        }
        rows_stack_step(cp, p.c_k, p.c_v, p.c_kv_row, in, bx_c, rows, POS_CONST, g + 1, SKIP_DONE, s);
      }
      const float *xg = g == 0 ? x_pre : bx_c;
      if (fused && g < nac - 1) {
        rgemm(EPI_STORE, true, lm_heads_p + (size_t)g * Vc * Hc, t16(xg), c_norm, cd.eps, none, nullptr,
              Act{p.logits_c, Vc}, Vc, Hc, rows, s, p.cp_keys + (size_t)g * kHandoffKeys, keys_row);
        continue;
      }
      rgemm(EPI_STORE, true, lm_heads_p + (size_t)g * Vc * Hc, t16(xg), c_norm, cd.eps, none, nullptr,
            Act{p.logits_c, Vc}, Vc, Hc, rows, s);
      SelectCpArgs a{p.logits_c, cp_emb + (size_t)g * Vc * Ht, p.cur, p.emb_sum, p.codes,
                     trace ? p.trace_c : nullptr, p.t_in, codec_emb, p.trailing, p.st, p.prm, Vc, Ht, groups, g};
      a.codes_row = p.codes_row;
      a.trace_row = p.trace_c_row;
      a.trailing_row = p.trailing_row;
      a.row_on = p.row_on;
      hip_check(launch_select_cp(a, s, rows), "launch_select_cp(rows)");
    }
    rows_stack_step(talker, p.t_k, p.t_v, p.t_kv_row, Act{p.t_in, Ht}, bx_t, rows, POS_TALKER_FRAME, 0,
                    SKIP_TALKER, s);
    rgemm(EPI_STORE, true, codec_head_p, t16(bx_t), t_norm, td.eps, none, nullptr, Act{p.logits_t, td.vocab},
          td.vocab, Ht, rows, s);
    select_talker_rows(rows, 1, t16(bx_t), s);  // + frame bookkeeping
  }
};

struct Stream {
  Engine *engine;
  int slot;
  int host_frame = 0;  // frames already handed to the caller
  int done = 0;
  int max_frames = 0;
  // Open text input (q3t_text_stream_start): text_rows trailing rows have been pushed; until
  // q3t_text_stream_finish a frame that needs row text_rows or later does not run.
  bool text_open = false;
  int text_rows = 0;
};

namespace {

void validate_sampling(int do_sample, int top_k, float top_p, float temperature, const char *name) {
  (void)do_sample;
  if (!(top_p > 0.0f && top_p <= 1.0f)) fail(Q3T_ERR_INVALID, "%s.top_p must be in (0, 1], got %g", name, top_p);
  if (!(temperature > 0.0f)) fail(Q3T_ERR_INVALID, "%s.temperature must be positive, got %g", name, temperature);
  if (top_k < 0) fail(Q3T_ERR_INVALID, "%s.top_k must be non-negative, got %d", name, top_k);
}

void validate_options(const q3t_generate_options *o) {
  if (!o) fail(Q3T_ERR_INVALID, "options must not be null");
  if (o->max_frames <= 0) fail(Q3T_ERR_INVALID, "max_frames must be non-zero");
  if (!(o->repetition_penalty > 0.0f)) fail(Q3T_ERR_INVALID, "repetition_penalty must be positive");
  if (o->repetition_penalty_per_occurrence != 0 && o->repetition_penalty_per_occurrence != 1)
    fail(Q3T_ERR_INVALID, "repetition_penalty_per_occurrence must be 0 or 1");
  validate_sampling(o->do_sample, o->top_k, o->top_p, o->temperature, "talker");
  validate_sampling(o->subtalker_dosample, o->subtalker_top_k, o->subtalker_top_p, o->subtalker_temperature,
                    "subtalker");
}

std::string read_file(const std::string &path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) fail(Q3T_ERR_NOT_FOUND, "cannot open %s", path.c_str());
  std::stringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

void alloc_pools(Engine &e, int n) {
  int64_t &t = e.device_bytes;
  Pools &p = e.pools;
  const Dims &td = e.td, &cd = e.cd;
  const size_t esz = e.kv_bf16 ? 2 : 4;
  const int Ht = e.talker_hidden, Hc = cd.hidden;
  p.n = n;
  p.t_kv_row = (size_t)td.layers * td.kv_heads * e.cap * td.head_dim;
  p.c_kv_row = (size_t)cd.layers * cd.kv_heads * e.cp.cap * cd.head_dim;
  p.s_qkv = std::max(td.qkv_rows(), cd.qkv_rows());
  p.s_attn = std::max(td.q_out(), cd.q_out());
  p.s_act = std::max(td.intermediate, cd.intermediate);
  p.part_chunks = std::max(attn_chunks(e.cap), attn_chunks(e.cp.cap));
  p.rows_part_chunks = (e.cap + attn_rows_chunk_len(e.cap) - 1) / attn_rows_chunk_len(e.cap);
  const int kvh = std::max(td.kv_heads, cd.kv_heads);
  const int gq = std::max(td.q_heads / td.kv_heads, cd.q_heads / cd.kv_heads);
  p.part_row = (int64_t)kvh * std::max(p.part_chunks, p.rows_part_chunks) * gq * (td.head_dim + 2);
  p.trailing_row = (int64_t)(e.cap + 1) * Ht;
  p.codes_row = (int64_t)e.cap * e.groups;
  auto zeroed = [&](size_t bytes) {
    char *q = dev_alloc<char>(bytes, t);
    HIPC(hipMemset(q, 0, bytes));
    return q;
  };
  auto fz = [&](size_t per_row) { return (float *)zeroed(per_row * n * 4); };
  p.t_k = zeroed(p.t_kv_row * esz * n);
  p.t_v = zeroed(p.t_kv_row * esz * n);
  p.c_k = zeroed(p.c_kv_row * esz * n);
  p.c_v = zeroed(p.c_kv_row * esz * n);
  p.x_t = fz(Ht);
  p.t_in = fz(Ht);
  p.qkv = fz(p.s_qkv);
  p.attn = fz(p.s_attn);
  p.act = fz(p.s_act);
  p.logits_t = fz(td.vocab);
  p.logits_c = fz(cd.vocab);
  p.x_c = fz(Hc);
  p.cp_prefix = fz(2 * (size_t)Ht);
  p.cp_in = fz(3 * (size_t)Hc);
  p.cur = fz(Ht);
  p.emb_sum = fz(Ht);
  p.trailing = fz(p.trailing_row);
  p.attn_part = fz(p.part_row);
  p.s_opart = std::max((int64_t)cd.kv_heads * Hc, (int64_t)td.kv_heads * Ht);
  p.opart = fz((size_t)p.s_opart);
  p.x_mid = fz(std::max(Hc, Ht));
  p.codes = (int32_t *)zeroed((size_t)p.codes_row * n * 4);
  p.cp_keys = (uint64_t *)zeroed((size_t)n * (e.groups - 1) * kHandoffKeys * 8);
  p.tok_cur = (int32_t *)zeroed((size_t)n * 4);
  p.st = (SlotState *)zeroed(sizeof(SlotState) * n);
  p.prm = (SlotParams *)zeroed(sizeof(SlotParams) * n);
  p.row_on = (int32_t *)zeroed(sizeof(int32_t) * n);
  p.prefill_rows = n * e.cap;
  p.px = dev_alloc<float>((size_t)p.prefill_rows * Ht, t);
  p.pqkv = dev_alloc<float>((size_t)p.prefill_rows * td.qkv_rows(), t);
  p.pattn = dev_alloc<float>((size_t)p.prefill_rows * td.q_out(), t);
  p.pact = dev_alloc<float>((size_t)p.prefill_rows * td.intermediate, t);
  p.pinv = dev_alloc<float>((size_t)p.prefill_rows, t);
  HIPC(hipHostMalloc((void **)&p.h_states, sizeof(SlotState) * n, hipHostMallocDefault));
  HIPC(hipHostMalloc((void **)&p.h_codes, (size_t)p.codes_row * n * 4, hipHostMallocDefault));
  HIPC(hipHostMalloc((void **)&p.h_row_on, sizeof(int32_t) * n, hipHostMallocDefault));
  std::memset(p.h_row_on, 0, sizeof(int32_t) * n);
  HIPC(hipStreamCreateWithFlags(&p.stream, hipStreamNonBlocking));
  e.slots.resize(n);
  for (int i = 0; i < n; ++i) {
    Slot &sl = e.slots[i];
    sl.t_k = p.t_k + p.t_kv_row * esz * i;
    sl.t_v = p.t_v + p.t_kv_row * esz * i;
    sl.c_k = p.c_k + p.c_kv_row * esz * i;
    sl.c_v = p.c_v + p.c_kv_row * esz * i;
    sl.x_t = p.x_t + (size_t)i * Ht;
    sl.t_in = p.t_in + (size_t)i * Ht;
    sl.qkv = p.qkv + (size_t)i * p.s_qkv;
    sl.attn = p.attn + (size_t)i * p.s_attn;
    sl.act = p.act + (size_t)i * p.s_act;
    sl.logits_t = p.logits_t + (size_t)i * td.vocab;
    sl.logits_c = p.logits_c + (size_t)i * cd.vocab;
    sl.x_c = p.x_c + (size_t)i * Hc;
    sl.cp_prefix = p.cp_prefix + (size_t)i * 2 * Ht;
    sl.cp_in = p.cp_in + (size_t)i * 3 * Hc;
    sl.cur = p.cur + (size_t)i * Ht;
    sl.emb_sum = p.emb_sum + (size_t)i * Ht;
    sl.trailing = p.trailing + (size_t)i * p.trailing_row;
    sl.attn_part = p.attn_part + (size_t)i * p.part_row;
    sl.attn_part_chunks = p.part_chunks;
    sl.opart = p.opart + (size_t)i * p.s_opart;
    sl.x_mid = p.x_mid + (size_t)i * std::max(Hc, Ht);
    sl.codes = p.codes + (size_t)i * p.codes_row;
    sl.cp_keys = p.cp_keys + (size_t)i * (e.groups - 1) * kHandoffKeys;
    sl.tok_cur = p.tok_cur + i;
    sl.st = p.st + i;
    sl.prm = p.prm + i;
    sl.h_state = p.h_states + i;
    HIPC(hipStreamCreateWithFlags(&sl.stream, hipStreamNonBlocking));
  }
}

void free_pools(Engine &e) {
  for (Slot &sl : e.slots) {
    if (sl.graph) (void)hipGraphExecDestroy(sl.graph);
    if (sl.graph_long) (void)hipGraphExecDestroy(sl.graph_long);
    for (hipGraphExec_t g : sl.phase_graph)
      if (g) (void)hipGraphExecDestroy(g);
    if (sl.stream) (void)hipStreamDestroy(sl.stream);
  }
  e.slots.clear();
  Pools &p = e.pools;
  p.drop_graphs();
  if (p.stream) (void)hipStreamDestroy(p.stream);
  void *ptrs[] = {p.t_k,      p.t_v,     p.c_k,   p.c_v,      p.x_t,      p.t_in,    p.qkv,  p.attn,
                  p.act,      p.logits_t, p.logits_c, p.x_c,  p.cp_prefix, p.cp_in,  p.cur,  p.emb_sum,
                  p.trailing, p.attn_part, p.trace_t, p.trace_c, p.codes,  p.st,      p.prm,  p.row_on,
                  p.px,       p.pqkv,    p.pattn, p.pact,     p.pinv,    p.cp_keys, p.opart, p.x_mid, p.tok_cur};
  for (void *q : ptrs)
    if (q) (void)hipFree(q);
  if (p.h_states) (void)hipHostFree(p.h_states);
  if (p.h_codes) (void)hipHostFree(p.h_codes);
  if (p.h_row_on) (void)hipHostFree(p.h_row_on);
  p = Pools();
}

// Greedy hand-off tables: layer 0's raw q/k/v row (and, with the projection, its input row)
// for every token of the embedding tables that feed CodePredictor groups 1 .. groups-2.  The
// prompt-prefill GEMMs compute them (matrix cores, fp32 activations split into exact bf16
// terms), so a table row equals the runtime GEMV's result up to fp32 summation order.
void build_cp_tables(Engine &e) {
  if (!e.handoff_ok()) return;
  const Dims &cd = e.cd;
  const int Vc = cd.vocab, Ht = e.talker_hidden, Hc = cd.hidden, Q = cd.qkv_rows(), n = e.groups - 2;
  int64_t &t = e.device_bytes;
  e.cp_qkv_table = dev_alloc<float>((size_t)n * Vc * Q, t);
  if (e.has_proj) e.cp_in_table = dev_alloc<float>((size_t)n * Vc * Hc, t);
  int64_t scratch_bytes = 0;
  float *X = dev_alloc<float>((size_t)Vc * Ht, scratch_bytes);
  float *inv = nullptr;
  try {
    inv = dev_alloc<float>((size_t)Vc, scratch_bytes);
    for (int g = 1; g <= n; ++g) {
      hip_check(launch_bf16_to_f32(e.cp_emb + (size_t)(g - 1) * Vc * Ht, X, (size_t)Vc * Ht, nullptr),
                "launch_bf16_to_f32");
      const float *src = X;
      if (e.has_proj) {
        GemmArgs p{};
        p.X = X; p.ldx = Ht; p.W = e.proj_w; p.bias = e.proj_b;
        p.Y = e.cp_in_table + (size_t)(g - 1) * Vc * Hc; p.ldy = Hc;
        p.M = Vc; p.N = Hc; p.K = Ht;
        hip_check(launch_gemm(EPI_BIAS, p, nullptr), "launch_gemm(projection table)");
        src = p.Y;
      }
      hip_check(launch_row_rms(src, Hc, Vc, Hc, cd.eps, inv, nullptr), "launch_row_rms(table)");
      GemmArgs q{};
      q.X = src; q.ldx = Hc; q.row_scale = inv; q.gamma = e.cp.layers[0].g_in; q.W = e.cp.layers[0].qkv;
      q.Y = e.cp_qkv_table + (size_t)(g - 1) * Vc * Q; q.ldy = Q;
      q.M = Vc; q.N = Q; q.K = Hc;
      hip_check(launch_gemm(EPI_STORE, q, nullptr), "launch_gemm(q/k/v table)");
    }
    HIPC(hipDeviceSynchronize());
  } catch (...) {
    (void)hipFree(X);
    if (inv) (void)hipFree(inv);
    throw;
  }
  (void)hipFree(X);
  (void)hipFree(inv);
}

// Packed weight copies and T16 activations for the batched frame (engines with more than
// one stream slot).  Packing runs on the device from the row-major copies.
void alloc_rows(Engine &e) {
  int64_t &t = e.device_bytes;
  const Dims &td = e.td, &cd = e.cd;
  auto pack_stack = [&](StackW &w) {
    const Dims &d = w.d;
    const size_t per_layer = (size_t)d.qkv_rows() * d.hidden + (size_t)d.hidden * d.q_out() +
                             (size_t)2 * d.intermediate * d.hidden + (size_t)d.hidden * d.intermediate;
    w.mats_p = dev_alloc<uint16_t>(per_layer * d.layers, t);
    for (LayerW &L : w.layers) {
      auto at = [&](const uint16_t *m) { return w.mats_p + (m - w.mats); };
      L.qkv_p = at(L.qkv);
      L.o_p = at(L.o);
      L.gu_p = at(L.gu);
      L.down_p = at(L.down);
      hip_check(launch_pack_weights(L.qkv, const_cast<uint16_t *>(L.qkv_p), d.qkv_rows(), d.hidden, nullptr), "pack");
      hip_check(launch_pack_weights(L.o, const_cast<uint16_t *>(L.o_p), d.hidden, d.q_out(), nullptr), "pack");
      hip_check(launch_pack_weights(L.gu, const_cast<uint16_t *>(L.gu_p), 2 * d.intermediate, d.hidden, nullptr),
                "pack");
      hip_check(launch_pack_weights(L.down, const_cast<uint16_t *>(L.down_p), d.hidden, d.intermediate, nullptr),
                "pack");
    }
  };
  pack_stack(e.talker);
  pack_stack(e.cp);
  const int Ht = e.talker_hidden, Hc = cd.hidden, Vt = td.vocab, Vc = cd.vocab, nac = e.groups - 1;
  e.codec_head_p = dev_alloc<uint16_t>((size_t)Vt * Ht, t);
  hip_check(launch_pack_weights(e.codec_head, e.codec_head_p, Vt, Ht, nullptr), "pack");
  e.lm_heads_p = dev_alloc<uint16_t>((size_t)nac * Vc * Hc, t);
  for (int g = 0; g < nac; ++g)
    hip_check(launch_pack_weights(e.lm_heads + (size_t)g * Vc * Hc, e.lm_heads_p + (size_t)g * Vc * Hc, Vc, Hc,
                                  nullptr),
              "pack");
  if (e.has_proj) {
    e.proj_w_p = dev_alloc<uint16_t>((size_t)Hc * Ht, t);
    hip_check(launch_pack_weights(e.proj_w, e.proj_w_p, Hc, Ht, nullptr), "pack");
  }
  auto zeroed = [&](size_t n) {
    float *q = dev_alloc<float>(n, t);
    HIPC(hipMemset(q, 0, n * 4));
    return q;
  };
  // The CodePredictor's buffers hold two 16-row blocks (its prefix pass runs both positions).
  e.bx_t = zeroed((size_t)16 * Ht);
  e.bx_c = zeroed((size_t)32 * Hc);
  e.battn = zeroed((size_t)16 * std::max(td.q_out(), 2 * cd.q_out()));
  e.bact = zeroed((size_t)16 * std::max(td.intermediate, 2 * cd.intermediate));
  e.bcp_in = zeroed((size_t)3 * 16 * Hc);
  e.bmid_floats = (size_t)16 * std::max(Ht, 2 * Hc);
  e.bmid = zeroed(e.bmid_floats);
  e.bqkv2 = zeroed((size_t)32 * cd.qkv_rows());
}

// Logit trace buffers for every slot, allocated the first time a traced stream starts.
void ensure_trace(Engine &e) {
  Pools &p = e.pools;
  if (!e.trace || p.trace_t) return;
  p.trace_t_row = (int64_t)(e.cap + 1) * e.td.vocab;
  p.trace_c_row = (int64_t)e.cap * (e.groups - 1) * e.cd.vocab;
  p.trace_t = dev_alloc<float>((size_t)p.trace_t_row * p.n, e.device_bytes);
  p.trace_c = dev_alloc<float>((size_t)p.trace_c_row * p.n, e.device_bytes);
  for (int i = 0; i < p.n; ++i) {
    e.slots[i].trace_t = p.trace_t + (size_t)i * p.trace_t_row;
    e.slots[i].trace_c = p.trace_c + (size_t)i * p.trace_c_row;
  }
}

// hipEvents that free themselves.
struct Events {
  std::vector<hipEvent_t> ev;
  explicit Events(int n) : ev(n, nullptr) {
    for (auto &x : ev) HIPC(hipEventCreate(&x));
  }
  ~Events() {
    for (auto x : ev)
      if (x) (void)hipEventDestroy(x);
  }
  double seconds(int a, int b) const {
    float ms = 0.f;
    HIPC(hipEventElapsedTime(&ms, ev[a], ev[b]));
    return ms * 1e-3;
  }
};

void sync_state(Slot &s) {
  HIPC(hipMemcpyAsync(s.h_state, s.st, sizeof(SlotState), hipMemcpyDeviceToHost, s.stream));
  HIPC(hipStreamSynchronize(s.stream));
}

// The slot's frames in the next call whose Talker step attends with the fused attention + O
// kernel: those at positions below Engine::fused_attn_rows.  The host mirror holds the state
// after the last synchronised call, and a frame advances the position by one (frames after
// the stream's end run nothing), so frame i of the call is at position P + frame + i at most.
int fused_frames(const Engine &e, const Slot &s, int n) {
  if (!e.talker_heads_o(e.talker)) return n;  // one variant only
  const int pos = s.h_state->prefill_steps + s.h_state->frame;
  return std::clamp(e.fused_attn_rows - pos, 0, n);
}

void run_frames(Engine &e, Slot &s, int n) {
  const int nf = fused_frames(e, s, n);
  if (e.use_graph) {
    if (s.graph_traced != (bool)e.trace || s.graph_cp_greedy != s.cp_greedy) {
      for (hipGraphExec_t *gp : {&s.graph, &s.graph_long})
        if (*gp) {
          HIPC(hipGraphExecDestroy(*gp));
          *gp = nullptr;
        }
      s.graph_traced = (bool)e.trace;
      s.graph_cp_greedy = s.cp_greedy;
    }
    for (const bool lc : {false, true}) {
      const int count = lc ? n - nf : nf;
      hipGraphExec_t &graph = lc ? s.graph_long : s.graph;
      if (count == 0) continue;
      if (!graph) {
        hipGraph_t g;
        HIPC(hipStreamBeginCapture(s.stream, hipStreamCaptureModeThreadLocal));
        try {
          e.enqueue_frame(s, s.stream, lc);
        } catch (...) {
          (void)hipStreamEndCapture(s.stream, &g);
          if (g) (void)hipGraphDestroy(g);
          throw;
        }
        HIPC(hipStreamEndCapture(s.stream, &g));
        const hipError_t err = hipGraphInstantiate(&graph, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (err != hipSuccess) graph = nullptr;
        hip_check(err, "hipGraphInstantiate");
      }
      for (int i = 0; i < count; ++i) HIPC(hipGraphLaunch(graph, s.stream));
    }
  } else {
    for (int i = 0; i < n; ++i) e.enqueue_frame(s, s.stream, i >= nf);
  }
}

// n batched frames over stream rows 0..rows-1 (pools.row_on already on the device).
void run_rows_frames_impl(Engine &e, int rows, int n, bool fused) {
  Pools &p = e.pools;
  if (rows < 1 || rows > kMaxRows) fail(Q3T_ERR_INVALID, "batched frame of %d rows", rows);
  if (e.use_graph) {
    if (p.graphs_traced != (bool)e.trace) {
      p.drop_graphs();
      p.graphs_traced = (bool)e.trace;
    }
    hipGraphExec_t &graph = p.graphs[rows][fused ? 1 : 0];
    if (!graph) {
      hipGraph_t g;
      HIPC(hipStreamBeginCapture(p.stream, hipStreamCaptureModeThreadLocal));
      try {
        e.enqueue_rows_frame(rows, fused, p.stream);
      } catch (...) {
        (void)hipStreamEndCapture(p.stream, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
      }
      HIPC(hipStreamEndCapture(p.stream, &g));
      const hipError_t err = hipGraphInstantiate(&graph, g, nullptr, nullptr, 0);
      (void)hipGraphDestroy(g);
      if (err != hipSuccess) graph = nullptr;
      hip_check(err, "hipGraphInstantiate");
    }
    for (int i = 0; i < n; ++i) HIPC(hipGraphLaunch(graph, p.stream));
  } else {
    for (int i = 0; i < n; ++i) e.enqueue_rows_frame(rows, fused, p.stream);
  }
}

// The split O / down GEMMs keep bmid all zeros between layers (each zeroes what it read).
// An error can stop a frame between the two, so after any error the next call first
// restores the zeros (outside any captured graph), and later frames never add onto stale sums.
void run_rows_frames(Engine &e, int rows, int n, bool fused) {
  Pools &p = e.pools;
  if (e.bmid_dirty && e.bmid) {
    HIPC(hipMemsetAsync(e.bmid, 0, e.bmid_floats * sizeof(float), p.stream));
    e.bmid_dirty = false;
  }
  try {
    run_rows_frames_impl(e, rows, n, fused);
  } catch (...) {
    e.bmid_dirty = true;
    throw;
  }
}

// Marks the rows of `slots_on` (others off) and returns the row count a launch must cover.
int set_rows(Engine &e, const std::vector<int> &slots_on, hipStream_t s) {
  Pools &p = e.pools;
  int rows = 0;
  std::memset(p.h_row_on, 0, sizeof(int32_t) * p.n);
  for (int i : slots_on) {
    p.h_row_on[i] = 1;
    rows = std::max(rows, i + 1);
  }
  HIPC(hipMemcpyAsync(p.row_on, p.h_row_on, sizeof(int32_t) * p.n, hipMemcpyHostToDevice, s));
  return rows;
}

}  // namespace
}  // namespace q3t

using q3t::Engine;
using q3t::fail;
using q3t::guarded;

struct q3t_engine : Engine {};
struct q3t_stream : q3t::Stream {};

extern "C" {

void q3t_generate_options_default(q3t_generate_options *o) {
  if (!o) return;
  o->speaker = 3;   // Speaker::Ryan
  o->language = 1;  // Language::English
  o->max_frames = 240;
  o->decode_audio = 1;
  o->do_sample = 1;
  o->top_k = 50;
  o->top_p = 1.0f;
  o->temperature = 0.9f;
  o->repetition_penalty = 1.05f;
  o->subtalker_dosample = 1;
  o->subtalker_top_k = 50;
  o->subtalker_top_p = 1.0f;
  o->subtalker_temperature = 0.9f;
  o->seed = 0;
  o->repetition_penalty_per_occurrence = 0;
}

const char *q3t_last_error(void) { return q3t::g_last_error.c_str(); }

int q3t_generate_options_validate(const q3t_generate_options *o) {
  return guarded([&] { q3t::validate_options(o); });
}

int q3t_engine_create(const q3t_engine_options *opts, q3t_engine **out) {
  return guarded([&] {
    using namespace q3t;
    if (!opts || !out || !opts->model_dir) fail(Q3T_ERR_INVALID, "engine options and output must not be null");
    *out = nullptr;
    auto e = std::make_unique<q3t_engine>();
    e->device = opts->device;
    e->cap = opts->max_cache_steps > 0 ? opts->max_cache_steps : 512;
    e->use_graph = opts->use_graph;
    if (opts->kv_dtype != 0 && opts->kv_dtype != 1) fail(Q3T_ERR_INVALID, "kv_dtype must be 0 (fp32) or 1 (bf16)");
    e->kv_bf16 = opts->kv_dtype;
    e->fused_attn_rows = e->kv_bf16 ? Engine::kFusedAttnRowsBf16 : Engine::kFusedAttnRowsF32;
    const int nslots = opts->max_streams > 0 ? opts->max_streams : 1;
    if (nslots > kMaxRows) fail(Q3T_ERR_INVALID, "max_streams %d exceeds %d", nslots, kMaxRows);
    const std::string dir = opts->model_dir;
    const json::Value cfg = json::parse(read_file(dir + "/config.json"));
    const json::Value &tc = cfg.at("talker_config");
    const json::Value &cc = tc.at("code_predictor_config");
    e->td = dims_from(tc);
    e->cd = dims_from(cc);
    e->groups = (int)tc.at("num_code_groups").integer();
    e->codec_eos = (int)tc.at("codec_eos_token_id").integer();
    e->talker_hidden = e->td.hidden;
    e->has_proj = e->td.hidden != e->cd.hidden;
    const Dims &td = e->td, &cd = e->cd;
    // Shape limits of the kernels (checked here so that no launch can index outside).
    for (const Dims *d : {&td, &cd}) {
      if (d->head_dim != 128) fail(Q3T_ERR_INVALID, "head_dim %d unsupported (kernels are built for 128)", d->head_dim);
      if (d->kv_heads <= 0 || d->q_heads % d->kv_heads || d->q_heads / d->kv_heads > 2)
        fail(Q3T_ERR_INVALID, "q_heads %d / kv_heads %d unsupported", d->q_heads, d->kv_heads);
      if (!gemv_supports_k(d->hidden) || !gemv_supports_k(d->intermediate) || !gemv_supports_k(d->q_out()))
        fail(Q3T_ERR_INVALID, "hidden %d / intermediate %d / q_out %d must be 512 x {1,2,3,4,6,8,12}", d->hidden,
             d->intermediate, d->q_out());
    }
    if (td.vocab > kMaxVocab || td.vocab < 1024 || cd.vocab > kMaxVocab)
      fail(Q3T_ERR_INVALID, "vocab sizes %d / %d unsupported", td.vocab, cd.vocab);
    if (e->groups < 2) fail(Q3T_ERR_INVALID, "CodePredictor needs at least one semantic and one acoustic group");
    if (e->cap > attn_max_cache_steps(td.q_heads, td.kv_heads))
      fail(Q3T_ERR_INVALID, "max_cache_steps %d exceeds the attention kernel limit %d", e->cap,
           attn_max_cache_steps(td.q_heads, td.kv_heads));
    if (e->codec_eos < 0 || e->codec_eos >= td.vocab) fail(Q3T_ERR_INVALID, "codec_eos out of range");
    e->rows_ok = gemm_skinny_supports(kMaxRows, td.hidden, true) && gemm_skinny_supports(kMaxRows, cd.hidden, true);

    SafeTensors st(dir + "/model.safetensors");
    HIPC(hipSetDevice(e->device));
    // the no-allocation scratch of this device (kept by the library until the process ends)
    e->scratch_status = noalloc_scratch_setup(e->device);
    int64_t &tally = e->device_bytes;
    load_stack(st, "talker.model", td, e->cap, e->talker, tally);
    load_stack(st, "talker.code_predictor.model", cd, e->groups, e->cp, tally);
    const int64_t Ht = td.hidden, Vt = td.vocab, Hc = cd.hidden, Vc = cd.vocab, nac = e->groups - 1;
    auto upload_bf16 = [&](const std::vector<std::string> &names, const std::vector<int64_t> &shape) {
      std::vector<uint16_t> host;
      for (auto &n : names) st.append_bf16(n, shape, host);
      uint16_t *d = dev_alloc<uint16_t>(host.size(), tally);
      HIPC(hipMemcpy(d, host.data(), host.size() * 2, hipMemcpyHostToDevice));
      return d;
    };
    auto upload_f32 = [&](const std::string &n, int64_t len) {
      auto v = st.f32(n, {len});
      float *d = dev_alloc<float>(v.size(), tally);
      HIPC(hipMemcpy(d, v.data(), v.size() * 4, hipMemcpyHostToDevice));
      return d;
    };
    e->codec_head = upload_bf16({"talker.codec_head.weight"}, {Vt, Ht});
    e->codec_emb = upload_bf16({"talker.model.codec_embedding.weight"}, {Vt, Ht});
    e->t_norm = upload_f32("talker.model.norm.weight", Ht);
    e->c_norm = upload_f32("talker.code_predictor.model.norm.weight", Hc);
    std::vector<std::string> heads, embs;
    for (int g = 0; g < nac; ++g) {
      heads.push_back("talker.code_predictor.lm_head." + std::to_string(g) + ".weight");
      embs.push_back("talker.code_predictor.model.codec_embedding." + std::to_string(g) + ".weight");
    }
    e->lm_heads = upload_bf16(heads, {Vc, Hc});
    e->cp_emb = upload_bf16(embs, {Vc, Ht});
    // Special ids and the speaker / language maps (config.rs:47-80).
    e->tok_im_start = (int)cfg.at("im_start_token_id").integer();
    e->tok_assistant = (int)cfg.at("assistant_token_id").integer();
    e->tok_tts_pad = (int)cfg.at("tts_pad_token_id").integer();
    e->tok_tts_bos = (int)cfg.at("tts_bos_token_id").integer();
    e->tok_tts_eos = (int)cfg.at("tts_eos_token_id").integer();
    e->codec_pad = (int)tc.at("codec_pad_id").integer();
    e->codec_bos = (int)tc.at("codec_bos_id").integer();
    e->codec_think = (int)tc.at("codec_think_id").integer();
    e->codec_think_bos = (int)tc.at("codec_think_bos_id").integer();
    e->codec_think_eos = (int)tc.at("codec_think_eos_id").integer();
    for (const auto &kv : tc.at("spk_id").obj) e->speaker_ids[kv.first] = (int)kv.second.integer();
    for (const auto &kv : tc.at("codec_language_id").obj) e->language_ids[kv.first] = (int)kv.second.integer();
    if (st.has("talker.model.text_embedding.weight")) {
      // TtsTextPrep::load (text.rs:267-329): table [vocab, text_hidden], fc1 [inter, text_hidden],
      // fc2 [H, inter].
      const std::vector<int64_t> ts = st.shape("talker.model.text_embedding.weight");
      const std::vector<int64_t> f1 = st.shape("talker.text_projection.linear_fc1.weight");
      const std::vector<int64_t> f2 = st.shape("talker.text_projection.linear_fc2.weight");
      if (ts.size() != 2 || f1.size() != 2 || f2.size() != 2 || f1[1] != ts[1] || f2[1] != f1[0] || f2[0] != Ht)
        fail(Q3T_ERR_INVALID, "invalid text embedding / text projection shapes");
      if (ts[1] % 32 || f1[0] % 32) fail(Q3T_ERR_INVALID, "text widths must be multiples of 32");
      e->text_vocab = (int)ts[0];
      e->text_hidden = (int)ts[1];
      e->tp_inter = (int)f1[0];
      e->text_emb = upload_bf16({"talker.model.text_embedding.weight"}, ts);
      e->tp_fc1 = upload_bf16({"talker.text_projection.linear_fc1.weight"}, f1);
      e->tp_b1 = upload_f32("talker.text_projection.linear_fc1.bias", f1[0]);
      e->tp_fc2 = upload_bf16({"talker.text_projection.linear_fc2.weight"}, f2);
      e->tp_b2 = upload_f32("talker.text_projection.linear_fc2.bias", Ht);
    }
    if (e->has_proj) {
      if (!gemv_supports_k((int)Ht)) fail(Q3T_ERR_INVALID, "projection width %d unsupported", (int)Ht);
      e->proj_w = upload_bf16({"talker.code_predictor.small_to_mtp_projection.weight"}, {Hc, Ht});
      e->proj_b = upload_f32("talker.code_predictor.small_to_mtp_projection.bias", Hc);
    }
    try {
      alloc_pools(*e, nslots);
      if (nslots > 1 && e->rows_ok) alloc_rows(*e);
      e->split_ws = dev_alloc<float>((size_t)Engine::kSplitFloats, e->device_bytes);
      build_cp_tables(*e);
      e->codec = codec_load(dir, &e->device_bytes);
    } catch (...) {
      free_pools(*e);
      throw;
    }
    HIPC(hipDeviceSynchronize());
    *out = e.release();
  });
}

int q3t_engine_destroy(q3t_engine *e) {
  return guarded([&] {
    if (!e) return;
    (void)hipSetDevice(e->device);
    (void)hipDeviceSynchronize();
    q3t::free_pools(*e);
    q3t::codec_free(e->codec);
    void *ptrs[] = {e->talker.mats, e->talker.gains, e->talker.rope, e->cp.mats,     e->cp.gains,
                    e->cp.rope,     e->codec_head,   e->codec_emb,   e->t_norm,      e->c_norm,
                    e->lm_heads,    e->cp_emb,       e->proj_w,      e->proj_b,      e->talker.mats_p,
                    e->cp.mats_p,   e->codec_head_p, e->lm_heads_p,  e->proj_w_p,    e->bx_t,
                    e->bx_c,        e->battn,        e->bact,        e->bcp_in,      e->cp_qkv_table,
                    e->cp_in_table, e->text_emb,     e->tp_fc1,      e->tp_fc2,      e->tp_b1,
                    e->tp_b2,       e->split_ws,    e->bmid,        e->bqkv2};
    for (void *p : ptrs)
      if (p) (void)hipFree(p);
    delete e;
  });
}

int q3t_engine_get_info(const q3t_engine *e, q3t_engine_info *o) {
  return guarded([&] {
    if (!e || !o) fail(Q3T_ERR_INVALID, "null argument");
    o->talker_hidden = e->td.hidden;
    o->talker_intermediate = e->td.intermediate;
    o->talker_layers = e->td.layers;
    o->talker_vocab = e->td.vocab;
    o->cp_hidden = e->cd.hidden;
    o->cp_intermediate = e->cd.intermediate;
    o->cp_layers = e->cd.layers;
    o->cp_vocab = e->cd.vocab;
    o->q_heads = e->td.q_heads;
    o->kv_heads = e->td.kv_heads;
    o->head_dim = e->td.head_dim;
    o->num_code_groups = e->groups;
    o->codec_eos = e->codec_eos;
    o->max_cache_steps = e->cap;
    o->max_streams = (int32_t)e->slots.size();
    o->device_bytes = e->device_bytes;
    o->text_vocab = e->text_vocab;
    o->text_hidden = e->text_hidden;
    o->samples_per_frame = e->codec ? q3t::kCodecSamplesPerFrame : 0;
  });
}

int q3t_engine_set_trace(q3t_engine *e, int32_t enabled) {
  return guarded([&] {
    if (!e) fail(Q3T_ERR_INVALID, "null engine");
    e->trace = enabled ? 1 : 0;
  });
}

int q3t_engine_set_fused_attention_rows(q3t_engine *e, int32_t rows) {
  return guarded([&] {
    if (!e) fail(Q3T_ERR_INVALID, "null engine");
    if (rows < 0) fail(Q3T_ERR_INVALID, "fused attention rows must not be negative");
    e->fused_attn_rows = rows;
  });
}

}  // extern "C"

namespace q3t {
namespace {

void validate_input(const Engine &e, const q3t_stream_input &in, const q3t_generate_options *o) {
  validate_options(o);
  if (in.prefill_steps <= 0) fail(Q3T_ERR_INVALID, "prefill steps must be non-zero");
  if (!in.prefill || !in.tts_pad || (in.trailing_steps > 0 && !in.trailing) || in.trailing_steps < 0)
    fail(Q3T_ERR_INVALID, "null input array");
  if ((int64_t)in.prefill_steps + o->max_frames > e.cap)
    fail(Q3T_ERR_CAPACITY,
         "requested %lld cache steps but engine was loaded for %d; call load_with_max_frames with a larger "
         "max_frames",
         (long long)in.prefill_steps + o->max_frames, e.cap);
}

// Uploads one stream's inputs (prompt rows into the prefill workspace at row0, trailing
// rows then tts_pad, loop state, options) onto stream s.
void stage_state(Engine &e, int slot, int prefill_steps, int trailing_rows, const q3t_generate_options *o,
                 hipStream_t s);

void stage_stream(Engine &e, int slot, int row0, const q3t_stream_input &in, const q3t_generate_options *o,
                  hipStream_t s) {
  Slot &sl = e.slots[slot];
  const int Ht = e.talker_hidden;
  const int rows = std::min<int>(in.trailing_steps, e.cap);
  HIPC(hipMemcpyAsync(e.pools.px + (size_t)row0 * Ht, in.prefill, (size_t)in.prefill_steps * Ht * 4,
                      hipMemcpyHostToDevice, s));
  if (rows > 0)
    HIPC(hipMemcpyAsync(sl.trailing, in.trailing, (size_t)rows * Ht * 4, hipMemcpyHostToDevice, s));
  HIPC(hipMemcpyAsync(sl.trailing + (size_t)rows * Ht, in.tts_pad, (size_t)Ht * 4, hipMemcpyHostToDevice, s));
  stage_state(e, slot, in.prefill_steps, rows, o, s);
}

// Loop state and options of a starting stream (its prompt rows are already staged on s).
void stage_state(Engine &e, int slot, int prefill_steps, int trailing_rows, const q3t_generate_options *o,
                 hipStream_t s) {
  Slot &sl = e.slots[slot];
  SlotState st0{};
  st0.frame = 0;
  st0.semantic = -1;
  st0.done = 0;
  st0.prefill_steps = prefill_steps;
  st0.max_frames = o->max_frames;
  st0.trailing_rows = trailing_rows;
  SlotParams pr{};
  pr.talker = SamplingParams{o->do_sample ? 1 : 0, o->top_k, o->top_p, o->temperature};
  pr.cp = SamplingParams{o->subtalker_dosample ? 1 : 0, o->subtalker_top_k, o->subtalker_top_p,
                         o->subtalker_temperature};
  pr.repetition_penalty = o->repetition_penalty;
  pr.use_history = (o->repetition_penalty != 1.0f || o->do_sample) ? 1 : 0;
  pr.penalty_per_occurrence = o->repetition_penalty_per_occurrence;
  pr.seed_lo = (uint32_t)(o->seed & 0xffffffffu);
  pr.seed_hi = (uint32_t)(o->seed >> 32);
  pr.trace = e.trace;
  pr.codec_eos = e.codec_eos;
  sl.cp_greedy = !o->subtalker_dosample;
  // Pageable sources: hipMemcpy returns once the host copy is taken.
  HIPC(hipStreamSynchronize(s));
  HIPC(hipMemcpy(sl.st, &st0, sizeof(SlotState), hipMemcpyHostToDevice));
  HIPC(hipMemcpy(sl.prm, &pr, sizeof(SlotParams), hipMemcpyHostToDevice));
}

// Speaker::config_key / Language::config_key order of the q3t_generate_options enums
// (text.rs:39-52, 103-116).
const char *const kSpeakerKeys[] = {"serena", "vivian", "uncle_fu", "ryan", "aiden",
                                    "ono_anna", "sohee", "eric", "dylan"};
const char *const kLanguageKeys[] = {"chinese", "english", "japanese", "korean", "german",
                                     "french", "russian", "portuguese", "spanish", "italian"};
constexpr int kNewline = 198;  // text.rs:15

int resolve_token(const std::map<std::string, int> &ids, const char *const *keys, int nkeys, int index,
                  const char *kind) {
  if (index < 0 || index >= nkeys) fail(Q3T_ERR_INVALID, "unknown %s %d", kind, index);
  auto it = ids.find(keys[index]);
  if (it == ids.end()) fail(Q3T_ERR_INVALID, "missing %s token id for %s", kind, keys[index]);  // text.rs:642-653
  return it->second;
}

// A prompt's rows as TtsTextPrep::prepare_custom_voice_with_lookahead lays them out
// (text.rs:340-382, 516-573): the text ids to project, the codec embedding row added to
// each (-1: none, kTextSpeakerRow: the voice-clone speaker embedding) and each row's
// destination ((kind << 24) | row: 0 prefill, 1 trailing, 2 tts_pad, 3 dropped).  With a
// speaker embedding (xvec, H floats) the speaker's codec row is that embedding instead
// (prepare_voice_clone_xvector_with_lookahead, text.rs:432-490, 507-514).
struct TextPlan {
  std::vector<int32_t> ids, codec, dst;
  std::vector<float> xvec;
  int prefill_steps = 0, trailing_steps = 0;
};

//
// open_text: the prefill of a text stream (custom_voice_prefill_from_content_tokens,
// text.rs:396-430): every id in the prefill and no trailing text, which the stream's pushes
// supply.
TextPlan plan_text(const Engine &e, const int32_t *content, int n, int speaker, int language, int lookahead,
                   int trailing_cap, const float *xvec = nullptr, int xvec_len = 0, bool open_text = false) {
  if (!e.text_emb)
    fail(Q3T_ERR_NOT_FOUND, "the model has no talker.model.text_embedding.weight: device text preparation "
                            "needs it");
  if (n < 0 || (n > 0 && !content)) fail(Q3T_ERR_INVALID, "null or negative content ids");
  if (lookahead <= 0) fail(Q3T_ERR_INVALID, "text_lookahead_tokens must be non-zero");
  if (open_text && n == 0) fail(Q3T_ERR_INVALID, "a text stream starts with at least one content token");
  for (int i = 0; i < n; ++i)
    if (content[i] < 0 || content[i] >= e.text_vocab)
      fail(Q3T_ERR_INVALID, "text token %d is out of range for vocab %d", content[i], e.text_vocab);
  if (xvec && xvec_len != e.talker_hidden)  // text.rs:445-451
    fail(Q3T_ERR_INVALID, "speaker embedding length %d does not match model hidden %d", xvec_len, e.talker_hidden);
  const int spk = xvec ? e.codec_pad : resolve_token(e.speaker_ids, kSpeakerKeys, 9, speaker, "speaker");
  const int lang = resolve_token(e.language_ids, kLanguageKeys, 10, language, "language");
  for (int c : {spk, lang, e.codec_pad, e.codec_bos, e.codec_think, e.codec_think_bos, e.codec_think_eos})
    if (c < 0 || c >= e.td.vocab) fail(Q3T_ERR_INVALID, "codec token %d is out of range for vocab %d", c, e.td.vocab);
  for (int t : {e.tok_im_start, e.tok_assistant, kNewline, e.tok_tts_pad, e.tok_tts_bos, e.tok_tts_eos})
    if (t < 0 || t >= e.text_vocab) fail(Q3T_ERR_INVALID, "text token %d is out of range for vocab %d", t, e.text_vocab);
  const int L = n == 0 ? 0 : std::max(1, std::min(lookahead, n));
  TextPlan p;
  auto row = [&](int id, int codec, int kind, int r) {
    p.ids.push_back(id);
    p.codec.push_back(codec);
    p.dst.push_back((kind << 24) | r);
  };
  // role prefix, then tts_pad x5 / tts_bos over [think, think_bos, language, think_eos,
  // speaker, pad], then the first L content ids over pad (bos on the last)
  const int role[3] = {e.tok_im_start, e.tok_assistant, kNewline};
  for (int i = 0; i < 3; ++i) row(role[i], -1, 0, i);
  const int codec6[6] = {e.codec_think, e.codec_think_bos, lang, e.codec_think_eos, xvec ? kTextSpeakerRow : spk,
                         e.codec_pad};
  if (xvec) p.xvec.assign(xvec, xvec + xvec_len);
  for (int i = 0; i < 6; ++i) row(i < 5 ? e.tok_tts_pad : e.tok_tts_bos, codec6[i], 0, 3 + i);
  for (int i = 0; i < L; ++i) row(content[i], i + 1 == L ? e.codec_bos : e.codec_pad, 0, 9 + i);
  p.prefill_steps = 9 + L;
  // trailing text: the rest of the content, then tts_eos; then the tts_pad row
  p.trailing_steps = open_text ? 0 : n - L + 1;
  for (int i = 0; i < p.trailing_steps; ++i) {
    const int id = i + L < n ? content[i + L] : e.tok_tts_eos;
    row(id, -1, i < trailing_cap ? 1 : 3, i < trailing_cap ? i : 0);
  }
  row(e.tok_tts_pad, -1, 2, 0);
  return p;
}

// Trailing text rows of an open text stream: id i projected into trailing row first_row + i
// (projected_text_embedding_for_token of each popped token, generation.rs:1367-1369).
TextPlan plan_trailing_rows(const Engine &e, const int32_t *ids, int n, int first_row) {
  TextPlan p;
  for (int i = 0; i < n; ++i) {
    if (ids[i] < 0 || ids[i] >= e.text_vocab)
      fail(Q3T_ERR_INVALID, "text token %d is out of range for vocab %d", ids[i], e.text_vocab);
    p.ids.push_back(ids[i]);
    p.codec.push_back(-1);
    p.dst.push_back((1 << 24) | (first_row + i));
  }
  p.trailing_steps = n;
  return p;
}

// Device workspace of one TextPlan run: ids / codec ids / destinations (3M int32), the
// gathered text-embedding rows X [M, text_hidden], the fc1 activations [M, tp_inter], the fc2
// output Y [M, H] and, for voice clone, the x-vector [H]; each part 256-byte aligned.
struct TextWorkspace {
  int32_t *ids = nullptr;
  float *X = nullptr, *Hd = nullptr, *Y = nullptr, *xvec = nullptr;
};

inline size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

size_t text_workspace_bytes(const Engine &e, const TextPlan &p) {
  const size_t M = p.ids.size();
  return align256(M * 4 * 3) + align256(M * e.text_hidden * 4) + align256(M * e.tp_inter * 4) +
         align256(M * e.talker_hidden * 4) + align256(p.xvec.size() * 4);
}

TextWorkspace carve_text_workspace(const Engine &e, const TextPlan &p, char *base) {
  const size_t M = p.ids.size();
  TextWorkspace w;
  w.ids = (int32_t *)base;
  base += align256(M * 4 * 3);
  w.X = (float *)base;
  base += align256(M * e.text_hidden * 4);
  w.Hd = (float *)base;
  base += align256(M * e.tp_inter * 4);
  w.Y = (float *)base;
  base += align256(M * e.talker_hidden * 4);
  if (!p.xvec.empty()) w.xvec = (float *)base;
  return w;
}

// Runs a TextPlan on stream s in the workspace w: text-embedding gather -> fc1 (+ bias) -> SiLU
// -> fc2 (+ bias) -> plus codec rows, into prefill / trailing / pad (device pointers).  Every
// workspace part is written before it is read (nothing needs to start at zero).  Synchronous.
void run_text_plan(Engine &e, const TextPlan &p, const TextWorkspace &w, float *prefill, float *trailing, float *pad,
                   hipStream_t s) {
  const int M = (int)p.ids.size(), H = e.talker_hidden;
  int32_t *ids = w.ids, *codec = w.ids + M, *dst = w.ids + 2 * M;
  if (!p.xvec.empty())
    HIPC(hipMemcpyAsync(w.xvec, p.xvec.data(), p.xvec.size() * 4, hipMemcpyHostToDevice, s));
  std::vector<int32_t> host(p.ids);
  host.insert(host.end(), p.codec.begin(), p.codec.end());
  host.insert(host.end(), p.dst.begin(), p.dst.end());
  HIPC(hipMemcpyAsync(ids, host.data(), host.size() * 4, hipMemcpyHostToDevice, s));
  hip_check(launch_text_gather(e.text_emb, e.text_hidden, ids, M, w.X, s), "launch_text_gather");
  GemmArgs g{};
  g.X = w.X; g.ldx = e.text_hidden; g.W = e.tp_fc1; g.bias = e.tp_b1; g.Y = w.Hd; g.ldy = e.tp_inter;
  g.M = M; g.N = e.tp_inter; g.K = e.text_hidden;
  g.split_ws = e.split_ws; g.split_cap = Engine::kSplitFloats;
  hip_check(launch_gemm(EPI_BIAS, g, s), "launch_gemm(text fc1)");
  hip_check(launch_silu(w.Hd, (size_t)M * e.tp_inter, s), "launch_silu");
  g = GemmArgs{};
  g.X = w.Hd; g.ldx = e.tp_inter; g.W = e.tp_fc2; g.bias = e.tp_b2; g.Y = w.Y; g.ldy = H;
  g.M = M; g.N = H; g.K = e.tp_inter;
  g.split_ws = e.split_ws; g.split_cap = Engine::kSplitFloats;
  hip_check(launch_gemm(EPI_BIAS, g, s), "launch_gemm(text fc2)");
  hip_check(launch_text_assemble(w.Y, H, M, codec, e.codec_emb, w.xvec, dst, prefill, trailing, pad, s),
            "launch_text_assemble");
  HIPC(hipStreamSynchronize(s));
}

// run_text_plan in a workspace allocated for the call.
void prepare_text_device(Engine &e, const TextPlan &p, float *prefill, float *trailing, float *pad, hipStream_t s) {
  int64_t bytes = 0;
  char *base = dev_alloc<char>(text_workspace_bytes(e, p), bytes);
  try {
    run_text_plan(e, p, carve_text_workspace(e, p, base), prefill, trailing, pad, s);
  } catch (...) {
    (void)hipFree(base);
    throw;
  }
  (void)hipFree(base);
}

q3t_stream *new_stream(Engine &e, int slot, int max_frames) {
  Slot &sl = e.slots[slot];
  sl.in_use = true;
  auto *stream = new q3t_stream();
  stream->engine = &e;
  stream->slot = slot;
  stream->max_frames = max_frames;
  stream->done = sl.h_state->done;
  return stream;
}

// A stream whose prompt rows (prefill workspace rows 0..P-1) and state are staged: the
// Talker prefill at positions 0..P-1, the head and the first semantic token with its EOS /
// max_frames check (talker.rs:207-233).
q3t_stream *start_staged(Engine &e, int slot, int P, const q3t_generate_options *o) {
  Slot &s = e.slots[slot];
  e.prefill_segments({PrefillSeg{slot, 0, P}}, P, s.stream);
  e.gemv(EPI_STORE, true, e.codec_head, s.x_t, e.t_norm, e.td.eps, nullptr, nullptr, s.logits_t, e.td.vocab,
         e.td.hidden, SKIP_NEVER, s.st, s.stream);
  e.select_talker(s, 0, s.stream);
  sync_state(s);
  return new_stream(e, slot, o->max_frames);
}

}  // namespace
}  // namespace q3t

extern "C" {

int q3t_stream_start(q3t_engine *e, const float *prefill, int32_t P, const float *trailing, int32_t T,
                     const float *tts_pad, const q3t_generate_options *o, q3t_stream **out) {
  return guarded([&] {
    using namespace q3t;
    if (!e || !out) fail(Q3T_ERR_INVALID, "null engine or output");
    *out = nullptr;
    const q3t_stream_input in{prefill, P, trailing, T, tts_pad};
    validate_input(*e, in, o);
    int slot = -1;
    for (size_t i = 0; i < e->slots.size(); ++i)
      if (!e->slots[i].in_use) {
        slot = (int)i;
        break;
      }
    if (slot < 0) fail(Q3T_ERR_BUSY, "all %zu stream slots are in use", e->slots.size());
    HIPC(hipSetDevice(e->device));
    ensure_trace(*e);
    stage_stream(*e, slot, 0, in, o, e->slots[slot].stream);
    *out = start_staged(*e, slot, P, o);
  });
}

int q3t_stream_start_profiled(q3t_engine *e, const float *prefill, int32_t P, const float *trailing, int32_t T,
                              const float *tts_pad, const q3t_generate_options *o, q3t_stream **out,
                              q3t_profile *prof) {
  return guarded([&] {
    using namespace q3t;
    if (!e || !out || !prof) fail(Q3T_ERR_INVALID, "null argument");
    *out = nullptr;
    const q3t_stream_input in{prefill, P, trailing, T, tts_pad};
    validate_input(*e, in, o);
    int slot = -1;
    for (size_t i = 0; i < e->slots.size(); ++i)
      if (!e->slots[i].in_use) {
        slot = (int)i;
        break;
      }
    if (slot < 0) fail(Q3T_ERR_BUSY, "all %zu stream slots are in use", e->slots.size());
    HIPC(hipSetDevice(e->device));
    ensure_trace(*e);
    hipStream_t s = e->slots[slot].stream;
    Events ev(3);
    HIPC(hipEventRecord(ev.ev[0], s));
    stage_stream(*e, slot, 0, in, o, s);
    HIPC(hipEventRecord(ev.ev[1], s));
    *out = start_staged(*e, slot, P, o);
    HIPC(hipEventRecord(ev.ev[2], s));
    HIPC(hipEventSynchronize(ev.ev[2]));
    prof->upload_seconds += ev.seconds(0, 1);
    prof->prefill_seconds += ev.seconds(1, 2);
  });
}

}  // extern "C"

namespace q3t {
namespace {

// q3t_prepare_text / q3t_prepare_text_voice_clone: runs the plan into a device staging
// buffer and copies its rows to the caller's host arrays.
void prepare_text_to_host(Engine *e, const TextPlan &p, float *prefill, int32_t *prefill_steps, float *trailing,
                          int32_t *trailing_steps, float *tts_pad) {
  HIPC(hipSetDevice(e->device));
  const size_t H = (size_t)e->talker_hidden;
  int64_t bytes = 0;
  float *d = dev_alloc<float>((size_t)(p.prefill_steps + p.trailing_steps + 1) * H, bytes);
  try {
    float *dt = d + (size_t)p.prefill_steps * H, *dp = dt + (size_t)p.trailing_steps * H;
    prepare_text_device(*e, p, d, dt, dp, e->pools.stream);
    HIPC(hipMemcpy(prefill, d, (size_t)p.prefill_steps * H * 4, hipMemcpyDeviceToHost));
    HIPC(hipMemcpy(trailing, dt, (size_t)p.trailing_steps * H * 4, hipMemcpyDeviceToHost));
    HIPC(hipMemcpy(tts_pad, dp, H * 4, hipMemcpyDeviceToHost));
  } catch (...) {
    (void)hipFree(d);
    throw;
  }
  (void)hipFree(d);
  *prefill_steps = p.prefill_steps;
  *trailing_steps = p.trailing_steps;
}

// q3t_stream_start_text / q3t_stream_start_voice_clone / q3t_text_stream_start: the plan's rows
// built straight into a free slot, then the prefill and the first semantic token.  An open
// text stream keeps the tts_pad row in the last trailing row (cap) and lets frame f read row f
// until q3t_text_stream_finish.
q3t_stream *start_text_stream(Engine *e, const TextPlan &p, const q3t_generate_options *o, bool open_text = false) {
  if ((int64_t)p.prefill_steps + o->max_frames > e->cap)
    fail(Q3T_ERR_CAPACITY,
         "requested %lld cache steps but engine was loaded for %d; call load_with_max_frames with a larger "
         "max_frames",
         (long long)p.prefill_steps + o->max_frames, e->cap);
  int slot = -1;
  for (size_t i = 0; i < e->slots.size(); ++i)
    if (!e->slots[i].in_use) {
      slot = (int)i;
      break;
    }
  if (slot < 0) fail(Q3T_ERR_BUSY, "all %zu stream slots are in use", e->slots.size());
  HIPC(hipSetDevice(e->device));
  ensure_trace(*e);
  Slot &s = e->slots[slot];
  const int rows = open_text ? e->cap : std::min(p.trailing_steps, e->cap);
  prepare_text_device(*e, p, e->pools.px, s.trailing, s.trailing + (size_t)rows * e->talker_hidden, s.stream);
  stage_state(*e, slot, p.prefill_steps, rows, o, s.stream);
  q3t_stream *out = start_staged(*e, slot, p.prefill_steps, o);
  out->text_open = open_text;
  return out;
}

// The frames a single-stream run just produced: codes, state and the stream's counters.
void collect_frames(q3t_stream *sp, int n, int32_t *codes, q3t_chunk_info *info) {
  Engine &e = *sp->engine;
  Slot &s = e.slots[sp->slot];
  // The state and the n frames' codes (those not produced are never read) in one round trip.
  int32_t *h = e.pools.h_codes + (size_t)sp->slot * e.pools.codes_row + (size_t)sp->host_frame * e.groups;
  HIPC(hipMemcpyAsync(h, s.codes + (size_t)sp->host_frame * e.groups, (size_t)n * e.groups * 4,
                      hipMemcpyDeviceToHost, s.stream));
  sync_state(s);
  const int produced = s.h_state->frame - sp->host_frame;
  if (produced < 0 || produced > n) fail(Q3T_ERR_HIP, "device loop state is inconsistent");
  if (produced > 0) std::memcpy(codes, h, (size_t)produced * e.groups * 4);
  sp->host_frame += produced;
  sp->done = s.h_state->done;
  info->frames = produced;
  info->total_frames = sp->host_frame;
  info->ended_by_eos = sp->done == 1;
}

}  // namespace
}  // namespace q3t

extern "C" {

int q3t_prepare_text(q3t_engine *e, const int32_t *content_ids, int32_t n_ids, int32_t speaker, int32_t language,
                     int32_t text_lookahead_tokens, float *prefill, int32_t *prefill_steps, float *trailing,
                     int32_t *trailing_steps, float *tts_pad) {
  return guarded([&] {
    using namespace q3t;
    if (!e || !prefill || !prefill_steps || !trailing || !trailing_steps || !tts_pad)
      fail(Q3T_ERR_INVALID, "null argument");
    const TextPlan p = plan_text(*e, content_ids, n_ids, speaker, language, text_lookahead_tokens, n_ids + 1);
    prepare_text_to_host(e, p, prefill, prefill_steps, trailing, trailing_steps, tts_pad);
  });
}

int q3t_prepare_text_noalloc(q3t_engine *e, const int32_t *content_ids, int32_t n_ids, int32_t speaker,
                             int32_t language, int32_t text_lookahead_tokens, float *prefill, int32_t *prefill_steps,
                             float *trailing, int32_t *trailing_steps, float *tts_pad) {
  return guarded([&] {
    using namespace q3t;
    if (!e || !prefill || !prefill_steps || !trailing || !trailing_steps || !tts_pad)
      fail(Q3T_ERR_INVALID, "null argument");
    const TextPlan p = plan_text(*e, content_ids, n_ids, speaker, language, text_lookahead_tokens, n_ids + 1);
    // scratch layout: the plan's workspace, then the output rows [prefill | trailing | pad]
    const size_t H = (size_t)e->talker_hidden, rows = (size_t)p.prefill_steps + p.trailing_steps + 1;
    const size_t ws = text_workspace_bytes(*e, p), need = ws + rows * H * 4;
    if (need > kNoAllocScratchBytes)
      fail(Q3T_ERR_INVALID,
           "%d content ids need %zu bytes of device scratch; q3t_prepare_text_noalloc holds at most %zu "
           "(use q3t_prepare_text for longer prompts)",
           n_ids, need, kNoAllocScratchBytes);
    if (e->scratch_status != hipSuccess) hip_check(e->scratch_status, "hipGetSymbolAddress(scratch)");
    HIPC(hipSetDevice(e->device));
    char *base = (char *)noalloc_scratch(e->device);
    if (!base) fail(Q3T_ERR_HIP, "no device scratch on device %d", e->device);
    float *d = (float *)(base + ws), *dt = d + (size_t)p.prefill_steps * H, *dp = dt + (size_t)p.trailing_steps * H;
    run_text_plan(*e, p, carve_text_workspace(*e, p, base), d, dt, dp, e->pools.stream);
    HIPC(hipMemcpy(prefill, d, (size_t)p.prefill_steps * H * 4, hipMemcpyDeviceToHost));
    HIPC(hipMemcpy(trailing, dt, (size_t)p.trailing_steps * H * 4, hipMemcpyDeviceToHost));
    HIPC(hipMemcpy(tts_pad, dp, H * 4, hipMemcpyDeviceToHost));
    *prefill_steps = p.prefill_steps;
    *trailing_steps = p.trailing_steps;
  });
}

int q3t_prepare_text_voice_clone(q3t_engine *e, const int32_t *content_ids, int32_t n_ids,
                                 const float *speaker_embedding, int32_t embedding_len, int32_t language,
                                 int32_t text_lookahead_tokens, float *prefill, int32_t *prefill_steps,
                                 float *trailing, int32_t *trailing_steps, float *tts_pad) {
  return guarded([&] {
    using namespace q3t;
    if (!e || !speaker_embedding || !prefill || !prefill_steps || !trailing || !trailing_steps || !tts_pad)
      fail(Q3T_ERR_INVALID, "null argument");
    const TextPlan p = plan_text(*e, content_ids, n_ids, 0, language, text_lookahead_tokens, n_ids + 1,
                                 speaker_embedding, embedding_len);
    prepare_text_to_host(e, p, prefill, prefill_steps, trailing, trailing_steps, tts_pad);
  });
}

int q3t_stream_start_text(q3t_engine *e, const int32_t *content_ids, int32_t n_ids, int32_t text_lookahead_tokens,
                          const q3t_generate_options *o, q3t_stream **out) {
  return guarded([&] {
    using namespace q3t;
    if (!e || !out) fail(Q3T_ERR_INVALID, "null engine or output");
    *out = nullptr;
    validate_options(o);
    const TextPlan p = plan_text(*e, content_ids, n_ids, o->speaker, o->language, text_lookahead_tokens, e->cap);
    *out = start_text_stream(e, p, o);
  });
}

int q3t_stream_start_voice_clone(q3t_engine *e, const int32_t *content_ids, int32_t n_ids,
                                 const float *speaker_embedding, int32_t embedding_len,
                                 int32_t text_lookahead_tokens, const q3t_generate_options *o, q3t_stream **out) {
  return guarded([&] {
    using namespace q3t;
    if (!e || !out || !speaker_embedding) fail(Q3T_ERR_INVALID, "null argument");
    *out = nullptr;
    validate_options(o);
    const TextPlan p = plan_text(*e, content_ids, n_ids, 0, o->language, text_lookahead_tokens, e->cap,
                                 speaker_embedding, embedding_len);
    *out = start_text_stream(e, p, o);
  });
}

int q3t_text_stream_start(q3t_engine *e, const int32_t *content_ids, int32_t n_ids, const float *speaker_embedding,
                          int32_t embedding_len, const q3t_generate_options *o, q3t_stream **out) {
  return guarded([&] {
    using namespace q3t;
    if (!e || !out) fail(Q3T_ERR_INVALID, "null engine or output");
    *out = nullptr;
    validate_options(o);
    const TextPlan p = plan_text(*e, content_ids, n_ids, o->speaker, o->language, std::max(n_ids, 1), e->cap,
                                 speaker_embedding, speaker_embedding ? embedding_len : 0, true);
    *out = start_text_stream(e, p, o, true);
  });
}

int q3t_text_stream_push(q3t_stream *sp, const int32_t *ids, int32_t n) {
  return guarded([&] {
    using namespace q3t;
    if (!sp || (n > 0 && !ids)) fail(Q3T_ERR_INVALID, "null argument");
    if (n < 0) fail(Q3T_ERR_INVALID, "token count must not be negative");
    if (!sp->text_open) fail(Q3T_ERR_INVALID, "cannot push text after finish_text");  // generation.rs:1108-1116
    Engine &e = *sp->engine;
    // Rows at max_frames or later are never read (frame f reads row f only when f + 1 < max_frames).
    const int keep = std::max(0, std::min(n, sp->max_frames - sp->text_rows));
    const TextPlan p = plan_trailing_rows(e, ids, n, sp->text_rows);  // checks every id
    if (keep > 0) {
      TextPlan q = p;
      q.ids.resize(keep);
      q.codec.resize(keep);
      q.dst.resize(keep);
      HIPC(hipSetDevice(e.device));
      prepare_text_device(e, q, nullptr, e.slots[sp->slot].trailing, nullptr, e.slots[sp->slot].stream);
    }
    sp->text_rows = std::min<int64_t>((int64_t)sp->text_rows + n, sp->max_frames);
  });
}

int q3t_text_stream_finish(q3t_stream *sp) {
  return guarded([&] {
    using namespace q3t;
    if (!sp) fail(Q3T_ERR_INVALID, "null argument");
    if (!sp->text_open) return;  // finish_text after finish_text is a no-op (generation.rs:1118-1121)
    Engine &e = *sp->engine;
    Slot &s = e.slots[sp->slot];
    const size_t H = (size_t)e.talker_hidden;
    const int R = std::min(sp->text_rows, sp->max_frames);
    HIPC(hipSetDevice(e.device));
    // tts_eos after the last pushed row, then tts_pad for every later frame (generation.rs:1371-1386)
    if (R < sp->max_frames) {
      const TextPlan p = plan_trailing_rows(e, &e.tok_tts_eos, 1, R);
      prepare_text_device(e, p, nullptr, s.trailing, nullptr, s.stream);
    }
    const int T = std::min(R + 1, sp->max_frames);
    HIPC(hipMemcpyAsync(s.trailing + (size_t)T * H, s.trailing + (size_t)e.cap * H, H * 4, hipMemcpyDeviceToDevice,
                        s.stream));
    HIPC(hipStreamSynchronize(s.stream));
    const int32_t rows = T;
    HIPC(hipMemcpy((char *)s.st + offsetof(SlotState, trailing_rows), &rows, sizeof(rows), hipMemcpyHostToDevice));
    sp->text_open = false;
  });
}

int q3t_streams_start(q3t_engine *e, int32_t n, const q3t_stream_input *inputs, const q3t_generate_options *opts,
                      q3t_stream **out) {
  return guarded([&] {
    using namespace q3t;
    if (!e || !inputs || !opts || !out) fail(Q3T_ERR_INVALID, "null argument");
    if (n <= 0) fail(Q3T_ERR_INVALID, "stream count must be positive");
    if (!e->rows_ok) fail(Q3T_ERR_INVALID, "multi-stream batching needs hidden sizes of at most 2048");
    if (!e->bx_t) fail(Q3T_ERR_INVALID, "multi-stream calls need an engine created with max_streams > 1");
    for (int j = 0; j < n; ++j) out[j] = nullptr;
    for (int j = 0; j < n; ++j) validate_input(*e, inputs[j], &opts[j]);
    std::vector<int> slots;
    for (size_t i = 0; i < e->slots.size() && (int)slots.size() < n; ++i)
      if (!e->slots[i].in_use) slots.push_back((int)i);
    if ((int)slots.size() < n)
      fail(Q3T_ERR_BUSY, "%d streams requested but only %zu of %zu slots are free", n, slots.size(), e->slots.size());
    HIPC(hipSetDevice(e->device));
    ensure_trace(*e);
    Pools &p = e->pools;
    // All prompts side by side in the prefill workspace: one GEMM per weight for every stream.
    std::vector<PrefillSeg> segs;
    int M = 0;
    for (int j = 0; j < n; ++j) {
      segs.push_back(PrefillSeg{slots[j], M, inputs[j].prefill_steps});
      M += inputs[j].prefill_steps;
    }
    if (M > p.prefill_rows) fail(Q3T_ERR_CAPACITY, "prompts total %d rows; the workspace holds %d", M, p.prefill_rows);
    for (int j = 0; j < n; ++j) stage_stream(*e, slots[j], segs[j].row0, inputs[j], &opts[j], p.stream);
    e->prefill_segments(segs, M, p.stream);
    const int rows = set_rows(*e, slots, p.stream);
    e->rgemm(EPI_STORE, true, e->codec_head_p, Engine::Act{p.x_t, e->talker_hidden}, e->t_norm, e->td.eps,
             Engine::Act{nullptr, 0}, nullptr, Engine::Act{p.logits_t, e->td.vocab}, e->td.vocab, e->talker_hidden,
             rows, p.stream);
    e->select_talker_rows(rows, 0, Engine::Act{p.x_t, e->talker_hidden}, p.stream);
    HIPC(hipMemcpyAsync(p.h_states, p.st, sizeof(SlotState) * rows, hipMemcpyDeviceToHost, p.stream));
    HIPC(hipStreamSynchronize(p.stream));
    for (int j = 0; j < n; ++j) out[j] = new_stream(*e, slots[j], opts[j].max_frames);
  });
}

int q3t_streams_next_codes(q3t_engine *e, q3t_stream *const *streams, int32_t n, int32_t max_chunk, int32_t *codes,
                           q3t_chunk_info *info) {
  return guarded([&] {
    using namespace q3t;
    if (!e || !streams || !info || (n > 0 && !codes)) fail(Q3T_ERR_INVALID, "null argument");
    if (n <= 0) fail(Q3T_ERR_INVALID, "stream count must be positive");
    if (max_chunk <= 0) fail(Q3T_ERR_INVALID, "max_chunk_frames must be non-zero");
    if (!e->rows_ok) fail(Q3T_ERR_INVALID, "multi-stream batching needs hidden sizes of at most 2048");
    if (!e->bx_t) fail(Q3T_ERR_INVALID, "multi-stream calls need an engine created with max_streams > 1");
    std::vector<int> seen(e->slots.size(), 0), on, want(n, 0);
    int nrun = 0;
    for (int j = 0; j < n; ++j) {
      q3t_stream *sp = streams[j];
      if (!sp || sp->engine != e) fail(Q3T_ERR_INVALID, "stream %d is null or belongs to another engine", j);
      if (seen[sp->slot]++) fail(Q3T_ERR_INVALID, "stream %d is listed twice", j);
      if (sp->text_open)
        fail(Q3T_ERR_INVALID, "stream %d has open text input; advance it with q3t_stream_next_codes", j);
      info[j].frames = 0;
      info[j].total_frames = sp->host_frame;
      info[j].ended_by_eos = sp->done == 1;
      if (sp->done || sp->host_frame >= sp->max_frames) continue;
      want[j] = std::min(max_chunk, sp->max_frames - sp->host_frame);
      nrun = std::max(nrun, want[j]);
      on.push_back(sp->slot);
    }
    if (nrun == 0) return;
    HIPC(hipSetDevice(e->device));
    if (on.size() == 1) {
      // One stream to run (the tail of a ragged batch, once the others have ended): the
      // single-stream frame (GEMV kernels, 1.7 ms for the 0.6B shape) instead of a batched
      // frame, which costs about the same at 1 live row as at 16 (2.7 ms).  Both read and
      // write the same per-slot state (caches, loop state, codes, the next pass's inputs) at
      // frame boundaries, so a stream may take either path at any frame.
      for (int j = 0; j < n; ++j)
        if (want[j]) {
          run_frames(*e, e->slots[streams[j]->slot], want[j]);
          collect_frames(streams[j], want[j], codes + (size_t)j * max_chunk * e->groups, &info[j]);
        }
      return;
    }
    Pools &p = e->pools;
    const int rows = set_rows(*e, on, p.stream);
    bool fused = e->rows_handoff_ok();
    for (int slot : on) fused = fused && e->slots[slot].cp_greedy;
    // Streams that need fewer frames than nrun reach max_frames on the device and stop there.
    run_rows_frames(*e, rows, nrun, fused);
    // Every row's frames [lo, hi) (a window covering each listed stream's frames; the rest is
    // never read) and the states in one round trip, instead of one synchronous copy per stream.
    int lo = INT32_MAX, hi = 0;
    for (int j = 0; j < n; ++j)
      if (want[j]) {
        lo = std::min(lo, streams[j]->host_frame);
        hi = std::max(hi, streams[j]->host_frame + want[j]);
      }
    const size_t pitch = (size_t)p.codes_row * 4;
    HIPC(hipMemcpy2DAsync(p.h_codes + (size_t)lo * e->groups, pitch, p.codes + (size_t)lo * e->groups, pitch,
                          (size_t)(hi - lo) * e->groups * 4, rows, hipMemcpyDeviceToHost, p.stream));
    HIPC(hipMemcpyAsync(p.h_states, p.st, sizeof(SlotState) * rows, hipMemcpyDeviceToHost, p.stream));
    HIPC(hipStreamSynchronize(p.stream));
    for (int j = 0; j < n; ++j) {
      q3t_stream *sp = streams[j];
      if (!want[j]) continue;
      const SlotState &hs = p.h_states[sp->slot];
      const int produced = hs.frame - sp->host_frame;
      if (produced < 0 || produced > want[j]) fail(Q3T_ERR_HIP, "device loop state is inconsistent");
      if (produced > 0)
        std::memcpy(codes + (size_t)j * max_chunk * e->groups,
                    p.h_codes + (size_t)sp->slot * p.codes_row + (size_t)sp->host_frame * e->groups,
                    (size_t)produced * e->groups * 4);
      sp->host_frame += produced;
      sp->done = hs.done;
      info[j].frames = produced;
      info[j].total_frames = sp->host_frame;
      info[j].ended_by_eos = sp->done == 1;
    }
  });
}

}  // extern "C"

namespace q3t {
namespace {

// The frames a next_codes call may run (0: none, the stream has ended or waits for text);
// fills info for the no-frames case.
int frames_to_run(q3t_stream *sp, int max_chunk, int32_t *codes, q3t_chunk_info *info) {
  if (!sp || !info || (max_chunk > 0 && !codes)) fail(Q3T_ERR_INVALID, "null argument");
  if (max_chunk <= 0) fail(Q3T_ERR_INVALID, "max_chunk_frames must be non-zero");
  info->frames = 0;
  info->total_frames = sp->host_frame;
  info->ended_by_eos = sp->done == 1;
  if (sp->done || sp->host_frame >= sp->max_frames) return 0;
  int n = std::min(max_chunk, sp->max_frames - sp->host_frame);
  // Open text: frame f (f + 1 < max_frames) reads trailing row f, which must have been pushed;
  // frames = 0 without the end flags is the reference's NeedMoreText (generation.rs:1150-1158,
  // 1200-1208).
  if (sp->text_open && sp->text_rows < sp->max_frames - 1)
    n = std::min(n, std::max(0, sp->text_rows - sp->host_frame));
  return n;
}

// The CodePredictor (phase 0) and the Talker step (phase 1) of a frame, each captured as a
// graph of the slot (as run_frames captures the whole frame).
void ensure_phase_graphs(Engine &e, Slot &s) {
  if (s.phase_graph[0] && s.phase_traced == (bool)e.trace && s.phase_cp_greedy == s.cp_greedy) return;
  for (hipGraphExec_t &g : s.phase_graph)
    if (g) {
      HIPC(hipGraphExecDestroy(g));
      g = nullptr;
    }
  for (int ph = 0; ph < 3; ++ph) {
    hipGraph_t g = nullptr;
    HIPC(hipStreamBeginCapture(s.stream, hipStreamCaptureModeThreadLocal));
    try {
      if (ph == 0) e.enqueue_code_predictor(s, s.stream, e.fold_last_group(s));
      else e.enqueue_talker_decode(s, s.stream, e.fold_last_group(s), ph == 2);
    } catch (...) {
      (void)hipStreamEndCapture(s.stream, &g);
      if (g) (void)hipGraphDestroy(g);
      throw;
    }
    HIPC(hipStreamEndCapture(s.stream, &g));
    const hipError_t err = hipGraphInstantiate(&s.phase_graph[ph], g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    hip_check(err, "hipGraphInstantiate");
  }
  s.phase_traced = (bool)e.trace;
  s.phase_cp_greedy = s.cp_greedy;
}

// After up to n frames ran: the new codes to the caller, the host's view of the stream.


}  // namespace
}  // namespace q3t

extern "C" {

int q3t_stream_next_codes(q3t_stream *sp, int32_t max_chunk, int32_t *codes, q3t_chunk_info *info) {
  return guarded([&] {
    using namespace q3t;
    const int n = frames_to_run(sp, max_chunk, codes, info);
    if (n == 0) return;
    Engine &e = *sp->engine;
    HIPC(hipSetDevice(e.device));
    run_frames(e, e.slots[sp->slot], n);
    collect_frames(sp, n, codes, info);
  });
}

int q3t_stream_next_codes_profiled(q3t_stream *sp, int32_t max_chunk, int32_t *codes, q3t_chunk_info *info,
                                   q3t_profile *prof) {
  return guarded([&] {
    using namespace q3t;
    if (!prof) fail(Q3T_ERR_INVALID, "null argument");
    const int n = frames_to_run(sp, max_chunk, codes, info);
    if (n == 0) return;
    Engine &e = *sp->engine;
    Slot &s = e.slots[sp->slot];
    HIPC(hipSetDevice(e.device));
    Events ev(3);
    int ran = 0;
    // One frame at a time (rollout_profiled, generation.rs:751-874): a frame after the end of
    // the stream is not run, so that it adds no time.
    while (ran < n && !s.h_state->done) {
      const bool split = fused_frames(e, s, 1) == 0;
      HIPC(hipEventRecord(ev.ev[0], s.stream));
      e.enqueue_code_predictor(s, s.stream, e.fold_last_group(s));
      HIPC(hipEventRecord(ev.ev[1], s.stream));
      e.enqueue_talker_decode(s, s.stream, e.fold_last_group(s), split);
      HIPC(hipEventRecord(ev.ev[2], s.stream));
      sync_state(s);
      prof->code_predictor_seconds += ev.seconds(0, 1);
      prof->talker_decode_seconds += ev.seconds(1, 2);
      ++ran;
    }
    collect_frames(sp, n, codes, info);
  });
}

int q3t_debug_phase_times(q3t_stream *sp, int32_t max_chunk, int32_t *codes, q3t_chunk_info *info, float *cp_us,
                          float *talker_us, int32_t *timed) {
  return guarded([&] {
    using namespace q3t;
    if (!cp_us || !talker_us || !timed) fail(Q3T_ERR_INVALID, "null argument");
    *timed = 0;
    const int n = frames_to_run(sp, max_chunk, codes, info);
    if (n == 0) return;
    Engine &e = *sp->engine;
    Slot &s = e.slots[sp->slot];
    HIPC(hipSetDevice(e.device));
    if (e.use_graph) ensure_phase_graphs(e, s);
    Events ev(3);
    int ran = 0;
    while (ran < n && !s.h_state->done) {
      const bool split = fused_frames(e, s, 1) == 0;
      HIPC(hipEventRecord(ev.ev[0], s.stream));
      if (e.use_graph) HIPC(hipGraphLaunch(s.phase_graph[0], s.stream));
      else e.enqueue_code_predictor(s, s.stream, e.fold_last_group(s));
      HIPC(hipEventRecord(ev.ev[1], s.stream));
      if (e.use_graph) HIPC(hipGraphLaunch(s.phase_graph[split ? 2 : 1], s.stream));
      else e.enqueue_talker_decode(s, s.stream, e.fold_last_group(s), split);
      HIPC(hipEventRecord(ev.ev[2], s.stream));
      sync_state(s);
      cp_us[ran] = (float)(1e6 * ev.seconds(0, 1));
      talker_us[ran] = (float)(1e6 * ev.seconds(1, 2));
      ++ran;
    }
    *timed = ran;
    collect_frames(sp, n, codes, info);
  });
}

int q3t_decode_codes(q3t_engine *e, const int32_t *codes, int32_t frames, float *samples) {
  return guarded([&] {
    using namespace q3t;
    if (!e || (frames > 0 && (!codes || !samples))) fail(Q3T_ERR_INVALID, "null argument");
    if (frames < 0) fail(Q3T_ERR_INVALID, "frame count must not be negative");
    if (!e->codec) fail(Q3T_ERR_NOT_FOUND, "the model directory has no speech_tokenizer/model.safetensors");
    if (frames == 0) return;  // decode_codes of no codes: no samples (generation.rs:628-630)
    HIPC(hipSetDevice(e->device));
    hipStream_t s = e->pools.stream;
    int32_t *dc = codec_codes_buffer(*e->codec, (size_t)frames * e->groups);
    float *ds = codec_samples_buffer(*e->codec, (size_t)frames * kCodecSamplesPerFrame);
    HIPC(hipMemcpyAsync(dc, codes, (size_t)frames * e->groups * 4, hipMemcpyHostToDevice, s));
    codec_decode(*e->codec, dc, frames, e->groups, ds, s);
    HIPC(hipMemcpy(samples, ds, (size_t)frames * kCodecSamplesPerFrame * 4, hipMemcpyDeviceToHost));
  });
}

int q3t_stream_next_audio(q3t_stream *sp, int32_t max_chunk, int32_t left_context, int32_t *codes, float *samples,
                          int32_t *n_samples, q3t_chunk_info *info) {
  using namespace q3t;
  if (!sp || !codes || !samples || !n_samples || !info) {
    g_last_error = "null argument";
    return Q3T_ERR_INVALID;
  }
  if (!sp->engine->codec) {
    g_last_error = "the model directory has no speech_tokenizer/model.safetensors";
    return Q3T_ERR_NOT_FOUND;
  }
  if (left_context < 0) {
    g_last_error = "left_context_frames must not be negative";
    return Q3T_ERR_INVALID;
  }
  *n_samples = 0;
  const int rc = q3t_stream_next_codes(sp, max_chunk, codes, info);
  if (rc != Q3T_OK || info->frames == 0) return rc;
  return guarded([&] {
    // next_audio_chunk (generation.rs:965-989): decode the chunk with up to left_context
    // earlier frames (the slot keeps every frame's codes on the device) and keep the chunk's
    // own samples.
    Engine &e = *sp->engine;
    HIPC(hipSetDevice(e.device));
    const int start = info->total_frames - info->frames;
    const int ctx = std::min(left_context, start);
    const int n = info->frames + ctx;
    hipStream_t s = e.slots[sp->slot].stream;
    float *ds = codec_samples_buffer(*e.codec, (size_t)n * kCodecSamplesPerFrame);
    codec_decode(*e.codec, e.slots[sp->slot].codes + (size_t)(start - ctx) * e.groups, n, e.groups, ds, s);
    HIPC(hipMemcpy(samples, ds + (size_t)ctx * kCodecSamplesPerFrame,
                   (size_t)info->frames * kCodecSamplesPerFrame * 4, hipMemcpyDeviceToHost));
    *n_samples = info->frames * kCodecSamplesPerFrame;
  });
}

int q3t_stream_destroy(q3t_stream *sp) {
  return guarded([&] {
    if (!sp) return;
    Engine &e = *sp->engine;
    (void)hipSetDevice(e.device);
    (void)hipStreamSynchronize(e.slots[sp->slot].stream);
    (void)hipStreamSynchronize(e.pools.stream);
    e.slots[sp->slot].in_use = false;
    delete sp;
  });
}

int q3t_stream_read_talker_logits(q3t_stream *sp, float *out, int32_t capacity, int32_t *rows) {
  return guarded([&] {
    if (!sp || !rows) fail(Q3T_ERR_INVALID, "null argument");
    Engine &e = *sp->engine;
    auto &s = e.slots[sp->slot];
    if (!s.trace_t) fail(Q3T_ERR_INVALID, "logit tracing was off when the stream started");
    // Row 0: prefill; row f + 1: after frame f (only frames followed by a Talker step).
    int n = sp->host_frame + 1;
    if (sp->host_frame >= sp->max_frames) n = sp->max_frames;  // the last frame has no Talker step
    n = std::min(n, capacity);
    if (n > 0 && out)
      HIPC(hipMemcpy(out, s.trace_t, (size_t)n * e.td.vocab * 4, hipMemcpyDeviceToHost));
    *rows = n;
  });
}

int q3t_stream_read_cp_logits(q3t_stream *sp, float *out, int32_t capacity, int32_t *frames) {
  return guarded([&] {
    if (!sp || !frames) fail(Q3T_ERR_INVALID, "null argument");
    Engine &e = *sp->engine;
    auto &s = e.slots[sp->slot];
    if (!s.trace_c) fail(Q3T_ERR_INVALID, "logit tracing was off when the stream started");
    const int n = std::min(sp->host_frame, capacity);
    if (n > 0 && out)
      HIPC(hipMemcpy(out, s.trace_c, (size_t)n * (e.groups - 1) * e.cd.vocab * 4, hipMemcpyDeviceToHost));
    *frames = n;
  });
}

int q3t_engine_synchronize(q3t_engine *e) {
  return guarded([&] {
    if (!e) fail(Q3T_ERR_INVALID, "null engine");
    HIPC(hipSetDevice(e->device));
    for (auto &s : e->slots) HIPC(hipStreamSynchronize(s.stream));
    HIPC(hipStreamSynchronize(e->pools.stream));
  });
}

}  // extern "C"

namespace q3t {
namespace {

// Stream slot 0 prepared for a parity hook: free, greedy on both heads, no history, frame 0.
Slot &hook_slot(Engine &e, int prefill_steps, int max_frames) {
  Slot &s = e.slots[0];
  if (s.in_use) fail(Q3T_ERR_BUSY, "stream slot 0 is in use");
  HIPC(hipSetDevice(e.device));
  HIPC(hipStreamSynchronize(s.stream));
  SlotState st0{};
  st0.semantic = 0;
  st0.prefill_steps = prefill_steps;
  st0.max_frames = max_frames;
  SlotParams pr{};
  pr.repetition_penalty = 1.0f;
  pr.codec_eos = e.codec_eos;
  s.cp_greedy = true;
  HIPC(hipMemcpy(s.st, &st0, sizeof st0, hipMemcpyHostToDevice));
  HIPC(hipMemcpy(s.prm, &pr, sizeof pr, hipMemcpyHostToDevice));
  return s;
}

// Talker head on slot 0 after a prefill or step: normed hidden (the CodePredictor prefix's
// first row), raw logits and the greedy token over the suppressed logits.
void talker_head_out(Engine &e, Slot &s, float *hidden, float *logits, int32_t *token) {
  e.gemv(EPI_STORE, true, e.codec_head, s.x_t, e.t_norm, e.td.eps, nullptr, nullptr, s.logits_t, e.td.vocab,
         e.td.hidden, SKIP_NEVER, s.st, s.stream);
  e.select_talker(s, 0, s.stream, false);
  HIPC(hipStreamSynchronize(s.stream));
  HIPC(hipMemcpy(hidden, s.cp_prefix, (size_t)e.td.hidden * 4, hipMemcpyDeviceToHost));
  HIPC(hipMemcpy(logits, s.logits_t, (size_t)e.td.vocab * 4, hipMemcpyDeviceToHost));
  SlotState st{};
  HIPC(hipMemcpy(&st, s.st, sizeof st, hipMemcpyDeviceToHost));
  *token = st.semantic;
}

}  // namespace
}  // namespace q3t

extern "C" {

int q3t_debug_talker_prefill(q3t_engine *e, const float *prefill, int32_t steps, float *hidden, float *logits,
                             int32_t *token) {
  return guarded([&] {
    using namespace q3t;
    if (!e || !prefill || !hidden || !logits || !token) fail(Q3T_ERR_INVALID, "null argument");
    if (steps <= 0) fail(Q3T_ERR_INVALID, "prefill steps must be non-zero");
    if (steps >= e->cap) fail(Q3T_ERR_CAPACITY, "prefill of %d steps needs a larger max_cache_steps (%d)", steps, e->cap);
    Slot &s = hook_slot(*e, steps, 1);
    HIPC(hipMemcpy(e->pools.px, prefill, (size_t)steps * e->td.hidden * 4, hipMemcpyHostToDevice));
    e->prefill_segments({PrefillSeg{0, 0, steps}}, steps, s.stream);
    talker_head_out(*e, s, hidden, logits, token);
  });
}

int q3t_debug_talker_step(q3t_engine *e, const float *input, int32_t offset, float *hidden, float *logits,
                          int32_t *token) {
  return guarded([&] {
    using namespace q3t;
    if (!e || !input || !hidden || !logits || !token) fail(Q3T_ERR_INVALID, "null argument");
    if (offset < 0 || offset >= e->cap) fail(Q3T_ERR_CAPACITY, "offset %d outside the %d-step cache", offset, e->cap);
    // position = prefill_steps + frame = offset; max_frames 2 keeps the step from being skipped
    Slot &s = hook_slot(*e, offset, 2);
    HIPC(hipMemcpy(s.t_in, input, (size_t)e->td.hidden * 4, hipMemcpyHostToDevice));
    e->stack_step(e->talker, s.t_k, s.t_v, s.t_in, s.x_t, s, POS_TALKER_FRAME, 0, SKIP_TALKER, s.stream);
    talker_head_out(*e, s, hidden, logits, token);
  });
}

int q3t_debug_code_predictor(q3t_engine *e, const float *talker_hidden, const float *semantic_embed, int32_t *tokens,
                             float *embedding_sum) {
  return guarded([&] {
    using namespace q3t;
    if (!e || !talker_hidden || !semantic_embed || !tokens || !embedding_sum) fail(Q3T_ERR_INVALID, "null argument");
    Slot &s = hook_slot(*e, 0, 1);
    const size_t row = (size_t)e->talker_hidden * 4;
    HIPC(hipMemcpy(s.cp_prefix, talker_hidden, row, hipMemcpyHostToDevice));
    HIPC(hipMemcpy(s.cp_prefix + e->talker_hidden, semantic_embed, row, hipMemcpyHostToDevice));
    e->enqueue_code_predictor(s, s.stream);
    HIPC(hipStreamSynchronize(s.stream));
    std::vector<int32_t> codes(e->groups);
    HIPC(hipMemcpy(codes.data(), s.codes, (size_t)e->groups * 4, hipMemcpyDeviceToHost));
    for (int g = 1; g < e->groups; ++g) tokens[g - 1] = codes[g];
    HIPC(hipMemcpy(embedding_sum, s.emb_sum, row, hipMemcpyDeviceToHost));
  });
}

namespace {
int bench_kernel_impl(q3t_engine *e, int32_t kernel, int32_t iters, double *avg_us, double *bytes, bool timed) {
  return q3t::guarded([&] {
    using namespace q3t;
    if (!e || !avg_us || !bytes) fail(Q3T_ERR_INVALID, "null argument");
    if (iters <= 0 || iters > 8192) fail(Q3T_ERR_INVALID, "iters must be in 1..8192");
    if (kernel < 0 || kernel > 10) fail(Q3T_ERR_INVALID, "unknown kernel class %d", kernel);
    if (kernel == 9 && !e->oproj_ok(e->cp)) fail(Q3T_ERR_INVALID, "the model's CodePredictor has no fused O projection");
    if (kernel == 10 && !e->talker_heads_o(e->talker))
      fail(Q3T_ERR_INVALID, "the model's Talker has no fused attention + O projection");
    Slot &s = e->slots[0];
    if (s.in_use) fail(Q3T_ERR_BUSY, "stream slot 0 is in use");
    HIPC(hipSetDevice(e->device));
    const Dims &td = e->td, &cd = e->cd;
    // The launch sequence one frame issues for this kernel class: Talker layers first, then
    // the CodePredictor layers of its 15 passes (the order enqueue_frame uses).
    struct L {
      const StackW *w;
      int layer;
    };
    std::vector<L> seq;
    if (kernel <= 3) {
      for (int l = 0; l < td.layers; ++l) seq.push_back({&e->talker, l});
      for (int g = 0; g < e->groups - 1; ++g)
        for (int l = 0; l < cd.layers; ++l) seq.push_back({&e->cp, l});
    } else if (kernel == 5 || kernel == 9) {  // CodePredictor attention: positions 0..groups-1, each over 5 layers
      for (int p = 0; p < e->groups; ++p)
        for (int l = 0; l < cd.layers; ++l) seq.push_back({&e->cp, l});
    } else if (kernel == 6 || kernel == 8) {  // one per CodePredictor group
      for (int g = 0; g < e->groups - 1; ++g) seq.push_back({&e->cp, 0});
    } else {
      for (int l = 0; l < td.layers; ++l) seq.push_back({&e->talker, l});
    }
    if (kernel == 6) {  // greedy selection, fixed state (frame 0, not done)
      SlotState st0{};
      st0.semantic = 0;
      st0.max_frames = 1;
      HIPC(hipMemcpy(s.st, &st0, sizeof st0, hipMemcpyHostToDevice));
      SlotParams pr{};
      pr.codec_eos = e->codec_eos;
      HIPC(hipMemcpy(s.prm, &pr, sizeof pr, hipMemcpyHostToDevice));
    }
    if (timed && kernel == 6) fail(Q3T_ERR_INVALID, "kernel class 6 has no timed launch");
    if (!timed && !e->use_graph)
      fail(Q3T_ERR_INVALID, "the engine runs without graphs (use_graph = 0); q3t_bench_kernel captures one: "
                            "use q3t_bench_kernel_timed");
    double total_bytes = 0.0;
    const LaunchTiming *lt = nullptr;  // set per launch in the timed mode
    auto enqueue = [&](int i, bool count) {
      const L &l = seq[(size_t)i % seq.size()];
      const Dims &d = l.w->d;
      const LayerW &W = l.w->layers[l.layer];
      const float *xin = l.w == &e->talker ? s.x_t : s.x_c;
      const bool nt = l.w == &e->talker;
      double b = 0.0;
      switch (kernel) {
        case 0:  // QKV projection with the input RMSNorm prologue
          e->gemv(EPI_STORE, true, W.qkv, xin, W.g_in, d.eps, nullptr, nullptr, s.qkv, d.qkv_rows(), d.hidden,
                  SKIP_NEVER, s.st, s.stream, nt, lt);
          b = 2.0 * d.qkv_rows() * d.hidden + 4.0 * (d.hidden * 2 + d.qkv_rows());
          break;
        case 1: {  // O projection + residual (Talker layers merge split-attention partials first;
                   // frames of a Talker with the fused attention + O run class 10 instead)
          GemvArgs og{W.o, s.attn, nullptr, s.act, nullptr, s.act, d.hidden, d.q_out(), 0.f, SKIP_NEVER, s.st};
          if (nt && attn_chunks(l.w->cap) <= kAttnGemvMergeChunks) {
            og.x = nullptr;
            og.attn_part = s.attn_part;
            og.attn_part_chunks = s.attn_part_chunks;
            og.attn_chunk = attn_chunk_len(l.w->cap);
            og.attn_pos_mode = POS_CONST;
            og.attn_pos_const = l.w->cap / 2;
            og.attn_q_heads = d.q_heads;
            og.attn_kv_heads = d.kv_heads;
          }
          hip_check(launch_gemv(EPI_RESIDUAL, false, nt, og, s.stream, lt), "launch_gemv");
          b = 2.0 * d.hidden * d.q_out() + 4.0 * (d.q_out() + 2 * d.hidden);
          break;
        }
        case 2: {  // gate/up projection with the post-attention RMSNorm prologue and SwiGLU; the
                   // CodePredictor's (fused O projection) also sums the per-head partials into x
          GemvArgs gu{W.gu, xin, W.g_post, nullptr, nullptr, s.act, d.intermediate, d.hidden, d.eps, SKIP_NEVER, s.st};
          b = 2.0 * 2 * d.intermediate * d.hidden + 4.0 * (2 * d.hidden + d.intermediate);
          if (e->oproj_ok(*l.w) || e->talker_heads_o(*l.w)) {
            gu.parts = s.opart;
            gu.n_parts = d.kv_heads;
            gu.ld_parts = d.hidden;
            gu.x_store = s.x_mid;
            b += 4.0 * (d.kv_heads + 1) * d.hidden;
          }
          hip_check(launch_gemv(EPI_SWIGLU, true, nt, gu, s.stream, lt), "launch_gemv");
          break;
        }
        case 3:  // down projection + residual
          e->gemv(EPI_RESIDUAL, false, W.down, s.act, nullptr, 0.f, s.attn, nullptr, s.attn, d.hidden,
                  d.intermediate, SKIP_NEVER, s.st, s.stream, nt, lt);
          b = 2.0 * d.hidden * d.intermediate + 4.0 * (d.intermediate + 2 * d.hidden);
          break;
        case 4: {  // Talker attention over a full cache (L = max_cache_steps)
          const size_t esz = e->kv_bf16 ? 2 : 4;
          const size_t layer_bytes = (size_t)d.kv_heads * l.w->cap * d.head_dim * esz;
          AttnArgs aa{s.qkv, W.gq, W.gk, l.w->rope, s.t_k + layer_bytes * l.layer, s.t_v + layer_bytes * l.layer,
                      s.attn, d.q_heads, d.kv_heads, l.w->cap, d.eps, 1.0f / std::sqrt((float)d.head_dim),
                      POS_CONST, l.w->cap - 1, SKIP_NEVER, e->kv_bf16, s.st, s.attn_part, s.attn_part_chunks,
                      attn_chunk_len(l.w->cap), attn_chunks(l.w->cap) > 1 ? 1 : 0};
          hip_check(launch_attn_decode(aa, d.head_dim, s.stream, lt), "launch_attn_decode");
          b = 2.0 * esz * d.kv_heads * d.head_dim * l.w->cap + 4.0 * (d.qkv_rows() + d.q_out());
          break;
        }
        case 5: {  // CodePredictor attention at position (i / layers) % groups (one chunk, direct output)
          const size_t esz = e->kv_bf16 ? 2 : 4;
          const size_t layer_bytes = (size_t)d.kv_heads * l.w->cap * d.head_dim * esz;
          const int pos = (i / d.layers) % e->groups;
          AttnArgs aa{s.qkv, W.gq, W.gk, l.w->rope, s.c_k + layer_bytes * l.layer, s.c_v + layer_bytes * l.layer,
                      s.attn, d.q_heads, d.kv_heads, l.w->cap, d.eps, 1.0f / std::sqrt((float)d.head_dim),
                      POS_CONST, pos, SKIP_NEVER, e->kv_bf16, s.st, s.attn_part, s.attn_part_chunks,
                      attn_chunk_len(l.w->cap), 0};
          hip_check(launch_attn_decode(aa, d.head_dim, s.stream, lt), "launch_attn_decode");
          b = 2.0 * esz * d.kv_heads * d.head_dim * (pos + 1) + 4.0 * (d.qkv_rows() + d.q_out());
          break;
        }
        case 6: {  // greedy CodePredictor token selection + embedding gathers
          const int g = i % (e->groups - 1);
          SelectCpArgs a{s.logits_c, e->cp_emb + (size_t)g * cd.vocab * e->talker_hidden, s.cur, s.emb_sum, s.codes,
                         nullptr, s.t_in, e->codec_emb, s.trailing, s.st, s.prm, cd.vocab, e->talker_hidden,
                         e->groups, g};
          hip_check(launch_select_cp(a, s.stream), "launch_select_cp");
          b = 4.0 * cd.vocab + 2.0 * e->talker_hidden;
          break;
        }
        case 7: {  // Talker attention at half the cache (split chunks; the O-projection merge not included)
          const size_t esz = e->kv_bf16 ? 2 : 4;
          const size_t layer_bytes = (size_t)d.kv_heads * l.w->cap * d.head_dim * esz;
          AttnArgs aa{s.qkv, W.gq, W.gk, l.w->rope, s.t_k + layer_bytes * l.layer, s.t_v + layer_bytes * l.layer,
                      s.attn, d.q_heads, d.kv_heads, l.w->cap, d.eps, 1.0f / std::sqrt((float)d.head_dim),
                      POS_CONST, l.w->cap / 2, SKIP_NEVER, e->kv_bf16, s.st, s.attn_part, s.attn_part_chunks,
                      attn_chunk_len(l.w->cap), attn_chunks(l.w->cap) > 1 ? 1 : 0};
          hip_check(launch_attn_decode(aa, d.head_dim, s.stream, lt), "launch_attn_decode");
          b = 2.0 * esz * d.kv_heads * d.head_dim * (l.w->cap / 2 + 1) + 4.0 * (d.qkv_rows() + d.q_out());
          break;
        }
        case 9: {  // CodePredictor attention with the O projection fused (per-head partials)
          const size_t esz = e->kv_bf16 ? 2 : 4;
          const size_t layer_bytes = (size_t)d.kv_heads * l.w->cap * d.head_dim * esz;
          const int pos = (i / d.layers) % e->groups;
          AttnArgs aa{s.qkv, W.gq, W.gk, l.w->rope, s.c_k + layer_bytes * l.layer, s.c_v + layer_bytes * l.layer,
                      nullptr, d.q_heads, d.kv_heads, l.w->cap, d.eps, 1.0f / std::sqrt((float)d.head_dim),
                      POS_CONST, pos, SKIP_NEVER, e->kv_bf16, s.st, nullptr, 0, attn_chunk_len(l.w->cap), 0};
          aa.wo = W.o;
          aa.wo_rows = d.hidden;
          aa.opart = s.opart;
          hip_check(launch_attn_oproj(aa, d.head_dim, s.stream, lt), "launch_attn_oproj");
          b = 2.0 * esz * d.kv_heads * d.head_dim * (pos + 1) + 4.0 * d.qkv_rows() + 2.0 * d.hidden * d.q_out() +
              4.0 * d.kv_heads * d.hidden;
          break;
        }
        case 10: {  // Talker attention with the O projection fused (per-head shares), half the cache
          const size_t esz = e->kv_bf16 ? 2 : 4;
          const size_t layer_bytes = (size_t)d.kv_heads * l.w->cap * d.head_dim * esz;
          const int pos = l.w->cap / 2;
          AttnArgs aa{s.qkv, W.gq, W.gk, l.w->rope, s.t_k + layer_bytes * l.layer, s.t_v + layer_bytes * l.layer,
                      nullptr, d.q_heads, d.kv_heads, l.w->cap, d.eps, 1.0f / std::sqrt((float)d.head_dim),
                      POS_CONST, pos, SKIP_NEVER, e->kv_bf16, s.st, nullptr, 0, attn_chunk_len(l.w->cap), 0};
          aa.wo = W.o;
          aa.wo_rows = d.hidden;
          aa.opart = s.opart;
          hip_check(launch_attn_oproj_full(aa, d.head_dim, s.stream, lt), "launch_attn_oproj_full");
          b = 2.0 * esz * d.kv_heads * d.head_dim * (pos + 1) + 4.0 * d.qkv_rows() + 2.0 * d.hidden * d.q_out() +
              4.0 * d.kv_heads * d.hidden;
          break;
        }
        case 8: {  // CodePredictor LM head (final norm prologue)
          const int g = i % (e->groups - 1);
          e->gemv(EPI_STORE, true, e->lm_heads + (size_t)g * cd.vocab * cd.hidden, s.x_c, e->c_norm, cd.eps,
                  nullptr, nullptr, s.logits_c, cd.vocab, cd.hidden, SKIP_NEVER, s.st, s.stream, false, lt);
          b = 2.0 * cd.vocab * cd.hidden + 4.0 * (2 * cd.hidden + cd.vocab);
          break;
        }
      }
      if (count) total_bytes += b;
    };
    // Capture the launches as one graph (the way frames run), replay once to warm, then
    // time one replay: average = elapsed / iters, inter-launch gaps included.
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    auto cleanup = [&] {
      if (ge) (void)hipGraphExecDestroy(ge);
      if (g) (void)hipGraphDestroy(g);
      if (ev0) (void)hipEventDestroy(ev0);
      if (ev1) (void)hipEventDestroy(ev1);
    };
    if (timed) {
      // Eager launches, each bracketed by its own dispatch's start / stop timestamps
      // (hipExtLaunchKernelGGL events): the kernel's duration without the launch gap, the
      // quantity a kernel trace reports per dispatch.  One warm pass first.
      Events evs(2 * iters);
      for (int i = 0; i < iters; ++i) enqueue(i, false);
      HIPC(hipStreamSynchronize(s.stream));
      for (int i = 0; i < iters; ++i) {
        const LaunchTiming t{evs.ev[2 * i], evs.ev[2 * i + 1]};
        lt = &t;
        enqueue(i, true);
        lt = nullptr;
      }
      HIPC(hipStreamSynchronize(s.stream));
      double us = 0.0;
      for (int i = 0; i < iters; ++i) us += 1e6 * evs.seconds(2 * i, 2 * i + 1);
      *avg_us = us / iters;
      *bytes = total_bytes / iters;
      return;
    }
    try {
      HIPC(hipStreamBeginCapture(s.stream, hipStreamCaptureModeThreadLocal));
      try {
        for (int i = 0; i < iters; ++i) enqueue(i, true);
      } catch (...) {
        (void)hipStreamEndCapture(s.stream, &g);
        throw;
      }
      HIPC(hipStreamEndCapture(s.stream, &g));
      HIPC(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
      HIPC(hipEventCreate(&ev0));
      HIPC(hipEventCreate(&ev1));
      HIPC(hipGraphLaunch(ge, s.stream));
      HIPC(hipEventRecord(ev0, s.stream));
      HIPC(hipGraphLaunch(ge, s.stream));
      HIPC(hipEventRecord(ev1, s.stream));
      HIPC(hipStreamSynchronize(s.stream));
      float ms = 0.f;
      HIPC(hipEventElapsedTime(&ms, ev0, ev1));
      *avg_us = 1000.0 * ms / iters;
      *bytes = total_bytes / iters;
    } catch (...) {
      cleanup();
      throw;
    }
    cleanup();
  });
}
}  // namespace

int q3t_bench_kernel(q3t_engine *e, int32_t kernel, int32_t iters, double *avg_us, double *bytes) {
  return bench_kernel_impl(e, kernel, iters, avg_us, bytes, false);
}

int q3t_bench_kernel_timed(q3t_engine *e, int32_t kernel, int32_t iters, double *avg_us, double *bytes) {
  return bench_kernel_impl(e, kernel, iters, avg_us, bytes, true);
}

int q3t_debug_gemm(q3t_engine *e, int32_t epi, const float *X, int32_t M, int32_t K, const uint16_t *W, int32_t N,
                   const float *gamma, float eps, const float *res, const float *bias, float *Y) {
  return guarded([&] {
    using namespace q3t;
    if (!e || !X || !W || !Y) fail(Q3T_ERR_INVALID, "null argument");
    if (M <= 0 || N <= 0 || K <= 0 || K % 32) fail(Q3T_ERR_INVALID, "need M, N > 0 and K a positive multiple of 32");
    // 4: the residual product in the batched frame's K-split form (GemmArgs::split2).
    const bool split2 = epi == 4;
    if (split2) {
      if (M > 16 || gamma || !gemm_skinny_split2_supports(K) || N % 32)
        fail(Q3T_ERR_INVALID, "the split GEMM needs M <= 16, K = 1024 * {1,2,3,4,6}, N %% 32 == 0, no RMSNorm");
      epi = EPI_RESIDUAL;
    }
    if (epi < EPI_STORE || epi > EPI_BIAS) fail(Q3T_ERR_INVALID, "unknown epilogue %d", epi);
    if ((epi == EPI_RESIDUAL && !res) || (epi == EPI_BIAS && !bias)) fail(Q3T_ERR_INVALID, "missing operand");
    HIPC(hipSetDevice(e->device));
    const size_t wrows = (size_t)(epi == EPI_SWIGLU ? 2 : 1) * N;
    std::vector<void *> owned;
    auto up = [&](const void *h, size_t bytes) {
      void *d = nullptr;
      HIPC(hipMalloc(&d, bytes));
      owned.push_back(d);
      if (h) HIPC(hipMemcpy(d, h, bytes, hipMemcpyHostToDevice));
      return d;
    };
    try {
      GemmArgs g{};
      g.X = (const float *)up(X, (size_t)M * K * 4);
      g.W = (const uint16_t *)up(W, wrows * K * 2);
      g.Y = (float *)up(nullptr, (size_t)M * N * 4);
      g.M = M;
      g.N = N;
      g.K = K;
      g.ldx = K;
      g.ldy = N;
      g.ldr = N;
      if (res) g.res = (const float *)up(res, (size_t)M * N * 4);
      if (bias) g.bias = (const float *)up(bias, (size_t)N * 4);
      if (split2) {
        // T16 operands (16 rows, the rows past M zero); Y starts at zero; res_zero starts at
        // ones and must come back zero in the M x N elements the product stored.
        std::vector<float> xt((size_t)16 * K, 0.f), yt((size_t)16 * N, 0.f), zt((size_t)16 * N, 1.f);
        for (int m = 0; m < M; ++m)
          for (int k = 0; k < K; ++k) xt[t16_index(m, k)] = X[(size_t)m * K + k];
        g.X = (const float *)up(xt.data(), xt.size() * 4);
        g.x_t16 = 1;
        g.Y = (float *)up(yt.data(), yt.size() * 4);
        g.y_t16 = 1;
        g.res_zero = (float *)up(zt.data(), zt.size() * 4);
        g.split2 = 1;
        uint16_t *packed = (uint16_t *)up(nullptr, (size_t)N * K * 2);
        hip_check(launch_pack_weights(g.W, packed, N, K, nullptr), "launch_pack_weights");
        g.W = packed;
        g.w_packed = 1;
        hip_check(launch_gemm_skinny(EPI_RESIDUAL, false, g, nullptr), "launch_gemm_skinny(split2)");
        HIPC(hipMemcpy(yt.data(), g.Y, yt.size() * 4, hipMemcpyDeviceToHost));
        HIPC(hipMemcpy(zt.data(), g.res_zero, zt.size() * 4, hipMemcpyDeviceToHost));
        for (int m = 0; m < M; ++m)
          for (int n = 0; n < N; ++n) {
            Y[(size_t)m * N + n] = yt[t16_index(m, n)];
            if (zt[t16_index(m, n)] != 0.f) fail(Q3T_ERR_HIP, "split GEMM left res_zero[%d][%d] unzeroed", m, n);
          }
        for (void *p : owned) (void)hipFree(p);
        return;
      }
      if (gemm_skinny_supports(M, K, gamma != nullptr)) {  // the batched-decode kernel (fused RMSNorm)
        if (gamma) g.gamma = (const float *)up(gamma, (size_t)K * 4);
        g.eps = eps;
        // Packed weights in whole 16-column tiles: the last tile's missing rows are zeros.
        if (N % 16 && epi == EPI_SWIGLU) fail(Q3T_ERR_INVALID, "the batched-decode SwiGLU GEMM needs N %% 16 == 0");
        const size_t prows = (wrows + 15) / 16 * 16;
        uint16_t *padded = (uint16_t *)up(nullptr, prows * K * 2);
        HIPC(hipMemset(padded, 0, prows * K * 2));
        HIPC(hipMemcpy(padded, g.W, wrows * K * 2, hipMemcpyDeviceToDevice));
        uint16_t *packed = (uint16_t *)up(nullptr, prows * K * 2);
        hip_check(launch_pack_weights(padded, packed, (int)prows, K, nullptr), "launch_pack_weights");
        g.W = packed;
        g.w_packed = 1;
        hip_check(launch_gemm_skinny(epi, gamma != nullptr, g, nullptr), "launch_gemm_skinny");
      } else {
        if (gamma) {
          g.gamma = (const float *)up(gamma, (size_t)K * 4);
          float *inv = (float *)up(nullptr, (size_t)M * 4);
          hip_check(launch_row_rms(g.X, K, M, K, eps, inv, nullptr), "launch_row_rms");
          g.row_scale = inv;
        }
        hip_check(launch_gemm(epi, g, nullptr), "launch_gemm");
      }
      HIPC(hipMemcpy(Y, g.Y, (size_t)M * N * 4, hipMemcpyDeviceToHost));
    } catch (...) {
      for (void *p : owned) (void)hipFree(p);
      throw;
    }
    for (void *p : owned) (void)hipFree(p);
  });
}

int q3t_sampler_draw(q3t_engine *e, const float *logits, int32_t V, int32_t do_sample, int32_t top_k, float top_p,
                     float temperature, uint64_t seed, int32_t kind, int32_t n, int32_t *tokens) {
  return guarded([&] {
    using namespace q3t;
    if (!e || !logits || !tokens) fail(Q3T_ERR_INVALID, "null argument");
    if (V <= 0 || V > kMaxVocab) fail(Q3T_ERR_INVALID, "vocabulary %d outside 1..%d", V, kMaxVocab);
    if (n <= 0) fail(Q3T_ERR_INVALID, "draw count must be positive");
    validate_sampling(do_sample, top_k, top_p, temperature, "sampler");
    HIPC(hipSetDevice(e->device));
    int64_t scratch = 0;
    float *d_logits = dev_alloc<float>(V, scratch);
    int32_t *d_out = nullptr;
    try {
      d_out = dev_alloc<int32_t>(n, scratch);
      HIPC(hipMemcpy(d_logits, logits, (size_t)V * 4, hipMemcpyHostToDevice));
      const SamplingParams sp{do_sample ? 1 : 0, top_k, top_p, temperature};
      hip_check(launch_sample_draws(d_logits, V, sp, seed, kind, n, d_out, nullptr), "launch_sample_draws");
      HIPC(hipMemcpy(tokens, d_out, (size_t)n * 4, hipMemcpyDeviceToHost));
    } catch (...) {
      (void)hipFree(d_logits);
      if (d_out) (void)hipFree(d_out);
      throw;
    }
    (void)hipFree(d_logits);
    (void)hipFree(d_out);
  });
}

int q3t_generate_codes(q3t_engine *e, const float *prefill, int32_t P, const float *trailing, int32_t T,
                       const float *tts_pad, const q3t_generate_options *o, int32_t *codes, int32_t *frames,
                       int32_t *ended_by_eos) {
  q3t_stream *sp = nullptr;
  int rc = q3t_stream_start(e, prefill, P, trailing, T, tts_pad, o, &sp);
  if (rc != Q3T_OK) return rc;
  rc = guarded([&] {
    if (!codes || !frames || !ended_by_eos) fail(Q3T_ERR_INVALID, "null output");
  });
  int total = 0;
  q3t_chunk_info info{};
  while (rc == Q3T_OK) {
    const int chunk = o->max_frames - total;
    if (chunk <= 0) break;
    rc = q3t_stream_next_codes(sp, chunk, codes + (size_t)total * e->groups, &info);
    if (rc != Q3T_OK || info.frames == 0) break;
    total = info.total_frames;
  }
  if (rc == Q3T_OK) {
    *frames = total;
    *ended_by_eos = info.ended_by_eos;
  }
  const int rc2 = q3t_stream_destroy(sp);
  return rc != Q3T_OK ? rc : rc2;
}

}  // extern "C"
