// Codec decoder host side: weights from speech_tokenizer/model.safetensors, laid out for the
// matrix-core GEMMs, and the decode pipeline (reference src/audio/codec_hip.rs:338-1072).
//
// Layout: activations are time-major [T][C] fp32.  Every convolution is one GEMM over
// (overlapping) rows of its input:
//   * a causal convolution with K taps and dilation d reads, for output row t, the K input rows
//     t - (K-1)d, .., t as one GEMM row of K segments (GemmArgs::xseg_*), from a buffer that
//     starts with zero rows; its weight [O][C][K] is stored as [O][K][C] to match;
//   * a transposed convolution with stride s and kernel 2s (right-trimmed) computes output rows
//     t*s + p from input rows t-1 and t: one GEMM row [x(t-1), x(t)] (2C wide) against s*O
//     weight rows (phase p, channel o), so its output is directly time-major [s*T][O];
//   * pointwise convolutions and linears are plain GEMMs.
// Weights are bf16 (the synthetic checkpoint's own values; an F32 checkpoint is rounded on
// load); activations enter the matrix cores as three exact bf16 terms with fp32 accumulation.
#include "q3t_codec.h"

#include <cmath>
#include <vector>

#include "q3t_host.h"
#include "q3t_kernels.h"

namespace q3t {

namespace {

constexpr int kGroups = 16, kCodebook = 2048, kCodebookDim = 256, kProjected = 512, kPreConv = 1024;
constexpr int kHidden = 512, kLayers = 8, kHeads = 16, kQ = kHeads * 64, kInter = 1024;
constexpr int kUp = 1024, kConvNext = 4096, kInit = 1536, kFinal = 96, kPad = 64;
constexpr float kRmsEps = 1e-5f, kLnEps = 1e-6f;
struct BlockShape {
  int ci, co, s;
};
constexpr BlockShape kBlocks[4] = {{1536, 768, 8}, {768, 384, 5}, {384, 192, 4}, {192, 96, 3}};
constexpr int kDilations[3] = {1, 3, 9};

}  // namespace

struct Codec {
  std::vector<void *> allocs;
  int64_t bytes = 0;
  float *cb_first = nullptr, *cb_rest = nullptr;  // normalized codebooks [V][D], [15][V][D]
  uint16_t *w_rvq = nullptr;                      // [512][first 256 | rest 256]
  uint16_t *pre_w = nullptr;                      // [1024][3][512]
  float *pre_b = nullptr;
  uint16_t *in_w = nullptr, *out_w = nullptr;
  float *in_b = nullptr, *out_b = nullptr, *norm = nullptr;
  struct Layer {
    float *g_in, *g_post, *attn_scale, *mlp_scale;
    uint16_t *qkv, *o, *gu, *down;  // [3*1024][512], [512][1024], [gate 1024 | up 1024][512], [512][1024]
  } layers[kLayers];
  float2 *rope = nullptr;  // [kCodecMaxAttnRows][32]
  struct Up {
    uint16_t *tw;  // [2 phases x 1024][1024]
    float *tb;     // [2 x 1024]
    float *dw_w, *dw_b, *ln_g, *ln_b, *pw1_b, *pw2_b, *gamma;
    uint16_t *pw1, *pw2;
  } up[2];
  uint16_t *init_w = nullptr;  // [1536][7][1024]
  float *init_b = nullptr;
  // Snake tables (a*: exp(alpha), b*: exp(beta) + 1e-9, per channel; launch_codec_snake).
  struct Unit {
    float *a1a, *a1b, *a2a, *a2b, *b1, *b2;
    uint16_t *w1, *w2;  // [co][7][co], [co][co]
  };
  struct Block {
    float *snake_a, *snake_b;
    uint16_t *tw;  // [s x co][previous ci | current ci]
    float *tb;     // [s x co]
    Unit u[3];
  } blocks[4];
  float *fin_a = nullptr, *fin_b = nullptr, *fin_w = nullptr, *fin_bias = nullptr;  // fin_w [7][96]
  float *ws = nullptr;  // decode workspace, grown to the largest frame count seen
  size_t ws_floats = 0;
  // K-split partial sums of the GEMMs that would otherwise run as few workgroups (short
  // windows: a streaming chunk decodes ~31 frames)
  float *split_ws = nullptr;
  static constexpr int64_t kSplitFloats = (int64_t)4 << 20;
  int32_t *codes_ws = nullptr;  // staging for host codes
  size_t codes_ws_n = 0;
  float *samples_ws = nullptr;  // staging for samples copied to the host
  size_t samples_ws_n = 0;

  template <typename T>
  T *upload(const std::vector<T> &v) {
    T *d = dev_alloc<T>(v.size(), bytes);
    allocs.push_back(d);
    HIPC(hipMemcpy(d, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice));
    return d;
  }
};

Codec *codec_load(const std::string &model_dir, int64_t *device_bytes) {
  const std::string path = model_dir + "/speech_tokenizer/model.safetensors";
  if (access(path.c_str(), R_OK) != 0) return nullptr;
  SafeTensors st(path);
  auto *c = new Codec();
  try {
    auto bf16 = [&](const std::string &n, const std::vector<int64_t> &shape) {
      std::vector<uint16_t> v;
      st.append_bf16(n, shape, v);
      return v;
    };
    auto f32 = [&](const std::string &n, int64_t len) { return st.f32(n, {len}); };
    auto up_f32 = [&](const std::string &n, int64_t len) { return c->upload(f32(n, len)); };
    // A Snake's alpha / beta (prefix + "alpha" / "beta"), turned into the per-channel tables
    // launch_codec_snake reads (exp(alpha), exp(beta) + 1e-9) on the device.
    auto up_snake = [&](const std::string &prefix, int64_t len, float *&a, float *&b) {
      a = up_f32(prefix + "alpha", len);
      b = up_f32(prefix + "beta", len);
      hip_check(launch_codec_snake_prep(a, b, (int)len, nullptr), "launch_codec_snake_prep");
    };
    // [O][C][K] -> [O][K][C]
    auto taps_last_to_first = [](const std::vector<uint16_t> &w, int O, int C, int K) {
      std::vector<uint16_t> r((size_t)O * C * K);
      for (int o = 0; o < O; ++o)
        for (int ci = 0; ci < C; ++ci)
          for (int k = 0; k < K; ++k) r[((size_t)o * K + k) * C + ci] = w[((size_t)o * C + ci) * K + k];
      return r;
    };

    // RVQ (load_normalized_codebook, codec_hip.rs:2135-2154; output projections 2156-2170)
    const std::string q = "decoder.quantizer";
    auto codebook = [&](const std::string &p, std::vector<float> &out) {
      const std::vector<float> sum = st.f32(p + ".embedding_sum", {kCodebook, kCodebookDim});
      const std::vector<float> usage = st.f32(p + ".cluster_usage", {kCodebook});
      for (int v = 0; v < kCodebook; ++v) {
        const float scale = std::max(usage[v], 1e-7f);
        for (int d = 0; d < kCodebookDim; ++d) out.push_back(sum[(size_t)v * kCodebookDim + d] / scale);
      }
    };
    std::vector<float> first, rest;
    codebook(q + ".rvq_first.vq.layers.0._codebook", first);
    for (int g = 0; g < kGroups - 1; ++g) codebook(q + ".rvq_rest.vq.layers." + std::to_string(g) + "._codebook", rest);
    c->cb_first = c->upload(first);
    c->cb_rest = c->upload(rest);
    {
      const auto w1 = bf16(q + ".rvq_first.output_proj.weight", {kProjected, kCodebookDim, 1});
      const auto w2 = bf16(q + ".rvq_rest.output_proj.weight", {kProjected, kCodebookDim, 1});
      std::vector<uint16_t> w((size_t)kProjected * 2 * kCodebookDim);
      for (int o = 0; o < kProjected; ++o)
        for (int d = 0; d < kCodebookDim; ++d) {
          w[(size_t)o * 2 * kCodebookDim + d] = w1[(size_t)o * kCodebookDim + d];
          w[(size_t)o * 2 * kCodebookDim + kCodebookDim + d] = w2[(size_t)o * kCodebookDim + d];
        }
      c->w_rvq = c->upload(w);
    }
    c->pre_w = c->upload(taps_last_to_first(bf16("decoder.pre_conv.conv.weight", {kPreConv, kProjected, 3}),
                                            kPreConv, kProjected, 3));
    c->pre_b = up_f32("decoder.pre_conv.conv.bias", kPreConv);

    // pre-transformer (codec_hip.rs:380-654, 1139-1188)
    const std::string t = "decoder.pre_transformer";
    c->in_w = c->upload(bf16(t + ".input_proj.weight", {kHidden, kPreConv}));
    c->in_b = up_f32(t + ".input_proj.bias", kHidden);
    c->out_w = c->upload(bf16(t + ".output_proj.weight", {kPreConv, kHidden}));
    c->out_b = up_f32(t + ".output_proj.bias", kPreConv);
    c->norm = up_f32(t + ".norm.weight", kHidden);
    for (int i = 0; i < kLayers; ++i) {
      const std::string p = t + ".layers." + std::to_string(i);
      Codec::Layer &L = c->layers[i];
      L.g_in = up_f32(p + ".input_layernorm.weight", kHidden);
      L.g_post = up_f32(p + ".post_attention_layernorm.weight", kHidden);
      L.attn_scale = up_f32(p + ".self_attn_layer_scale.scale", kHidden);
      L.mlp_scale = up_f32(p + ".mlp_layer_scale.scale", kHidden);
      std::vector<uint16_t> qkv;
      for (const char *n : {"q_proj", "k_proj", "v_proj"}) st.append_bf16(p + ".self_attn." + n + ".weight", {kQ, kHidden}, qkv);
      L.qkv = c->upload(qkv);
      L.o = c->upload(bf16(p + ".self_attn.o_proj.weight", {kHidden, kQ}));
      std::vector<uint16_t> gu;
      st.append_bf16(p + ".mlp.gate_proj.weight", {kInter, kHidden}, gu);
      st.append_bf16(p + ".mlp.up_proj.weight", {kInter, kHidden}, gu);
      L.gu = c->upload(gu);
      L.down = c->upload(bf16(p + ".mlp.down_proj.weight", {kHidden, kInter}));
    }
    {
      std::vector<float2> rope((size_t)kCodecMaxAttnRows * 32);
      for (int r = 0; r < kCodecMaxAttnRows; ++r)
        for (int i = 0; i < 32; ++i) {
          const double ang = (double)r * std::pow(1e4, -(2.0 * i) / 64.0);
          rope[(size_t)r * 32 + i] = make_float2((float)std::cos(ang), (float)std::sin(ang));
        }
      c->rope = c->upload(rope);
    }

    // upsample stages (codec_hip.rs:702-800, 1190-1251)
    for (int i = 0; i < 2; ++i) {
      const std::string p = "decoder.upsample." + std::to_string(i);
      Codec::Up &U = c->up[i];
      const auto tw = bf16(p + ".0.conv.weight", {kUp, kUp, 2});  // [in][out][k]
      std::vector<uint16_t> w((size_t)2 * kUp * kUp);
      for (int ph = 0; ph < 2; ++ph)
        for (int o = 0; o < kUp; ++o)
          for (int ci = 0; ci < kUp; ++ci) w[((size_t)ph * kUp + o) * kUp + ci] = tw[((size_t)ci * kUp + o) * 2 + ph];
      U.tw = c->upload(w);
      std::vector<float> tb = f32(p + ".0.conv.bias", kUp);
      tb.insert(tb.end(), tb.begin(), tb.end());
      U.tb = c->upload(tb);
      U.dw_w = c->upload(st.f32(p + ".1.dwconv.conv.weight", {kUp, 1, 7}));
      U.dw_b = up_f32(p + ".1.dwconv.conv.bias", kUp);
      U.ln_g = up_f32(p + ".1.norm.weight", kUp);
      U.ln_b = up_f32(p + ".1.norm.bias", kUp);
      U.pw1 = c->upload(bf16(p + ".1.pwconv1.weight", {kConvNext, kUp}));
      U.pw1_b = up_f32(p + ".1.pwconv1.bias", kConvNext);
      U.pw2 = c->upload(bf16(p + ".1.pwconv2.weight", {kUp, kConvNext}));
      U.pw2_b = up_f32(p + ".1.pwconv2.bias", kUp);
      U.gamma = up_f32(p + ".1.gamma", kUp);
    }

    // decoder (codec_hip.rs:802-1072, 1253-1394)
    c->init_w = c->upload(taps_last_to_first(bf16("decoder.decoder.0.conv.weight", {kInit, kPreConv, 7}), kInit,
                                             kPreConv, 7));
    c->init_b = up_f32("decoder.decoder.0.conv.bias", kInit);
    for (int b = 0; b < 4; ++b) {
      const auto [ci, co, s] = kBlocks[b];
      const std::string p = "decoder.decoder." + std::to_string(b + 1) + ".block";
      Codec::Block &B = c->blocks[b];
      up_snake(p + ".0.", ci, B.snake_a, B.snake_b);
      const auto tw = bf16(p + ".1.conv.weight", {ci, co, 2 * s});  // [in][out][2s]
      std::vector<uint16_t> w((size_t)s * co * 2 * ci);
      for (int ph = 0; ph < s; ++ph)
        for (int o = 0; o < co; ++o)
          for (int k = 0; k < ci; ++k) {
            uint16_t *row = &w[((size_t)ph * co + o) * 2 * ci];
            row[k] = tw[((size_t)k * co + o) * 2 * s + ph + s];  // input row t-1
            row[ci + k] = tw[((size_t)k * co + o) * 2 * s + ph];  // input row t
          }
      B.tw = c->upload(w);
      const std::vector<float> b1 = f32(p + ".1.conv.bias", co);
      std::vector<float> tb;
      for (int ph = 0; ph < s; ++ph) tb.insert(tb.end(), b1.begin(), b1.end());
      B.tb = c->upload(tb);
      for (int u = 0; u < 3; ++u) {
        const std::string r = p + "." + std::to_string(u + 2);
        Codec::Unit &Un = B.u[u];
        up_snake(r + ".act1.", co, Un.a1a, Un.a1b);
        up_snake(r + ".act2.", co, Un.a2a, Un.a2b);
        Un.w1 = c->upload(taps_last_to_first(bf16(r + ".conv1.conv.weight", {co, co, 7}), co, co, 7));
        Un.b1 = up_f32(r + ".conv1.conv.bias", co);
        Un.w2 = c->upload(bf16(r + ".conv2.conv.weight", {co, co, 1}));
        Un.b2 = up_f32(r + ".conv2.conv.bias", co);
      }
    }
    up_snake("decoder.decoder.5.", kFinal, c->fin_a, c->fin_b);
    HIPC(hipStreamSynchronize(nullptr));
    {
      const std::vector<float> w = st.f32("decoder.decoder.6.conv.weight", {1, kFinal, 7});
      std::vector<float> r((size_t)7 * kFinal);
      for (int ci = 0; ci < kFinal; ++ci)
        for (int k = 0; k < 7; ++k) r[(size_t)k * kFinal + ci] = w[(size_t)ci * 7 + k];
      c->fin_w = c->upload(r);
    }
    c->fin_bias = up_f32("decoder.decoder.6.conv.bias", 1);
    c->split_ws = dev_alloc<float>((size_t)Codec::kSplitFloats, c->bytes);
    c->allocs.push_back(c->split_ws);
  } catch (...) {
    codec_free(c);
    throw;
  }
  *device_bytes += c->bytes;
  return c;
}

void codec_free(Codec *c) {
  if (!c) return;
  for (void *p : c->allocs) (void)hipFree(p);
  if (c->ws) (void)hipFree(c->ws);
  if (c->codes_ws) (void)hipFree(c->codes_ws);
  if (c->samples_ws) (void)hipFree(c->samples_ws);
  delete c;
}

int32_t *codec_codes_buffer(Codec &c, size_t n) {
  if (n > c.codes_ws_n) {
    if (c.codes_ws) (void)hipFree(c.codes_ws);
    c.codes_ws = nullptr;
    c.codes_ws_n = 0;
    HIPC(hipMalloc(&c.codes_ws, n * sizeof(int32_t)));
    c.codes_ws_n = n;
  }
  return c.codes_ws;
}

float *codec_samples_buffer(Codec &c, size_t n) {
  if (n > c.samples_ws_n) {
    if (c.samples_ws) (void)hipFree(c.samples_ws);
    c.samples_ws = nullptr;
    c.samples_ws_n = 0;
    HIPC(hipMalloc(&c.samples_ws, n * sizeof(float)));
    c.samples_ws_n = n;
  }
  return c.samples_ws;
}

namespace {

// Floats of the decode workspace for F frames (buffer list of codec_decode, in order).
size_t workspace_floats(size_t F) {
  const size_t pad_max = (size_t)kPad * kInit;
  const size_t big = (size_t)kCodecSamplesPerFrame * kFinal * F;  // largest T x C of the decoder blocks
  return 256 * 24 + F * 2 * kCodebookDim + (kPad + F) * kProjected + F * kPreConv + F * kHidden + F * 3 * kQ +
         F * kQ + F * kInter + F + F * kPreConv + 2 * ((kPad + 4 * F) * kUp) + 4 * F * kUp + 4 * F * kConvNext +
         big + (pad_max + (size_t)640 * 192 * F) + (pad_max + big) + 2 * big;
}

}  // namespace

void codec_decode(Codec &c, const int32_t *codes, int F, int groups, float *samples, hipStream_t s) {
  if (F <= 0 || F > kCodecMaxAttnRows) fail(Q3T_ERR_INVALID, "codec decode of %d frames (1..%d)", F, kCodecMaxAttnRows);
  if (groups != kGroups) fail(Q3T_ERR_INVALID, "codec frames have %d codes, expected %d", groups, kGroups);
  const size_t need = workspace_floats(F);
  if (need > c.ws_floats) {
    if (c.ws) (void)hipFree(c.ws);
    c.ws = nullptr;
    c.ws_floats = 0;
    HIPC(hipMalloc(&c.ws, need * sizeof(float)));
    c.ws_floats = need;
  }
  size_t off = 0;
  auto take = [&](size_t n) {
    float *p = c.ws + off;
    off += (n + 63) & ~(size_t)63;  // 256-byte alignment
    if (off > c.ws_floats) fail(Q3T_ERR_INVALID, "codec workspace plan is too small");
    return p;
  };
  auto zero_pad = [&](float *buf, int C) { HIPC(hipMemsetAsync(buf, 0, (size_t)kPad * C * sizeof(float), s)); };
  auto gemm = [&](int epi, const float *X, int ldx, int M, const uint16_t *W, int N, int K, float *Y, int ldy,
                  const float *bias, const float *res = nullptr, int ldr = 0, const float *scale = nullptr,
                  const float *row_scale = nullptr, const float *gamma = nullptr, int seg_len = 0,
                  int seg_stride = 0) {
    GemmArgs g{};
    g.X = X; g.ldx = ldx; g.W = W; g.Y = Y; g.ldy = ldy; g.M = M; g.N = N; g.K = K;
    g.bias = bias; g.res = res; g.ldr = ldr; g.scale = scale; g.row_scale = row_scale; g.gamma = gamma;
    g.xseg_len = seg_len; g.xseg_stride = seg_stride;
    g.split_ws = c.split_ws; g.split_cap = Codec::kSplitFloats;
    hip_check(launch_gemm(epi, g, s), "launch_gemm(codec)");
  };

  // 1. RVQ dequantisation and its 1x1 projections; 2. causal pre-conv, kernel 3
  float *E = take((size_t)F * 2 * kCodebookDim);
  hip_check(launch_codec_rvq(codes, F, groups, c.cb_first, c.cb_rest, kCodebook, kCodebookDim, E, s), "rvq");
  float *Qp = take((size_t)(kPad + F) * kProjected);
  zero_pad(Qp, kProjected);
  float *Q = Qp + (size_t)kPad * kProjected;
  gemm(EPI_STORE, E, 2 * kCodebookDim, F, c.w_rvq, kProjected, 2 * kCodebookDim, Q, kProjected, nullptr);
  float *PC = take((size_t)F * kPreConv);
  gemm(EPI_BIAS, Qp + (size_t)(kPad - 2) * kProjected, kProjected, F, c.pre_w, kPreConv, 3 * kProjected, PC, kPreConv,
       c.pre_b);

  // 3. pre-transformer
  float *H = take((size_t)F * kHidden);
  float *QKV = take((size_t)F * 3 * kQ);
  float *ATT = take((size_t)F * kQ);
  float *ACT = take((size_t)F * kInter);
  float *INV = take((size_t)F);
  gemm(EPI_BIAS, PC, kPreConv, F, c.in_w, kHidden, kPreConv, H, kHidden, c.in_b);
  for (int i = 0; i < kLayers; ++i) {
    const Codec::Layer &L = c.layers[i];
    hip_check(launch_row_rms(H, kHidden, F, kHidden, kRmsEps, INV, s), "row_rms");
    gemm(EPI_STORE, H, kHidden, F, L.qkv, 3 * kQ, kHidden, QKV, 3 * kQ, nullptr, nullptr, 0, nullptr, INV, L.g_in);
    hip_check(launch_codec_rope(QKV, F, 3 * kQ, kHeads, c.rope, s), "codec_rope");
    hip_check(launch_codec_attention(QKV, F, 3 * kQ, kHeads, 0.125f, ATT, kQ, s), "codec_attention");
    gemm(EPI_AFFINE_RES, ATT, kQ, F, L.o, kHidden, kQ, H, kHidden, nullptr, H, kHidden, L.attn_scale);
    hip_check(launch_row_rms(H, kHidden, F, kHidden, kRmsEps, INV, s), "row_rms");
    gemm(EPI_SWIGLU, H, kHidden, F, L.gu, kInter, kHidden, ACT, kInter, nullptr, nullptr, 0, nullptr, INV, L.g_post);
    gemm(EPI_AFFINE_RES, ACT, kInter, F, L.down, kHidden, kInter, H, kHidden, nullptr, H, kHidden, L.mlp_scale);
  }
  float *TR = take((size_t)F * kPreConv);
  hip_check(launch_row_rms(H, kHidden, F, kHidden, kRmsEps, INV, s), "row_rms");
  gemm(EPI_BIAS, H, kHidden, F, c.out_w, kPreConv, kHidden, TR, kPreConv, c.out_b, nullptr, 0, nullptr, INV, c.norm);

  // 4. two upsample stages: transposed conv (stride 2) + ConvNeXt block
  float *Up = take((size_t)(kPad + 4 * F) * kUp);
  float *Uo = take((size_t)(kPad + 4 * F) * kUp);
  float *D = take((size_t)4 * F * kUp);
  float *G = take((size_t)4 * F * kConvNext);
  const float *xin = TR;
  int T = F;
  for (int i = 0; i < 2; ++i) {
    const Codec::Up &U = c.up[i];
    zero_pad(Up, kUp);
    float *Y = Up + (size_t)kPad * kUp;
    gemm(EPI_BIAS, xin, kUp, T, U.tw, 2 * kUp, kUp, Y, 2 * kUp, U.tb);
    T *= 2;
    hip_check(launch_codec_dwconv(Up + (size_t)(kPad - 6) * kUp, U.dw_w, U.dw_b, T, kUp, 7, D, s), "dwconv");
    hip_check(launch_codec_layernorm(D, U.ln_g, U.ln_b, T, kUp, kLnEps, D, s), "layernorm");
    gemm(EPI_BIAS_GELU, D, kUp, T, U.pw1, kConvNext, kUp, G, kConvNext, U.pw1_b);
    zero_pad(Uo, kUp);
    float *O = Uo + (size_t)kPad * kUp;
    gemm(EPI_AFFINE_RES, G, kConvNext, T, U.pw2, kUp, kConvNext, O, kUp, U.pw2_b, Y, kUp, U.gamma);
    xin = O;
  }

  // 5. decoder: causal conv kernel 7, four blocks, Snake, last conv, clamp
  const size_t big = (size_t)kCodecSamplesPerFrame * kFinal * F;
  float *R = take(big);
  float *S = take((size_t)kPad * kInit + (size_t)640 * 192 * F);
  float *A = take((size_t)kPad * kInit + big);
  float *C1 = take(big);
  float *A2 = take(big);
  gemm(EPI_BIAS, Uo + (size_t)(kPad - 6) * kUp, kUp, T, c.init_w, kInit, 7 * kUp, R, kInit, c.init_b, nullptr, 0,
       nullptr, nullptr, nullptr, kUp, kUp);
  for (int b = 0; b < 4; ++b) {
    const auto [ci, co, st] = kBlocks[b];
    const Codec::Block &B = c.blocks[b];
    zero_pad(S, ci);
    hip_check(launch_codec_snake(R, B.snake_a, B.snake_b, ci, (size_t)T * ci, S + (size_t)kPad * ci, s), "snake");
    gemm(EPI_BIAS, S + (size_t)(kPad - 1) * ci, ci, T, B.tw, st * co, 2 * ci, R, st * co, B.tb, nullptr, 0, nullptr,
         nullptr, nullptr, ci, ci);
    T *= st;
    for (int u = 0; u < 3; ++u) {
      const Codec::Unit &Un = B.u[u];
      const int d = kDilations[u];
      zero_pad(A, co);
      hip_check(launch_codec_snake(R, Un.a1a, Un.a1b, co, (size_t)T * co, A + (size_t)kPad * co, s), "snake");
      gemm(EPI_BIAS, A + (size_t)(kPad - 6 * d) * co, co, T, Un.w1, co, 7 * co, C1, co, Un.b1, nullptr, 0, nullptr,
           nullptr, nullptr, co, d * co);
      hip_check(launch_codec_snake(C1, Un.a2a, Un.a2b, co, (size_t)T * co, A2, s), "snake");
      gemm(EPI_AFFINE_RES, A2, co, T, Un.w2, co, co, R, co, Un.b2, R, co, nullptr);
    }
  }
  zero_pad(A, kFinal);
  hip_check(launch_codec_snake(R, c.fin_a, c.fin_b, kFinal, (size_t)T * kFinal, A + (size_t)kPad * kFinal, s), "snake");
  hip_check(launch_codec_final(A + (size_t)(kPad - 6) * kFinal, c.fin_w, c.fin_bias, T, kFinal, 7, samples, s),
            "codec_final");
  HIPC(hipStreamSynchronize(s));
}

}  // namespace q3t
