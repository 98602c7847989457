// Codec decoder (speech tokenizer decoder): codec frames [F][16] -> F * 1920 samples at 24 kHz,
// the reference's HipCodecInitial (src/audio/codec_hip.rs) on the gfx950 matrix cores.
#pragma once

#include <string>

#include "q3t_device.h"

namespace q3t {

constexpr int kCodecSamplesPerFrame = 1920;  // 2 x 2 (upsampling) x 8 x 5 x 4 x 3 (decoder blocks)
constexpr int kCodecMaxAttnRows = 8192;      // frames one pre-transformer attention covers

struct Codec;

// Loads <model_dir>/speech_tokenizer/model.safetensors (codec_hip.rs:214-336); returns null
// when the file does not exist.  Adds the device bytes it holds to *device_bytes.
Codec *codec_load(const std::string &model_dir, int64_t *device_bytes);
void codec_free(Codec *c);
// Decodes `frames` frames of device codes (frame-major, `groups` per frame) into frames * 1920
// samples (device pointer) on stream s, synchronously.  The workspace grows to the largest
// frame count seen.
void codec_decode(Codec &c, const int32_t *codes, int frames, int groups, float *samples, hipStream_t s);
// Device staging buffers owned by the codec (grown on demand): n codes, n samples.
int32_t *codec_codes_buffer(Codec &c, size_t n);
float *codec_samples_buffer(Codec &c, size_t n);

// Kernels (q3t_codec.hip).
hipError_t launch_codec_rvq(const int32_t *codes, int frames, int groups, const float *first, const float *rest,
                            int V, int D, float *E, hipStream_t s);
// Snake over [n / C][C]: out = x + sin(x * ea[c])^2 / eb[c], with the per-channel tables
// ea = exp(alpha), eb = exp(beta) + 1e-9 that launch_codec_snake_prep makes in place from the
// checkpoint's alpha / beta (snake_beta_f32, kernels.rs).
hipError_t launch_codec_snake(const float *x, const float *ea, const float *eb, int C, size_t n, float *out,
                              hipStream_t s);
hipError_t launch_codec_snake_prep(float *alpha, float *beta, int C, hipStream_t s);
hipError_t launch_codec_dwconv(const float *xin, const float *w, const float *b, int T, int C, int K, float *out,
                               hipStream_t s);
hipError_t launch_codec_layernorm(const float *x, const float *g, const float *b, int T, int C, float eps, float *out,
                                  hipStream_t s);
hipError_t launch_codec_rope(float *qkv, int T, int ld, int heads, const float2 *table, hipStream_t s);
hipError_t launch_codec_attention(const float *qkv, int T, int ld, int heads, float scale, float *out, int ldo,
                                  hipStream_t s);
hipError_t launch_codec_final(const float *xin, const float *w, const float *b, int T, int C, int K, float *out,
                              hipStream_t s);

}  // namespace q3t
