// gfx950 kernels of the codec decoder (codec frames -> 24 kHz audio) besides its matrix-core
// GEMMs (launch_gemm): RVQ gather, Snake, depthwise causal conv, LayerNorm, RoPE, causal
// attention, and the last convolution.  Activations are time-major [T][C] fp32; a "padded"
// buffer starts with zero rows so that causal convolutions read rows before time 0 as zeros.
#include "q3t_codec.h"

#include <float.h>
#include <math.h>

namespace q3t {
namespace {

__device__ __forceinline__ float wave_sum64(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// E[t][0, D) = first[codes[t][0] mod V]; E[t][D, 2D) = sum over groups g = 1 .. G-1 (in that
// order) of rest[g-1][codes[t][g] mod V] (codec_rvq_project_f32's gathers, kernels.rs:454-495).
__global__ void k_codec_rvq(const int32_t *codes, int groups, const float *first, const float *rest, int V, int D,
                            float *E) {
  const int t = blockIdx.x;
  const int32_t *c = codes + (size_t)t * groups;
  auto wrap = [&](int32_t code) { return ((code % V) + V) % V; };
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    E[(size_t)t * 2 * D + d] = first[(size_t)wrap(c[0]) * D + d];
    float r = 0.f;
    for (int g = 1; g < groups; ++g) r += rest[((size_t)(g - 1) * V + wrap(c[g])) * D + d];
    E[(size_t)t * 2 * D + D + d] = r;
  }
}

// out[t][c] = x + sin(x e^alpha[c])^2 / (e^beta[c] + 1e-9) (codec_snake_beta_f32, kernels.rs:692-710).
// alpha := exp(alpha), beta := exp(beta) + 1e-9 (once, at load): the per-channel factors of
// every Snake launch, computed by the same device expf the per-element form used.
__global__ void k_codec_snake_prep(float *alpha, float *beta, int C) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  alpha[c] = expf(alpha[c]);
  beta[c] = expf(beta[c]) + 1.0e-9f;
}

__device__ __forceinline__ float snake1(float v, float ea, float eb) {
  const float s = sinf(v * ea);
  return v + (s * s) / eb;
}

// Four channels per thread (C % 4 == 0, 16-byte aligned rows): n4 = n / 4 quads, c4 = C / 4.
__global__ void k_codec_snake4(const float4 *x, const float4 *ea, const float4 *eb, uint32_t c4, uint32_t n4,
                               float4 *out) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n4) return;
  const uint32_t c = i % c4;
  const float4 v = x[i], a = ea[c], b = eb[c];
  out[i] = make_float4(snake1(v.x, a.x, b.x), snake1(v.y, a.y, b.y), snake1(v.z, a.z, b.z), snake1(v.w, a.w, b.w));
}

__global__ void k_codec_snake(const float *x, const float *ea, const float *eb, int C, size_t n, float *out) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int c = (int)(i % C);
  out[i] = snake1(x[i], ea[c], eb[c]);
}

// Depthwise causal conv, kernel K: out[t][c] = b[c] + sum_j xin[t + j][c] w[c][j], where xin
// row 0 is time -(K-1) (codec_depthwise_causal_conv1d_f32, kernels.rs:642-667).
__global__ void k_codec_dwconv(const float *xin, const float *w, const float *b, int T, int C, int K, float *out) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)T * C) return;
  const int c = (int)(i % C);
  const size_t t = i / C;
  float s = b[c];
  for (int j = 0; j < K; ++j) s += xin[(t + j) * C + c] * w[c * K + j];
  out[i] = s;
}

// LayerNorm of each row (codec_layernorm_f32, kernels.rs:582-612): variance E[x^2] - mean^2,
// clamped at 0.  One 256-thread workgroup per row.
__global__ void k_codec_layernorm(const float *x, const float *g, const float *b, int C, float eps, float *out) {
  const float *r = x + (size_t)blockIdx.x * C;
  float *o = out + (size_t)blockIdx.x * C;
  __shared__ float ps[4], pq[4];
  float s = 0.f, q = 0.f;
  for (int c = threadIdx.x; c < C; c += 256) {
    const float v = r[c];
    s += v;
    q += v * v;
  }
  s = wave_sum64(s);
  q = wave_sum64(q);
  if ((threadIdx.x & 63) == 0) {
    ps[threadIdx.x >> 6] = s;
    pq[threadIdx.x >> 6] = q;
  }
  __syncthreads();
  const float mean = (((ps[0] + ps[1]) + ps[2]) + ps[3]) / (float)C;
  const float var = fmaxf((((pq[0] + pq[1]) + pq[2]) + pq[3]) / (float)C - mean * mean, 0.f);
  const float inv = rsqrtf(var + eps);
  for (int c = threadIdx.x; c < C; c += 256) o[c] = (r[c] - mean) * inv * g[c] + b[c];
}

// Rotate-half RoPE in place on the q and k heads of each row of qkv ([T][ld]: q heads, then k
// heads, 64 dims each), position = row (rope_bhsd_f32, kernels.rs:40-77); cos/sin table [T][32].
__global__ void k_codec_rope(float *qkv, int T, int ld, int heads, const float2 *table) {
  const int t = blockIdx.x;
  const int h = blockIdx.y;  // 0 .. 2 * heads - 1: q heads then k heads
  const int i = threadIdx.x;  // pair 0 .. 31
  float *v = qkv + (size_t)t * ld + h * 64;
  const float2 cs = table[(size_t)t * 32 + i];
  const float a = v[i], b = v[i + 32];
  v[i] = a * cs.x - b * cs.y;
  v[i + 32] = b * cs.x + a * cs.y;
}

// Causal attention over rows 0..t for query row t and head h: scores scaled by `scale`,
// softmax, weighted sum of V (attention_scores_causal_f32 + masked softmax + apply_value,
// kernels.rs:980-1040).  qkv rows: [q heads | k heads | v heads] x 64 dims.  The four waves
// score interleaved batches of 8 keys (each score one wave sum, the same in every lane and
// whichever wave computes it); wave 0 then forms the probabilities with the scores' maximum
// and sums V in key order.
__global__ __launch_bounds__(256) void k_codec_attention(const float *qkv, int T, int ld, int heads, float scale,
                                                         float *out, int ldo) {
  extern __shared__ float sc[];  // [T]
  __shared__ float mw[4];
  const int h = blockIdx.x, t = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int Q = heads * 64;
  const float q = qkv[(size_t)t * ld + h * 64 + lane];
  float m = -FLT_MAX;
  // Key rows in batches of 8, every load of a batch issued before its reductions.
  constexpr int KB = 8;
  for (int u0 = wave * KB; u0 <= t; u0 += 4 * KB) {
    float kv[KB];
#pragma unroll
    for (int j = 0; j < KB; ++j) kv[j] = qkv[(size_t)min(u0 + j, t) * ld + Q + h * 64 + lane];
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      // A rounded product, not contracted into the butterfly's first add (which would add
      // each lane's own exact product to its partner's rounded one): every lane then holds
      // the same score.
#pragma clang fp contract(off)
      if (u0 + j > t) break;
      const float s = wave_sum64(q * kv[j]) * scale;
      if (lane == 0) sc[u0 + j] = s;
      m = fmaxf(m, s);
    }
  }
  if (lane == 0) mw[wave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(mw[0], mw[1]), fmaxf(mw[2], mw[3]));
  float l = 0.f;
  if (wave == 0) {
    for (int u = lane; u <= t; u += 64) {
      const float p = expf(sc[u] - m);
      sc[u] = p;
      l += p;
    }
    l = wave_sum64(l);
  }
  __syncthreads();
  if (wave != 0) return;
  float acc = 0.f;
  for (int u0 = 0; u0 <= t; u0 += KB) {
    float vv[KB];
#pragma unroll
    for (int j = 0; j < KB; ++j) vv[j] = qkv[(size_t)min(u0 + j, t) * ld + 2 * Q + h * 64 + lane];
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      if (u0 + j > t) break;
      acc = fmaf(sc[u0 + j], vv[j], acc);
    }
  }
  out[(size_t)t * ldo + h * 64 + lane] = acc / l;
}

// Last convolution to one channel + clamp to [-1, 1]: out[t] = clamp(b + sum_{j, c}
// xin[t + j][c] w[j][c]) with xin row 0 = time -(K-1) (kernels.rs:742-770, 903-918).  A
// workgroup stages the kFinalTile + K - 1 input rows its kFinalTile outputs read in LDS
// (unit-stride loads), rows C + 1 floats apart so that the 64 lanes of a wave, which read
// rows t .. t + 63 at one channel, fall in different banks (at a pitch of C = 96 every lane
// hit the same bank); each thread then sums its K * C products in (j, c) order.
constexpr int kFinalTile = 128, kFinalMaxC = 96, kFinalMaxK = 7;

__global__ __launch_bounds__(kFinalTile) void k_codec_final(const float *xin, const float *w, const float *b, int T,
                                                            int C, int K, float *out) {
  __shared__ float xs[(kFinalTile + kFinalMaxK - 1) * (kFinalMaxC + 1)];
  __shared__ float ws[kFinalMaxK * kFinalMaxC];
  const int t0 = blockIdx.x * kFinalTile;
  const int rows = min(kFinalTile, T - t0) + K - 1;
  const int pitch = C + 1;
  const float *src = xin + (size_t)t0 * C;
  for (int i = threadIdx.x; i < rows * C; i += kFinalTile) {
    const int r = i / C;
    xs[r * pitch + (i - r * C)] = src[i];
  }
  for (int i = threadIdx.x; i < K * C; i += kFinalTile) ws[i] = w[i];
  __syncthreads();
  const int t = t0 + (int)threadIdx.x;
  if (t >= T) return;
  float s = b[0];
  for (int j = 0; j < K; ++j) {
    const float *xr = xs + (threadIdx.x + j) * pitch;
    for (int c = 0; c < C; ++c) s += xr[c] * ws[j * C + c];
  }
  out[t] = fminf(fmaxf(s, -1.0f), 1.0f);
}

// The same for C % 4 == 0: rows C + 4 floats apart (16-byte aligned; the 16 lanes of a
// 128-bit LDS read start in distinct banks), x and w read four channels at a time, the
// products still added one by one in (j, c) order.
__global__ __launch_bounds__(kFinalTile) void k_codec_final4(const float *xin, const float *w, const float *b, int T,
                                                             int C, int K, float *out) {
  __shared__ float4 xs4[(kFinalTile + kFinalMaxK - 1) * (kFinalMaxC + 4) / 4];
  __shared__ float4 ws4[kFinalMaxK * kFinalMaxC / 4];
  const int t0 = blockIdx.x * kFinalTile;
  const int rows = min(kFinalTile, T - t0) + K - 1;
  const int c4 = C / 4, pitch4 = c4 + 1;
  const float4 *src = reinterpret_cast<const float4 *>(xin + (size_t)t0 * C);
  for (int i = threadIdx.x; i < rows * c4; i += kFinalTile) {
    const int r = i / c4;
    xs4[r * pitch4 + (i - r * c4)] = src[i];
  }
  for (int i = threadIdx.x; i < K * c4; i += kFinalTile) ws4[i] = reinterpret_cast<const float4 *>(w)[i];
  __syncthreads();
  const int t = t0 + (int)threadIdx.x;
  if (t >= T) return;
  float s = b[0];
  for (int j = 0; j < K; ++j) {
    const float4 *xr = xs4 + (threadIdx.x + j) * pitch4;
    const float4 *wr = ws4 + j * c4;
#pragma unroll 4
    for (int c = 0; c < c4; ++c) {
      const float4 x = xr[c], v = wr[c];
      s += x.x * v.x;
      s += x.y * v.y;
      s += x.z * v.z;
      s += x.w * v.w;
    }
  }
  out[t] = fminf(fmaxf(s, -1.0f), 1.0f);
}

unsigned blocks_for(size_t n, unsigned threads) { return (unsigned)((n + threads - 1) / threads); }

}  // namespace

hipError_t launch_codec_rvq(const int32_t *codes, int frames, int groups, const float *first, const float *rest,
                            int V, int D, float *E, hipStream_t s) {
  if (frames <= 0 || groups < 2 || V <= 0 || D <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_codec_rvq, dim3(frames), dim3(256), 0, s, codes, groups, first, rest, V, D, E);
  return hipGetLastError();
}

hipError_t launch_codec_snake(const float *x, const float *ea, const float *eb, int C, size_t n, float *out,
                              hipStream_t s) {
  if (C <= 0 || n % C) return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;
  auto aligned = [](const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  if (C % 4 == 0 && n / 4 < (size_t)UINT32_MAX && aligned(x) && aligned(ea) && aligned(eb) && aligned(out)) {
    const size_t n4 = n / 4;
    hipLaunchKernelGGL(k_codec_snake4, dim3(blocks_for(n4, 256)), dim3(256), 0, s, reinterpret_cast<const float4 *>(x),
                       reinterpret_cast<const float4 *>(ea), reinterpret_cast<const float4 *>(eb), (uint32_t)(C / 4),
                       (uint32_t)n4, reinterpret_cast<float4 *>(out));
  } else {
    hipLaunchKernelGGL(k_codec_snake, dim3(blocks_for(n, 256)), dim3(256), 0, s, x, ea, eb, C, n, out);
  }
  return hipGetLastError();
}

hipError_t launch_codec_snake_prep(float *alpha, float *beta, int C, hipStream_t s) {
  if (C <= 0 || !alpha || !beta) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_codec_snake_prep, dim3((C + 255) / 256), dim3(256), 0, s, alpha, beta, C);
  return hipGetLastError();
}

hipError_t launch_codec_dwconv(const float *xin, const float *w, const float *b, int T, int C, int K, float *out,
                               hipStream_t s) {
  if (T <= 0 || C <= 0 || K <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_codec_dwconv, dim3(blocks_for((size_t)T * C, 256)), dim3(256), 0, s, xin, w, b, T, C, K, out);
  return hipGetLastError();
}

hipError_t launch_codec_layernorm(const float *x, const float *g, const float *b, int T, int C, float eps, float *out,
                                  hipStream_t s) {
  if (T <= 0 || C <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_codec_layernorm, dim3(T), dim3(256), 0, s, x, g, b, C, eps, out);
  return hipGetLastError();
}

hipError_t launch_codec_rope(float *qkv, int T, int ld, int heads, const float2 *table, hipStream_t s) {
  if (T <= 0 || heads <= 0 || ld < 2 * heads * 64) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_codec_rope, dim3(T, 2 * heads), dim3(32), 0, s, qkv, T, ld, heads, table);
  return hipGetLastError();
}

hipError_t launch_codec_attention(const float *qkv, int T, int ld, int heads, float scale, float *out, int ldo,
                                  hipStream_t s) {
  if (T <= 0 || T > kCodecMaxAttnRows || heads <= 0 || ld < 3 * heads * 64 || ldo < heads * 64)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_codec_attention, dim3(heads, T), dim3(256), (size_t)T * sizeof(float), s, qkv, T, ld, heads,
                     scale, out, ldo);
  return hipGetLastError();
}

hipError_t launch_codec_final(const float *xin, const float *w, const float *b, int T, int C, int K, float *out,
                              hipStream_t s) {
  if (T <= 0 || C <= 0 || K <= 0 || C > kFinalMaxC || K > kFinalMaxK) return hipErrorInvalidValue;
  auto aligned = [](const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  if (C % 4 == 0 && aligned(xin) && aligned(w))
    hipLaunchKernelGGL(k_codec_final4, dim3(blocks_for(T, kFinalTile)), dim3(kFinalTile), 0, s, xin, w, b, T, C, K,
                       out);
  else
    hipLaunchKernelGGL(k_codec_final, dim3(blocks_for(T, kFinalTile)), dim3(kFinalTile), 0, s, xin, w, b, T, C, K, out);
  return hipGetLastError();
}

}  // namespace q3t
