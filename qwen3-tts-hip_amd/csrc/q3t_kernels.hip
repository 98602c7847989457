// gfx950 kernels for the Qwen3-TTS token loop (batch-1 decode).
//
// Numerics: bf16 weights and KV cache, fp32 activations and accumulation.  Every
// reduction has a fixed order (per-lane sequential, then a 64-lane butterfly, then a
// fixed cross-wave order), so results are bit-reproducible run to run.
#include "q3t_kernels.h"

#include <float.h>
#include <math.h>

namespace q3t {
namespace {

constexpr int kWave = 64;

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
// Round to nearest, ties to even (inputs are finite).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}

__device__ __forceinline__ bool skip_work(const SlotState *st, int mode) {
  if (mode == SKIP_NEVER) return false;
  if (st->done) return true;
  if (mode == SKIP_TALKER && st->frame + 1 >= st->max_frames) return true;
  return false;
}

__device__ __forceinline__ float dot8(uint4 w, const float *x) {
  float a = 0.f;
  a = fmaf(bf_lo(w.x), x[0], a);
  a = fmaf(bf_hi(w.x), x[1], a);
  a = fmaf(bf_lo(w.y), x[2], a);
  a = fmaf(bf_hi(w.y), x[3], a);
  a = fmaf(bf_lo(w.z), x[4], a);
  a = fmaf(bf_hi(w.z), x[5], a);
  a = fmaf(bf_lo(w.w), x[6], a);
  a = fmaf(bf_hi(w.w), x[7], a);
  return a;
}

// ---------------------------------------------------------------------------------------
// GEMV: one output row per (wave, r); each lane owns 8 consecutive K elements of every
// 512-wide chunk, so a wave streams 1 KiB of a row per 16-byte load.  All RW x KC loads
// of a wave are issued before any arithmetic.
// ---------------------------------------------------------------------------------------
template <int EPI, bool NORM, int KC, int RW>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a) {
  if (skip_work(a.st, a.skip)) return;
  constexpr int K = KC * 512;
  constexpr int NR = (EPI == EPI_SWIGLU) ? 2 * RW : RW;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int unit0 = (blockIdx.x * 4 + wave) * RW;

  uint4 w[NR][KC];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int unit = unit0 + (EPI == EPI_SWIGLU ? (r >> 1) : r);
    const int row = (EPI == EPI_SWIGLU && (r & 1)) ? a.N + unit : unit;
    const bool ok = unit < a.N;
    const uint4 *pw = reinterpret_cast<const uint4 *>(a.W + (size_t)(ok ? row : 0) * K) + lane;
#pragma unroll
    for (int c = 0; c < KC; ++c) w[r][c] = ok ? pw[c * 64] : make_uint4(0, 0, 0, 0);
  }

  float xv[KC][8];
#pragma unroll
  for (int c = 0; c < KC; ++c) {
    const float4 *px = reinterpret_cast<const float4 *>(a.x + c * 512 + lane * 8);
    const float4 p0 = px[0], p1 = px[1];
    xv[c][0] = p0.x; xv[c][1] = p0.y; xv[c][2] = p0.z; xv[c][3] = p0.w;
    xv[c][4] = p1.x; xv[c][5] = p1.y; xv[c][6] = p1.z; xv[c][7] = p1.w;
  }
  if constexpr (NORM) {
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < KC; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = fmaf(xv[c][j], xv[c][j], ss);
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      const float4 *pg = reinterpret_cast<const float4 *>(a.gamma + c * 512 + lane * 8);
      const float4 g0 = pg[0], g1 = pg[1];
      const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) xv[c][j] = (xv[c][j] * inv) * g[j];
    }
  }

  float acc[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < KC; ++c) s += dot8(w[r][c], xv[c]);
    acc[r] = wave_sum(s);
  }

#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int unit = unit0 + r;
    if (lane == r && unit < a.N) {
      if constexpr (EPI == EPI_STORE) {
        a.out[unit] = acc[r];
      } else if constexpr (EPI == EPI_RESIDUAL) {
        a.out[unit] = a.res[unit] + acc[r];
      } else if constexpr (EPI == EPI_BIAS) {
        a.out[unit] = acc[r] + a.bias[unit];
      } else {
        const float g = acc[2 * r], u = acc[2 * r + 1];
        a.out[unit] = g / (1.0f + expf(-g)) * u;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// KV-cache element access.  The cache holds fp32 (default: bit-faithful to the fp32
// reference) or bf16 (half the KV bytes; rounding happens once, at the store).
// ---------------------------------------------------------------------------------------
template <typename T>
struct KvIo;

template <>
struct KvIo<float> {
  __device__ static float store(float *p, float x) {
    *p = x;
    return x;
  }
  __device__ static void load8(const float *p, float *o) {
    const float4 a = reinterpret_cast<const float4 *>(p)[0];
    const float4 b = reinterpret_cast<const float4 *>(p)[1];
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  }
  __device__ static float2 load2(const float *p) { return *reinterpret_cast<const float2 *>(p); }
};

template <>
struct KvIo<uint16_t> {
  __device__ static float store(uint16_t *p, float x) {
    const uint16_t b = f32_to_bf16(x);
    *p = b;
    return bf16_to_f32(b);
  }
  __device__ static void load8(const uint16_t *p, float *o) {
    const uint4 w = *reinterpret_cast<const uint4 *>(p);
    o[0] = bf_lo(w.x); o[1] = bf_hi(w.x); o[2] = bf_lo(w.y); o[3] = bf_hi(w.y);
    o[4] = bf_lo(w.z); o[5] = bf_hi(w.z); o[6] = bf_lo(w.w); o[7] = bf_hi(w.w);
  }
  __device__ static float2 load2(const uint16_t *p) {
    const uint32_t w = *reinterpret_cast<const uint32_t *>(p);
    return make_float2(bf_lo(w), bf_hi(w));
  }
};

// ---------------------------------------------------------------------------------------
// Decode attention for one KV head (head_dim D = 128) and its G query heads.
//   1. q/k head RMSNorm and rotate-half RoPE at `pos` (wave per vector, lane owns the
//      RoPE pair (i, i + 64));
//   2. K and V stored at cache row `pos` (rounded to the cache type);
//   3. scores over rows 0..pos (16 lanes per row, 8 dims per lane), softmax, P.V.
// The row at `pos` is taken from LDS (the values just stored), older rows from the cache.
// ---------------------------------------------------------------------------------------
template <int D, int G, typename KVT>
__global__ __launch_bounds__(256) void k_attn_decode(AttnArgs a) {
  static_assert(D == 128, "lane layout assumes head_dim 128");
  static_assert(G >= 1 && G <= 4, "query heads per KV head");
  if (skip_work(a.st, a.skip)) return;
  const int h = blockIdx.x;
  const int pos = (a.pos_mode == POS_TALKER_FRAME) ? a.st->prefill_steps + a.st->frame : a.pos_const;
  if (pos < 0 || pos >= a.cap) return;  // host validates; never index outside the cache
  const int L = pos + 1;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int q_out = a.q_heads * D;
  const int kv_out = a.kv_heads * D;
  KVT *kcache = reinterpret_cast<KVT *>(a.kcache);
  KVT *vcache = reinterpret_cast<KVT *>(a.vcache);

  extern __shared__ float smem[];
  float *qs = smem;               // [G][D]
  float *ks = qs + G * D;         // [D]  K row at pos, as stored
  float *vs = ks + D;             // [D]  V row at pos, as stored
  float *red = vs + D;            // [4][G][D] cross-wave partials
  float *stat = red + 4 * G * D;  // [2][G][4] max / sum partials
  float *sc = stat + 8 * G;       // [G][L]

  // 1 + 2: norm, rope, cache write.  Vectors: q_0..q_{G-1}, k, v.
  const float2 cs = a.rope[(size_t)pos * (D / 2) + lane];
  for (int vec = wave; vec < G + 2; vec += 4) {
    const float *src;
    const float *gain;
    if (vec < G) {
      src = a.qkv + (h * G + vec) * D;
      gain = a.gq;
    } else if (vec == G) {
      src = a.qkv + q_out + h * D;
      gain = a.gk;
    } else {
      src = a.qkv + q_out + kv_out + h * D;
      gain = nullptr;
    }
    float x0 = src[lane], x1 = src[lane + 64];
    if (gain) {
      const float ss = wave_sum(fmaf(x0, x0, x1 * x1));
      const float inv = 1.0f / sqrtf(ss / (float)D + a.eps);
      x0 = (x0 * inv) * gain[lane];
      x1 = (x1 * inv) * gain[lane + 64];
      const float r0 = x0 * cs.x - x1 * cs.y;
      const float r1 = x1 * cs.x + x0 * cs.y;
      x0 = r0;
      x1 = r1;
    }
    if (vec < G) {
      qs[vec * D + lane] = x0;
      qs[vec * D + lane + 64] = x1;
    } else {
      KVT *cache = (vec == G) ? kcache : vcache;
      float *keep = (vec == G) ? ks : vs;
      const size_t row = ((size_t)h * a.cap + pos) * D;
      keep[lane] = KvIo<KVT>::store(cache + row + lane, x0);
      keep[lane + 64] = KvIo<KVT>::store(cache + row + lane + 64, x1);
    }
  }
  __syncthreads();

  // 3a: scores.  Lane group of 16 per row, 8 dims per lane.
  const int sub = lane & 15;
  const int grp = lane >> 4;
  const KVT *kbase = kcache + (size_t)h * a.cap * D;
  for (int base = wave * 4; base < L; base += 16) {
    const int t = base + grp;
    float kv[8];
    if (t < pos) {
      KvIo<KVT>::load8(kbase + (size_t)t * D + sub * 8, kv);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) kv[j] = (t == pos) ? ks[sub * 8 + j] : 0.f;
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) s = fmaf(qs[g * D + sub * 8 + j], kv[j], s);
      s += __shfl_xor(s, 8, 16);
      s += __shfl_xor(s, 4, 16);
      s += __shfl_xor(s, 2, 16);
      s += __shfl_xor(s, 1, 16);
      if (sub == 0 && t < L) sc[g * L + t] = s * a.scale;
    }
  }
  __syncthreads();

  // 3b: softmax statistics per query head (fixed-order block reduction).
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float m = -FLT_MAX;
    for (int t = threadIdx.x; t < L; t += 256) m = fmaxf(m, sc[g * L + t]);
    m = wave_max(m);
    if (lane == 0) stat[g * 4 + wave] = m;
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float m = fmaxf(fmaxf(stat[g * 4 + 0], stat[g * 4 + 1]), fmaxf(stat[g * 4 + 2], stat[g * 4 + 3]));
    float s = 0.f;
    for (int t = threadIdx.x; t < L; t += 256) {
      const float p = expf(sc[g * L + t] - m);
      sc[g * L + t] = p;
      s += p;
    }
    s = wave_sum(s);
    if (lane == 0) stat[4 * G + g * 4 + wave] = s;
  }
  __syncthreads();

  // 3c: P.V.  Wave w takes rows t = w (mod 4); lane owns dims 2*lane, 2*lane + 1.
  float acc[G][2];
#pragma unroll
  for (int g = 0; g < G; ++g) acc[g][0] = acc[g][1] = 0.f;
  const KVT *vbase = vcache + (size_t)h * a.cap * D;
  for (int t = wave; t < L; t += 4) {
    const float2 v = (t < pos) ? KvIo<KVT>::load2(vbase + (size_t)t * D + 2 * lane)
                               : make_float2(vs[2 * lane], vs[2 * lane + 1]);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float p = sc[g * L + t];
      acc[g][0] = fmaf(p, v.x, acc[g][0]);
      acc[g][1] = fmaf(p, v.y, acc[g][1]);
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    red[(wave * G + g) * D + 2 * lane] = acc[g][0];
    red[(wave * G + g) * D + 2 * lane + 1] = acc[g][1];
  }
  __syncthreads();
  for (int o = threadIdx.x; o < G * D; o += 256) {
    const int g = o / D, dd = o % D;
    const float sum = ((stat[4 * G + g * 4 + 0] + stat[4 * G + g * 4 + 1]) + stat[4 * G + g * 4 + 2]) +
                      stat[4 * G + g * 4 + 3];
    const float v = ((red[(0 * G + g) * D + dd] + red[(1 * G + g) * D + dd]) + red[(2 * G + g) * D + dd]) +
                    red[(3 * G + g) * D + dd];
    a.out[(h * G + g) * D + dd] = v / sum;
  }
}

// ---------------------------------------------------------------------------------------
// Token selection (one 1024-thread workgroup).
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t mulhi32(uint32_t a, uint32_t b) {
  return (uint32_t)(((uint64_t)a * b) >> 32);
}

// Philox4x32-10 (Salmon et al., SC'11).
__device__ uint4 philox4x32_10(uint4 c, uint2 k) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint32_t hi0 = mulhi32(0xD2511F53u, c.x), lo0 = 0xD2511F53u * c.x;
    const uint32_t hi1 = mulhi32(0xCD9E8D57u, c.z), lo1 = 0xCD9E8D57u * c.z;
    c = make_uint4(hi1 ^ c.y ^ k.x, lo1, hi0 ^ c.w ^ k.y, lo0);
    k.x += 0x9E3779B9u;
    k.y += 0xBB67AE85u;
  }
  return c;
}

__device__ __forceinline__ float sampler_uniform(const SlotParams &p, int step, int kind) {
  const uint4 o = philox4x32_10(make_uint4((uint32_t)step, (uint32_t)kind, 0u, 0u), make_uint2(p.seed_lo, p.seed_hi));
  return (float)(o.x >> 8) * (1.0f / 16777216.0f);
}

// Monotone map float -> uint32 (larger float, larger key).
__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

struct SelectShared {
  float lg[kMaxVocab];
  float cv[kMaxVocab];
  int ci[kMaxVocab];
  float sv[kMaxVocab];
  int si[kMaxVocab];
  uint32_t hist[256];
  float wv[16];
  int wi[16];
  int misc[8];
  uint32_t umisc[4];
};

// Argmax over lg[0..V): largest value, ties to the lowest index; -inf and NaN never win
// over a finite value.
__device__ int block_argmax(SelectShared &sh, int V) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float bv = -FLT_MAX;
  int bi = 0;
  for (int i = tid; i < V; i += 1024) {
    const float v = sh.lg[i];
    if (v > bv) {  // i increases, so ties keep the earlier index
      bv = v;
      bi = i;
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ov = __shfl_xor(bv, m, kWave);
    const int oi = __shfl_xor(bi, m, kWave);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) {
    sh.wv[wave] = bv;
    sh.wi[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    float v = sh.wv[0];
    int idx = sh.wi[0];
    for (int w = 1; w < 16; ++w)
      if (sh.wv[w] > v || (sh.wv[w] == v && sh.wi[w] < idx)) {
        v = sh.wv[w];
        idx = sh.wi[w];
      }
    sh.misc[0] = idx;
  }
  __syncthreads();
  return sh.misc[0];
}

// Top-k / temperature / top-p sampling over the finite entries of lg[0..V).
// k-th largest found by an 8-bit radix select on order keys; the candidates are ranked by
// (value desc, index asc); inverse CDF over the kept prefix with target = u * sum(p).
__device__ int block_sample(SelectShared &sh, int V, const SamplingParams &sp, float u) {
  const int tid = threadIdx.x;
  if (tid == 0) {
    sh.misc[1] = 0;  // finite count
    sh.misc[2] = 0;  // candidate count
  }
  __syncthreads();
  int local = 0;
  for (int i = tid; i < V; i += 1024) local += isfinite(sh.lg[i]) ? 1 : 0;
  if (local) atomicAdd(&sh.misc[1], local);
  __syncthreads();
  const int n_finite = sh.misc[1];
  if (n_finite == 0) return 0;
  const int k_eff = (sp.top_k > 0 && sp.top_k < n_finite) ? sp.top_k : n_finite;

  uint32_t thresh = 0;  // keys >= thresh are candidates
  if (k_eff < n_finite) {
    uint32_t prefix = 0, mask = 0;
    int remaining = k_eff;
    for (int shift = 24; shift >= 0; shift -= 8) {
      if (tid < 256) sh.hist[tid] = 0;
      __syncthreads();
      for (int i = tid; i < V; i += 1024) {
        const float v = sh.lg[i];
        if (!isfinite(v)) continue;
        const uint32_t key = order_key(v);
        if ((key & mask) == prefix) atomicAdd(&sh.hist[(key >> shift) & 255u], 1u);
      }
      __syncthreads();
      if (tid == 0) {
        int cum = 0, sel = 0;
        for (int b = 255; b >= 0; --b) {
          const int c = (int)sh.hist[b];
          if (cum + c >= remaining) {
            sel = b;
            break;
          }
          cum += c;
        }
        sh.misc[3] = remaining - cum;
        sh.umisc[0] = prefix | ((uint32_t)sel << shift);
      }
      __syncthreads();
      remaining = sh.misc[3];
      prefix = sh.umisc[0];
      mask |= 255u << shift;
      __syncthreads();
    }
    thresh = prefix;
  }

  for (int i = tid; i < V; i += 1024) {
    const float v = sh.lg[i];
    if (isfinite(v) && order_key(v) >= thresh) {
      const int p = atomicAdd(&sh.misc[2], 1);
      sh.cv[p] = v;
      sh.ci[p] = i;
    }
  }
  __syncthreads();
  const int n_cand = sh.misc[2];
  for (int c = tid; c < n_cand; c += 1024) {
    const float v = sh.cv[c];
    const int idx = sh.ci[c];
    int rank = 0;
    for (int o = 0; o < n_cand; ++o) {
      const float ov = sh.cv[o];
      rank += (ov > v || (ov == v && sh.ci[o] < idx)) ? 1 : 0;
    }
    if (rank < k_eff) {
      sh.sv[rank] = v;
      sh.si[rank] = idx;
    }
  }
  __syncthreads();
  if (tid == 0) {
    const float vmax = sh.sv[0];
    float sum = 0.f;
    for (int i = 0; i < k_eff; ++i) {
      const float p = expf((sh.sv[i] - vmax) / sp.temperature);
      sum += p;
      sh.cv[i] = sum;  // running prefix sums
    }
    int kept = k_eff;
    if (sp.top_p < 1.0f) {
      const float cut = sp.top_p * sum;
      for (int i = 0; i < k_eff; ++i)
        if (sh.cv[i] >= cut) {
          kept = i + 1;
          break;
        }
    }
    const float target = u * sh.cv[kept - 1];
    int pick = kept - 1;
    for (int i = 0; i < kept; ++i)
      if (target <= sh.cv[i]) {
        pick = i;
        break;
      }
    sh.misc[0] = sh.si[pick];
  }
  __syncthreads();
  return sh.misc[0];
}

__global__ __launch_bounds__(1024) void k_select_talker(SelectTalkerArgs a) {
  if (a.after_frame && skip_work(a.st, SKIP_TALKER)) return;
  __shared__ SelectShared sh;
  __shared__ unsigned char seen[kMaxVocab];
  __shared__ float red[16];
  const int tid = threadIdx.x;
  const SlotParams prm = *a.prm;
  const int frame = a.st->frame;
  const int step = a.after_frame ? frame + 1 : 0;
  const bool hist = a.after_frame && prm.use_history;
  if (hist) {
    for (int i = tid; i < a.V; i += 1024) seen[i] = 0;
    __syncthreads();
    for (int f = tid; f <= frame; f += 1024) {
      const int t = a.codes[(size_t)f * a.groups];
      if (t >= 0 && t < a.V) seen[t] = 1;
    }
    __syncthreads();
  }
  const float pen = prm.repetition_penalty;
  for (int i = tid; i < a.V; i += 1024) {
    float l = a.logits[i];
    if (a.trace) a.trace[(size_t)step * a.V + i] = l;
    if (hist && seen[i]) l = (l < 0.0f) ? l * pen : l / pen;
    if (i >= a.V - 1024 && i != prm.codec_eos) l = -INFINITY;
    sh.lg[i] = l;
  }
  __syncthreads();
  const int tok = prm.talker.do_sample ? block_sample(sh, a.V, prm.talker, sampler_uniform(prm, step, 0))
                                       : block_argmax(sh, a.V);
  if (tid == 0) a.st->semantic = tok;

  // CodePredictor prefix: [RMSNorm(x) * gamma ; codec_emb[tok]]
  float ss = 0.f;
  for (int i = tid; i < a.H; i += 1024) ss = fmaf(a.x[i], a.x[i], ss);
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
  for (int w = 0; w < 16; ++w) tot += red[w];
  const float inv = 1.0f / sqrtf(tot / (float)a.H + a.eps);
  for (int i = tid; i < a.H; i += 1024) {
    a.cp_prefix[i] = (a.x[i] * inv) * a.gamma[i];
    a.cp_prefix[a.H + i] = bf16_to_f32(a.codec_emb[(size_t)tok * a.H + i]);
  }
}

__global__ __launch_bounds__(1024) void k_select_cp(SelectCpArgs a) {
  if (skip_work(a.st, SKIP_DONE)) return;
  __shared__ SelectShared sh;
  const int tid = threadIdx.x;
  const SlotParams prm = *a.prm;
  const int frame = a.st->frame;
  const int semantic = a.st->semantic;
  for (int i = tid; i < a.Vc; i += 1024) {
    const float l = a.logits[i];
    if (a.trace) a.trace[((size_t)frame * (a.groups - 1) + a.group) * a.Vc + i] = l;
    sh.lg[i] = l;
  }
  __syncthreads();
  const int tok = prm.cp.do_sample ? block_sample(sh, a.Vc, prm.cp, sampler_uniform(prm, frame, 1 + a.group))
                                   : block_argmax(sh, a.Vc);
  if (tid == 0) {
    a.codes[(size_t)frame * a.groups + 1 + a.group] = tok;
    if (a.group == 0) a.codes[(size_t)frame * a.groups] = semantic;
  }
  const bool last = a.group == a.groups - 2;
  const int trow = min(frame, a.st->trailing_rows);
  for (int i = tid; i < a.Ht; i += 1024) {
    const float e = bf16_to_f32(a.emb[(size_t)tok * a.Ht + i]);
    a.cur[i] = e;
    const float s = (a.group == 0) ? e : a.emb_sum[i] + e;
    a.emb_sum[i] = s;
    if (last)
      a.talker_in[i] = (bf16_to_f32(a.codec_emb[(size_t)semantic * a.Ht + i]) + s) + a.trailing[(size_t)trow * a.Ht + i];
  }
}

// Standalone draws from one logit row: block b draws with Philox counter (b, kind, 0, 0).
__global__ __launch_bounds__(1024) void k_sample_draws(const float *logits, int V, SamplingParams sp, uint32_t seed_lo,
                                                       uint32_t seed_hi, int kind, int32_t *out) {
  __shared__ SelectShared sh;
  for (int i = threadIdx.x; i < V; i += 1024) sh.lg[i] = logits[i];
  __syncthreads();
  SlotParams p{};
  p.seed_lo = seed_lo;
  p.seed_hi = seed_hi;
  const int tok = sp.do_sample ? block_sample(sh, V, sp, sampler_uniform(p, blockIdx.x, kind)) : block_argmax(sh, V);
  if (threadIdx.x == 0) out[blockIdx.x] = tok;
}

// Ends a frame (advance = 1) or checks the token drawn after the prefill (advance = 0).
__global__ void k_frame_end(SlotState *st, const SlotParams *prm, int advance) {
  if (threadIdx.x != 0 || st->done) return;
  const int f = st->frame + advance;
  st->frame = f;
  if (st->semantic == prm->codec_eos)
    st->done = 1;
  else if (f >= st->max_frames)
    st->done = 2;
}

}  // namespace

// ---------------------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------------------
bool gemv_supports_k(int K) {
  if (K <= 0 || K % 512) return false;
  const int c = K / 512;
  return c == 1 || c == 2 || c == 3 || c == 4 || c == 6 || c == 8 || c == 12;
}

template <int EPI, bool NORM, int KC, int RW>
static void gemv_launch(const GemvArgs &a, hipStream_t s) {
  const int units = 4 * RW;
  hipLaunchKernelGGL((k_gemv<EPI, NORM, KC, RW>), dim3((a.N + units - 1) / units), dim3(256), 0, s, a);
}

template <int EPI, bool NORM, int KC>
static hipError_t gemv_rw(const GemvArgs &a, hipStream_t s) {
  // Rows per wave: as many as keep >= 256 workgroups, with at most 16 outstanding
  // 16-byte weight loads per lane.
  constexpr int per_unit = (EPI == EPI_SWIGLU) ? 2 : 1;
  constexpr bool can4 = 4 * per_unit * KC <= 16;
  constexpr bool can2 = 2 * per_unit * KC <= 16;
  if (can4 && a.N >= 256 * 4 * 4) {
    if constexpr (can4) gemv_launch<EPI, NORM, KC, 4>(a, s);
  } else if (can2 && a.N >= 256 * 4 * 2) {
    if constexpr (can2) gemv_launch<EPI, NORM, KC, 2>(a, s);
  } else {
    gemv_launch<EPI, NORM, KC, 1>(a, s);
  }
  return hipGetLastError();
}

template <int EPI, bool NORM>
static hipError_t gemv_k(const GemvArgs &a, hipStream_t s) {
  switch (a.K / 512) {
    case 1: return gemv_rw<EPI, NORM, 1>(a, s);
    case 2: return gemv_rw<EPI, NORM, 2>(a, s);
    case 3: return gemv_rw<EPI, NORM, 3>(a, s);
    case 4: return gemv_rw<EPI, NORM, 4>(a, s);
    case 6: return gemv_rw<EPI, NORM, 6>(a, s);
    case 8: return gemv_rw<EPI, NORM, 8>(a, s);
    case 12: return gemv_rw<EPI, NORM, 12>(a, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_gemv(int epi, bool norm, const GemvArgs &a, hipStream_t s) {
  if (!gemv_supports_k(a.K) || a.N <= 0) return hipErrorInvalidValue;
  switch (epi) {
    case EPI_STORE: return norm ? gemv_k<EPI_STORE, true>(a, s) : gemv_k<EPI_STORE, false>(a, s);
    case EPI_RESIDUAL: return norm ? hipErrorInvalidValue : gemv_k<EPI_RESIDUAL, false>(a, s);
    case EPI_SWIGLU: return norm ? gemv_k<EPI_SWIGLU, true>(a, s) : hipErrorInvalidValue;
    case EPI_BIAS: return norm ? hipErrorInvalidValue : gemv_k<EPI_BIAS, false>(a, s);
  }
  return hipErrorInvalidValue;
}

static size_t attn_lds_bytes(int G, int L) {
  return sizeof(float) * ((size_t)G * 128 + 2 * 128 + 4 * (size_t)G * 128 + 8 * (size_t)G + (size_t)G * L);
}

int attn_max_cache_steps(int q_heads, int kv_heads) {
  const int G = q_heads / kv_heads;
  const size_t fixed = attn_lds_bytes(G, 0);
  const size_t budget = 128 * 1024;
  return fixed >= budget ? 0 : (int)((budget - fixed) / (sizeof(float) * G));
}

hipError_t launch_attn_decode(const AttnArgs &a, int head_dim, hipStream_t s) {
  if (head_dim != 128 || a.kv_heads <= 0 || a.q_heads % a.kv_heads || a.q_heads / a.kv_heads > 4 ||
      a.q_heads / a.kv_heads == 3)
    return hipErrorInvalidValue;
  if (a.cap > attn_max_cache_steps(a.q_heads, a.kv_heads)) return hipErrorInvalidValue;
  const int G = a.q_heads / a.kv_heads;
  // LDS sized for the longest row range this cache can hold.
  const size_t lds = attn_lds_bytes(G, a.cap);
  const dim3 grid(a.kv_heads), block(256);
  if (a.kv_bf16) {
    switch (G) {
      case 1: hipLaunchKernelGGL((k_attn_decode<128, 1, uint16_t>), grid, block, lds, s, a); break;
      case 2: hipLaunchKernelGGL((k_attn_decode<128, 2, uint16_t>), grid, block, lds, s, a); break;
      case 4: hipLaunchKernelGGL((k_attn_decode<128, 4, uint16_t>), grid, block, lds, s, a); break;
      default: return hipErrorInvalidValue;
    }
  } else {
    switch (G) {
      case 1: hipLaunchKernelGGL((k_attn_decode<128, 1, float>), grid, block, lds, s, a); break;
      case 2: hipLaunchKernelGGL((k_attn_decode<128, 2, float>), grid, block, lds, s, a); break;
      case 4: hipLaunchKernelGGL((k_attn_decode<128, 4, float>), grid, block, lds, s, a); break;
      default: return hipErrorInvalidValue;
    }
  }
  return hipGetLastError();
}

hipError_t launch_select_talker(const SelectTalkerArgs &a, hipStream_t s) {
  if (a.V > kMaxVocab || a.V < 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_select_talker, dim3(1), dim3(1024), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_select_cp(const SelectCpArgs &a, hipStream_t s) {
  if (a.Vc > kMaxVocab) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_select_cp, dim3(1), dim3(1024), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_sample_draws(const float *logits, int V, const SamplingParams &sp, uint64_t seed, int kind, int n,
                               int32_t *out, hipStream_t s) {
  if (V <= 0 || V > kMaxVocab || n <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_sample_draws, dim3(n), dim3(1024), 0, s, logits, V, sp, (uint32_t)(seed & 0xffffffffu),
                     (uint32_t)(seed >> 32), kind, out);
  return hipGetLastError();
}

hipError_t launch_frame_end(SlotState *st, const SlotParams *prm, int advance, hipStream_t s) {
  hipLaunchKernelGGL(k_frame_end, dim3(1), dim3(64), 0, s, st, prm, advance);
  return hipGetLastError();
}

}  // namespace q3t
