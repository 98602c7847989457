// gfx950 kernels for the Qwen3-TTS token loop (batch-1 decode).
//
// Numerics: bf16 weights and KV cache, fp32 activations and accumulation.  Every
// reduction has a fixed order (per-lane sequential, then a 64-lane butterfly, then a
// fixed cross-wave order), so results are bit-reproducible run to run.
#include "q3t_kernels.h"

#include <float.h>
#include <math.h>

#include <algorithm>
#include <mutex>

#include <hip/hip_ext.h>

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

// Cross-lane reductions on DPP (data-parallel primitives: VALU lane permutes, no LDS round
// trip).  Each step adds a permuted copy: quad_perm [1,0,3,2] and [2,3,0,1] (quads),
// row_half_mirror and row_mirror (rows of 16), then row_bcast:15 / row_bcast:31 fold the
// four rows into lane 63.  The order is fixed, so results are deterministic.
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ float dpp_f(float v, float fill) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, fill), __builtin_bit_cast(int, v),
                                                               CTRL, ROWS, 0xf, false));
}

// Sum over each row of 16 lanes, in every lane of the row.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<0xB1>(v, 0.f);
  v += dpp_f<0x4E>(v, 0.f);
  v += dpp_f<0x141>(v, 0.f);
  v += dpp_f<0x140>(v, 0.f);
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  v += dpp_f<0x142, 0xa>(v, 0.f);
  v += dpp_f<0x143, 0xc>(v, 0.f);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v, v));
  v = fmaxf(v, dpp_f<0x4E>(v, v));
  v = fmaxf(v, dpp_f<0x141>(v, v));
  v = fmaxf(v, dpp_f<0x140>(v, v));
  v = fmaxf(v, dpp_f<0x142, 0xa>(v, v));
  v = fmaxf(v, dpp_f<0x143, 0xc>(v, v));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Argmax as a 64-bit maximum: order_key(v, i) = (v's bits mapped to an unsigned order) << 32 |
// (2^32 - 1 - i), so the largest key is the largest value and, among equal values, the lowest
// index.  Values that block_argmax never picks (NaN, -inf, -FLT_MAX) map to 0, which is also
// the empty key; key_token(0) = 0, block_argmax's answer when nothing beats -FLT_MAX.
__device__ __forceinline__ uint64_t order_key(float v, int idx) {
  if (!(v > -FLT_MAX)) return 0;
  uint32_t u = __float_as_uint(v);
  if (u == 0x80000000u) u = 0;  // -0 ties with +0
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | (uint64_t)(0xffffffffu - (uint32_t)idx);
}

__device__ __forceinline__ int key_token(uint64_t key) {
  return key ? (int)(0xffffffffu - (uint32_t)(key & 0xffffffffu)) : 0;
}

template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  const int lo = (int)(uint32_t)v, hi = (int)(uint32_t)(v >> 32);
  const uint32_t plo = (uint32_t)__builtin_amdgcn_update_dpp(lo, lo, CTRL, ROWS, 0xf, false);
  const uint32_t phi = (uint32_t)__builtin_amdgcn_update_dpp(hi, hi, CTRL, ROWS, 0xf, false);
  return ((uint64_t)phi << 32) | plo;
}

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// The value of lane (lane ^ J) on the VALU instead of an LDS permute (ds_bpermute): quad
// permutes for J = 1, 2; row shifts by J, one chosen per lane, for J = 4, 8 (the partner is
// always inside the row of 16); gfx950's row swaps for J = 16 (v_permlane16_swap: lane l gets
// lanes l & ~16 and l | 16) and J = 32 (v_permlane32_swap: lanes l & ~32 and l | 32).
template <int J>
__device__ __forceinline__ uint32_t lane_xor_u32(uint32_t x) {
  const uint32_t lane = threadIdx.x & 63;
  if constexpr (J == 1) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0xB1, 0xf, 0xf, false);
  } else if constexpr (J == 2) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xf, 0xf, false);
  } else if constexpr (J == 4 || J == 8) {
    const uint32_t up = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x100 + J, 0xf, 0xf, false);  // lane + J
    const uint32_t dn = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x110 + J, 0xf, 0xf, false);  // lane - J
    return (lane & J) ? dn : up;
  } else if constexpr (J == 16) {
    const auto q = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return (lane & 16) ? q[0] : q[1];
  } else {
    static_assert(J == 32, "lane distance");
    const auto q = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return (lane & 32) ? q[0] : q[1];
  }
}

template <int J>
__device__ __forceinline__ uint64_t lane_xor_u64(uint64_t x) {
  return ((uint64_t)lane_xor_u32<J>((uint32_t)(x >> 32)) << 32) | lane_xor_u32<J>((uint32_t)x);
}

// x + (x of lane ^ 16) and x + (x of lane ^ 32): the same sum in both lanes of each pair.
__device__ __forceinline__ float pair16_sum(float x) {
  const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}
__device__ __forceinline__ float pair32_sum(float x) {
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// Largest key of the wave, in every lane (same permutation sequence as wave_max).
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  v = umax64(v, dpp_u64<0xB1>(v));
  v = umax64(v, dpp_u64<0x4E>(v));
  v = umax64(v, dpp_u64<0x141>(v));
  v = umax64(v, dpp_u64<0x140>(v));
  v = umax64(v, dpp_u64<0x142, 0xa>(v));
  v = umax64(v, dpp_u64<0x143, 0xc>(v));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 63);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 63);
  return ((uint64_t)hi << 32) | lo;
}

// Whether a kernel skips an ended stream's work: SKIP_DONE once it has ended, SKIP_TALKER
// also for the Talker step after its last frame.
__device__ __forceinline__ bool skip_state(const SlotState &sv, int mode) {
  if (mode == SKIP_NEVER) return false;
  if (sv.done) return true;
  if (mode == SKIP_TALKER && sv.frame + 1 >= sv.max_frames) return true;
  return false;
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
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ uint4 load_w(const u32x4 *p) {
  u32x4 v;
  if constexpr (NT)
    v = __builtin_nontemporal_load(p);
  else
    v = *p;
  return make_uint4(v.x, v.y, v.z, v.w);
}

// NT = streaming (non-temporal) weight loads: used for the Talker, whose weights are read once
// per frame, so that they do not displace the CodePredictor weights that every frame rereads
// 15 times from the last-level cache.
// The partials one thread merges (8 output elements at `base`, every chunk slot), loaded
// without waiting for the stream state: indices are clamped to the workspace, not to the
// chunks in use.
struct MergeRegs {
  float mv[kAttnGemvMergeChunks], lv[kAttnGemvMergeChunks], av[kAttnGemvMergeChunks][8];
};

__device__ __forceinline__ void merge_load(const GemvArgs &a, int base, MergeRegs &r) {
  constexpr int D = 128;
  const int G = a.attn_q_heads / a.attn_kv_heads;
  const int hq = base / D, d0 = base % D;
  const int h = hq / G, g = hq % G;
  const float *p0 = a.attn_part + (((size_t)h * a.attn_part_chunks) * G + g) * (D + 2);
  const size_t stride = (size_t)G * (D + 2);
#pragma unroll
  for (int c = 0; c < kAttnGemvMergeChunks; ++c) {
    const float *pc = p0 + min(c, a.attn_part_chunks - 1) * stride;
    r.mv[c] = pc[0];
    r.lv[c] = pc[1];
#pragma unroll
    for (int j = 0; j < 8; ++j) r.av[c][j] = pc[2 + d0 + j];  // records are 130 floats: not 16-B aligned
  }
}

// The max and the weighted sums over the chunks in use, in chunk order, into xs[base ..].
__device__ __forceinline__ void merge_finish(const GemvArgs &a, int base, const MergeRegs &r, float *xs) {
  const int pos = (a.attn_pos_mode == POS_TALKER_FRAME) ? a.st->prefill_steps + a.st->frame : a.attn_pos_const;
  const int nchunks = (pos + a.attn_chunk) / a.attn_chunk;  // ceil((pos + 1) / chunk)
  const float *mv = r.mv, *lv = r.lv;
  const float(*av)[8] = r.av;
  {
    float M = -FLT_MAX;
#pragma unroll
    for (int c = 0; c < kAttnGemvMergeChunks; ++c)
      if (c < nchunks) M = fmaxf(M, mv[c]);
    float den = 0.f, num[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < kAttnGemvMergeChunks; ++c)
      if (c < nchunks) {
        const float w = expf(mv[c] - M);
        den = fmaf(w, lv[c], den);
#pragma unroll
        for (int j = 0; j < 8; ++j) num[j] = fmaf(w, av[c][j], num[j]);
      }
#pragma unroll
    for (int j = 0; j < 8; ++j) xs[base + j] = num[j] / den;
  }
}

__device__ void merge_attention(const GemvArgs &a, float *xs);

// Most per-head partials a GEMV input sums (GemvArgs::parts): the KV heads of a layer.
constexpr int kMaxParts = 8;

// The input vector of k_gemv: IN_X = x, loaded whole by every lane (the two-row form);
// IN_XLDS = x loaded once per workgroup into LDS (the one-row form); IN_ATTN = the merge of
// attention partials (see merge_attention); IN_PARTS = x plus the per-head partials of the
// fused attention + O projection (GemvArgs::parts), summed through LDS; IN_TALKER = the next
// Talker input from the last CodePredictor group's hand-off (GemvArgs::tin), assembled
// through LDS.  With the RMSNorm prologue the LDS forms take the gain through LDS too.
constexpr int IN_X = 0, IN_ATTN = 1, IN_PARTS = 2, IN_TALKER = 3, IN_XLDS = 4;

// Waves per workgroup of the IN_PARTS form: every workgroup sums the partials into LDS, so
// it runs the launch's waves in fewer, larger workgroups (the partials are read from L2 once
// per workgroup).
constexpr int kPartsWaves = 12;
// Waves per workgroup of the IN_XLDS form for K >= 512 * kXldsWideKC (the 1.7B Talker's down
// projection, K = 6144): every workgroup loads the whole input (24 KB) into LDS, so 8-wave
// workgroups halve the input bytes a launch pulls from L2.  Smaller K (inputs of 8-12 KB)
// keeps 4 waves, which measured as fast or faster there.
constexpr int kXldsWideKC = 12;
constexpr int kXldsWideWaves = 8;
template <int IN, int KC>
constexpr int gemv_waves() {
  return IN == IN_PARTS ? kPartsWaves : (IN == IN_XLDS && KC >= kXldsWideKC) ? kXldsWideWaves : 4;
}

// MR = input rows (1, or 2: row 1 at x + ldx_r, res + ldr_r, out + ldo_r) against the same
// weight loads.
// HO = greedy token hand-off producer (GemvArgs::keys_out).
template <int EPI, bool NORM, int KC, int RW, bool NT, int IN = IN_X, int MR = 1, bool HO = false>
__global__ __launch_bounds__((64 * gemv_waves<IN, KC>())) void k_gemv(GemvArgs a) {
  constexpr bool ATTN = IN == IN_ATTN;
  constexpr bool PARTS = IN == IN_PARTS;
  constexpr bool TIN = IN == IN_TALKER;
  // IN_XLDS: x (and the norm gain) loaded once per workgroup, one float4 per thread and pass,
  // and read by every wave from LDS: each lane otherwise loads the whole vector (2 KC loads,
  // and 2 KC more for the gain), more load instructions than its weight rows take.
  constexpr bool XLDS = IN == IN_XLDS;
  static_assert(!XLDS || MR == 1, "x through LDS: one row");
  constexpr int WPB = gemv_waves<IN, KC>();
  constexpr int NTH = 64 * WPB;
  static_assert(!ATTN || MR == 1, "the attention merge feeds one row");
  static_assert(!PARTS || (KC == 1 || KC == 2), "the partial sum feeds rows of K <= 1024");
  static_assert(!HO || (MR == 1 && (IN == IN_X || IN == IN_XLDS) && EPI == EPI_STORE),
                "the hand-off producer stores one row");
  static_assert(!TIN || (MR == 1 && EPI == EPI_STORE && NORM && (KC == 1 || KC == 2 || KC == 4)),
                "the Talker input feeds one normed row of K 512, 1024 or 2048");
  constexpr int K = KC * 512;
  constexpr int NR = (EPI == EPI_SWIGLU) ? 2 * RW : RW;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int unit0 = (blockIdx.x * WPB + wave) * RW;
  __shared__ float xs[PARTS ? MR : 1][(ATTN || PARTS || TIN || XLDS) ? K : 1];
  // The norm gain goes through LDS with the input wherever the input does (GLDS).
  constexpr bool GLDS = NORM && (XLDS || PARTS || TIN);
  __shared__ float gsh[GLDS ? K : 1];
  __shared__ uint64_t wkeys[HO ? 4 : 1];
  // IN_PARTS: thread t sums elements 4t .. 4t+3 of x and of every part (K <= 1024), for each
  // input row m (x + m * ldx_r, parts + m * ldp_r).
  constexpr int PR = PARTS ? MR : 1;
  float4 px_[PR], pp_[PARTS ? kMaxParts : 1][PR];
  if constexpr (PARTS) {
    const int i = 4 * (int)threadIdx.x;
    if (i < K) {  // threads past K / 4 (whole waves) have nothing to sum
#pragma unroll
      for (int m = 0; m < PR; ++m) {
        px_[m] = *reinterpret_cast<const float4 *>(a.x + m * a.ldx_r + i);
#pragma unroll
        for (int p = 0; p < kMaxParts; ++p)
          pp_[p][m] = *reinterpret_cast<const float4 *>(a.parts + (size_t)m * a.ldp_r +
                                                        (size_t)min(p, a.n_parts - 1) * a.ld_parts + i);
      }
    }
  }

  // IN_TALKER: thread t covers elements 4t .. 4t+3 and 1024 + 4t .. (K <= 2048); the hand-off
  // keys (four per lane, every wave reduces them all) and the running sum are loaded first.
  uint64_t tkey[TIN ? 4 : 1];
  float4 tsum[TIN ? 2 : 1];
  if constexpr (TIN) {
#pragma unroll
    for (int j = 0; j < 4; ++j) tkey[j] = a.tin.keys[min(lane + 64 * j, a.tin.n_keys - 1)];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int i = 4 * (int)threadIdx.x + 1024 * j;
      tsum[j] = i < K ? *reinterpret_cast<const float4 *>(a.tin.sum + i) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }

  // Load order: activations (and the norm gain), then every weight row of this wave, then
  // nothing else until the arithmetic.  The norm then only waits for the small activation
  // loads while the whole launch's weights are in flight (one DRAM round trip per launch).
  float xv[MR][KC][8];
  float gv[NORM ? KC : 1][8];
  // Attention input over K <= 2048 (one 8-element slice per thread): its partials are loaded
  // first, ahead of the weights and of the stream-state check.
  constexpr bool ATTN_EARLY = ATTN && K <= 256 * 8;
  MergeRegs mregs;
  if constexpr (ATTN_EARLY) {
    if (threadIdx.x * 8 < K) merge_load(a, threadIdx.x * 8, mregs);
  }
  constexpr int XQ = XLDS ? (K + 4 * NTH - 1) / (4 * NTH) : 1;
  float4 xq[XQ];
  if constexpr (XLDS) {
#pragma unroll
    for (int j = 0; j < XQ; ++j) {
      const int i = 4 * (int)threadIdx.x + 4 * NTH * j;
      xq[j] = i < K ? *reinterpret_cast<const float4 *>(a.x + i) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  constexpr int GQ = GLDS ? (K + 4 * NTH - 1) / (4 * NTH) : 1;
  float4 gq[GQ];
  if constexpr (GLDS) {
#pragma unroll
    for (int j = 0; j < GQ; ++j) {
      const int i = 4 * (int)threadIdx.x + 4 * NTH * j;
      gq[j] = i < K ? *reinterpret_cast<const float4 *>(a.gamma + i) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  // the gain's LDS stores (before the input's barrier) and the lane's reads (after it)
  auto gain_store = [&] {
    if constexpr (GLDS) {
#pragma unroll
      for (int j = 0; j < GQ; ++j) {
        const int i = 4 * (int)threadIdx.x + 4 * NTH * j;
        if (i < K) *reinterpret_cast<float4 *>(&gsh[i]) = gq[j];
      }
    }
  };
  auto gain_read = [&] {
    if constexpr (GLDS) {
#pragma unroll
      for (int c = 0; c < KC; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) gv[c][j] = gsh[c * 512 + lane * 8 + j];
    }
  };
#pragma unroll
  for (int c = 0; c < KC; ++c) {
    if constexpr (ATTN || PARTS || TIN || XLDS) break;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float4 *px = reinterpret_cast<const float4 *>(a.x + m * a.ldx_r + c * 512 + lane * 8);
      const float4 p0 = px[0], p1 = px[1];
      xv[m][c][0] = p0.x; xv[m][c][1] = p0.y; xv[m][c][2] = p0.z; xv[m][c][3] = p0.w;
      xv[m][c][4] = p1.x; xv[m][c][5] = p1.y; xv[m][c][6] = p1.z; xv[m][c][7] = p1.w;
    }
  }
  if constexpr (NORM && !GLDS) {
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      const float4 *pg = reinterpret_cast<const float4 *>(a.gamma + c * 512 + lane * 8);
      const float4 g0 = pg[0], g1 = pg[1];
      gv[c][0] = g0.x; gv[c][1] = g0.y; gv[c][2] = g0.z; gv[c][3] = g0.w;
      gv[c][4] = g1.x; gv[c][5] = g1.y; gv[c][6] = g1.z; gv[c][7] = g1.w;
    }
  }
  // The epilogue operand of this lane's output row (lane r stores row unit0 + r), loaded
  // before the weights so that the store waits on nothing.
  float eadd[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    eadd[m] = 0.f;
    if constexpr (EPI == EPI_RESIDUAL) eadd[m] = a.res[m * a.ldr_r + min(unit0 + min(lane, RW - 1), a.N - 1)];
    if constexpr (EPI == EPI_BIAS) eadd[m] = a.bias[min(unit0 + min(lane, RW - 1), a.N - 1)];
  }
  // Keep the activation loads ahead of the weight loads in issue order: loads complete in
  // order, so the norm can then start before the weights have arrived.
  __builtin_amdgcn_sched_barrier(0);
  // Rows past the end (a partial last workgroup) load the last row instead of branching;
  // their results are never stored.
  uint4 w[NR][KC];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int unit = min(unit0 + (EPI == EPI_SWIGLU ? (r >> 1) : r), a.N - 1);
    const int row = (EPI == EPI_SWIGLU && (r & 1)) ? a.N + unit : unit;
    const u32x4 *pw = reinterpret_cast<const u32x4 *>(a.W + (size_t)row * K) + lane;
#pragma unroll
    for (int c = 0; c < KC; ++c) w[r][c] = load_w<NT>(pw + c * 64);
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (TIN) {
    // The last group's token and the Talker input (the selection kernel's arithmetic, in its
    // order), stored by workgroup 0 unless the stream has ended; then the launch's own skip
    // check (after the last frame the Talker step does not run, the stores above do).
    if (a.st->done) return;
    const int tok = key_token(wave_max_u64(umax64(umax64(tkey[0], tkey[1]), umax64(tkey[2], tkey[3]))));
    const int frame = a.st->frame, sem = a.st->semantic;
    const int trow = min(frame, a.st->trailing_rows);
    float4 te[2], tc[2], tt[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int i = 4 * (int)threadIdx.x + 1024 * j;
      if (i < K) {
        const uint2 we = *reinterpret_cast<const uint2 *>(a.tin.emb + (size_t)tok * K + i);
        const uint2 wc = *reinterpret_cast<const uint2 *>(a.tin_codec_emb + (size_t)sem * K + i);
        te[j] = make_float4(bf_lo(we.x), bf_hi(we.x), bf_lo(we.y), bf_hi(we.y));
        tc[j] = make_float4(bf_lo(wc.x), bf_hi(wc.x), bf_lo(wc.y), bf_hi(wc.y));
        tt[j] = *reinterpret_cast<const float4 *>(a.tin_trailing + (size_t)trow * K + i);
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int i = 4 * (int)threadIdx.x + 1024 * j;
      if (i < K) {
        const float4 sm = make_float4(tsum[j].x + te[j].x, tsum[j].y + te[j].y, tsum[j].z + te[j].z,
                                      tsum[j].w + te[j].w);
        const float4 v = make_float4((tc[j].x + sm.x) + tt[j].x, (tc[j].y + sm.y) + tt[j].y,
                                     (tc[j].z + sm.z) + tt[j].z, (tc[j].w + sm.w) + tt[j].w);
        *reinterpret_cast<float4 *>(&xs[0][i]) = v;
        if (blockIdx.x == 0) *reinterpret_cast<float4 *>(a.tin_x + i) = v;
      }
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) a.tin.codes[(size_t)frame * a.tin.groups + a.tin.code] = tok;
    gain_store();
    __syncthreads();
    if (skip_work(a.st, a.skip)) return;
    gain_read();
#pragma unroll
    for (int c = 0; c < KC; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) xv[0][c][j] = xs[0][c * 512 + lane * 8 + j];
  } else {
    // The stream-state check comes after the loads (every address above is valid whatever
    // the state), so its round trip overlaps theirs instead of preceding them.  Nothing is
    // stored before it.
    if (skip_work(a.st, a.skip)) return;
  }
  if constexpr (PARTS) {
    const int i = 4 * (int)threadIdx.x;
    if (i < K) {
#pragma unroll
      for (int m = 0; m < PR; ++m) {
        float4 v = px_[m];
#pragma unroll
        for (int p = 0; p < kMaxParts; ++p)
          if (p < a.n_parts) {
            v.x += pp_[p][m].x;
            v.y += pp_[p][m].y;
            v.z += pp_[p][m].z;
            v.w += pp_[p][m].w;
          }
        *reinterpret_cast<float4 *>(&xs[m][i]) = v;
        if (a.x_store && blockIdx.x == 0) *reinterpret_cast<float4 *>(a.x_store + m * a.ldxs_r + i) = v;
      }
    }
    gain_store();
    __syncthreads();
    gain_read();
#pragma unroll
    for (int m = 0; m < PR; ++m)
#pragma unroll
      for (int c = 0; c < KC; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) xv[m][c][j] = xs[m][c * 512 + lane * 8 + j];
  }
  if constexpr (XLDS) {
#pragma unroll
    for (int j = 0; j < XQ; ++j) {
      const int i = 4 * (int)threadIdx.x + 4 * NTH * j;
      if (i < K) *reinterpret_cast<float4 *>(&xs[0][i]) = xq[j];
    }
    gain_store();
    __syncthreads();
    gain_read();
#pragma unroll
    for (int c = 0; c < KC; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) xv[0][c][j] = xs[0][c * 512 + lane * 8 + j];
  }
  if constexpr (ATTN_EARLY) {
    if (threadIdx.x * 8 < K) merge_finish(a, threadIdx.x * 8, mregs, xs[0]);
    __syncthreads();
#pragma unroll
    for (int c = 0; c < KC; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) xv[0][c][j] = xs[0][c * 512 + lane * 8 + j];
  } else if constexpr (ATTN) {
    merge_attention(a, xs[0]);
    __syncthreads();
#pragma unroll
    for (int c = 0; c < KC; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) xv[0][c][j] = xs[0][c * 512 + lane * 8 + j];
  }

  if constexpr (NORM) {
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float ss = 0.f;
#pragma unroll
      for (int c = 0; c < KC; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) ss = fmaf(xv[m][c][j], xv[m][c][j], ss);
      ss = wave_sum(ss);
      const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
#pragma unroll
      for (int c = 0; c < KC; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) xv[m][c][j] = (xv[m][c][j] * inv) * gv[c][j];
    }
  }

  float acc[MR][NR];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      float s = 0.f;
#pragma unroll
      for (int c = 0; c < KC; ++c) s += dot8(w[r][c], xv[m][c]);
      acc[m][r] = wave_sum(s);
    }

  if constexpr (HO) {
    // acc is wave-uniform: the wave's best key, then the workgroup's, in a fixed order.
    uint64_t best = 0;
#pragma unroll
    for (int r = 0; r < RW; ++r)
      if (unit0 + r < a.N) best = umax64(best, order_key(acc[0][r], unit0 + r));
    if (lane == 0) wkeys[wave] = best;
    if (a.trace) {
      float *tr = a.trace + (size_t)a.st->frame * a.trace_frame;
#pragma unroll
      for (int r = 0; r < RW; ++r)
        if (lane == r && unit0 + r < a.N) tr[unit0 + r] = acc[0][r];
    }
    __syncthreads();
    if (threadIdx.x == 0)
      a.keys_out[blockIdx.x] = umax64(umax64(wkeys[0], wkeys[1]), umax64(wkeys[2], wkeys[3]));
  }

#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int unit = unit0 + r;
      float *out = a.out + m * a.ldo_r;
      if (lane == r && unit < a.N) {
        if constexpr (EPI == EPI_STORE) {
          out[unit] = acc[m][r];
        } else if constexpr (EPI == EPI_RESIDUAL) {
          out[unit] = eadd[m] + acc[m][r];
        } else if constexpr (EPI == EPI_BIAS) {
          out[unit] = acc[m][r] + eadd[m];
        } else {
          const float g = acc[m][2 * r], u = acc[m][2 * r + 1];
          out[unit] = g / (1.0f + expf(-g)) * u;
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
  __device__ static float round(float x) { return x; }

  template <bool NT = false>
  __device__ static void load8(const float *p, float *o) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4 *q = reinterpret_cast<const f4 *>(p);
    f4 a, b;
    if constexpr (NT) {
      a = __builtin_nontemporal_load(q);
      b = __builtin_nontemporal_load(q + 1);
    } else {
      a = q[0];
      b = q[1];
    }
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  }
  __device__ static float2 load2(const float *p) { return *reinterpret_cast<const float2 *>(p); }
  template <bool NT = false>
  __device__ static float4 load4(const float *p) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    if constexpr (NT) {
      const f4 v = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(p));
      return make_float4(v.x, v.y, v.z, v.w);
    }
    return *reinterpret_cast<const float4 *>(p);
  }
  // Elements 4 sub .. 4 sub + 3 and 64 + 4 sub .. 64 + 4 sub + 3 of a 128-element row: 16 lanes
  // then read the row as two contiguous 256-byte halves; split_dim(sub, j) is element j's index.
  __device__ static void load8_split(const float *row, int sub, float *o) {
    const float4 a = *reinterpret_cast<const float4 *>(row + 4 * sub);
    const float4 b = *reinterpret_cast<const float4 *>(row + 64 + 4 * sub);
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  }
  __device__ static constexpr int split_dim(int sub, int j) { return j < 4 ? 4 * sub + j : 60 + 4 * sub + j; }
};

template <>
struct KvIo<uint16_t> {
  __device__ static float store(uint16_t *p, float x) {
    const uint16_t b = f32_to_bf16(x);
    *p = b;
    return bf16_to_f32(b);
  }
  __device__ static float round(float x) { return bf16_to_f32(f32_to_bf16(x)); }

  template <bool NT = false>
  __device__ static void load8(const uint16_t *p, float *o) {
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    u4 w;
    if constexpr (NT)
      w = __builtin_nontemporal_load(reinterpret_cast<const u4 *>(p));
    else
      w = *reinterpret_cast<const u4 *>(p);
    o[0] = bf_lo(w.x); o[1] = bf_hi(w.x); o[2] = bf_lo(w.y); o[3] = bf_hi(w.y);
    o[4] = bf_lo(w.z); o[5] = bf_hi(w.z); o[6] = bf_lo(w.w); o[7] = bf_hi(w.w);
  }
  __device__ static float2 load2(const uint16_t *p) {
    const uint32_t w = *reinterpret_cast<const uint32_t *>(p);
    return make_float2(bf_lo(w), bf_hi(w));
  }
  template <bool NT = false>
  __device__ static float4 load4(const uint16_t *p) {
    typedef unsigned int u2 __attribute__((ext_vector_type(2)));
    u2 w;
    if constexpr (NT)
      w = __builtin_nontemporal_load(reinterpret_cast<const u2 *>(p));
    else
      w = *reinterpret_cast<const u2 *>(p);
    return make_float4(bf_lo(w.x), bf_hi(w.x), bf_lo(w.y), bf_hi(w.y));
  }
  // bf16 rows: one 16-byte load of 8 consecutive elements already covers 256 contiguous bytes
  // per row over 16 lanes.
  __device__ static void load8_split(const uint16_t *row, int sub, float *o) { load8(row + 8 * sub, o); }
  __device__ static constexpr int split_dim(int sub, int j) { return 8 * sub + j; }
};

// ---------------------------------------------------------------------------------------
// Decode attention, split over the key positions (flash-decoding).
// Grid (kv_heads, max_chunks); workgroup (h, c) owns key rows [c * chunk, min(L, (c+1) * chunk))
// of KV head h and its G query heads.
//   1. q head RMSNorm + rotate-half RoPE at `pos` (every workgroup, wave per head); the
//      workgroup whose chunk holds `pos` also normalises/rotates k, stores K and V at row
//      `pos` (rounded to the cache type) and keeps them in LDS;
//   2. scores (16 lanes per row, 8 dims per lane), chunk max m, p = exp(s - m), l = sum p,
//      acc = sum p * V;
//   3. partial_out = 0 (one chunk by construction): out = acc / l.  partial_out = 1: the
//      chunk's (m, l, acc) go to `part`; the consumer (the O-projection GEMV) merges the
//      chunks in chunk order after the kernel boundary, so no workgroup fences or waits.
// ---------------------------------------------------------------------------------------
constexpr int kAttnMaxChunk = 128;
constexpr int kAttnMaxChunks = kAttnGemvMergeChunks;

// The stores of a TokenHandoff, by one 256-thread workgroup: thread t covers elements
// 4t .. 4t+3 and 1024 + 4t .. (widths up to 2048).  handoff_load issues every load (the
// embedding row, the running sum, the table row), handoff_store the sums and stores.
__device__ __forceinline__ void handoff_load(const TokenHandoff &h, int row, int tok, float4 *e, float4 *sum,
                                             float4 *cur) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int i = 4 * (int)threadIdx.x + 1024 * j;
    e[j] = sum[j] = cur[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (i < h.emb_width) {
      const uint2 w = *reinterpret_cast<const uint2 *>(h.emb + (size_t)tok * h.emb_width + i);
      e[j] = make_float4(bf_lo(w.x), bf_hi(w.x), bf_lo(w.y), bf_hi(w.y));
      if (!h.first) sum[j] = *reinterpret_cast<const float4 *>(h.sum + row * h.sum_row + i);
    }
    if (h.cur_table && i < h.cur_width)
      cur[j] = *reinterpret_cast<const float4 *>(h.cur_table + (size_t)tok * h.cur_width + i);
  }
}

__device__ __forceinline__ void handoff_store(const TokenHandoff &h, int row, int tok, const SlotState *st,
                                              const float4 *e, const float4 *sum, const float4 *cur) {
  float *hsum = h.sum + row * h.sum_row, *hcur = h.cur + row * h.cur_row;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int i = 4 * (int)threadIdx.x + 1024 * j;
    if (i < h.emb_width) {
      const float4 s = h.first ? e[j]
                               : make_float4(sum[j].x + e[j].x, sum[j].y + e[j].y, sum[j].z + e[j].z, sum[j].w + e[j].w);
      *reinterpret_cast<float4 *>(hsum + i) = s;
      if (!h.cur_table) *reinterpret_cast<float4 *>(hcur + i) = e[j];
    }
    if (h.cur_table && i < h.cur_width) *reinterpret_cast<float4 *>(hcur + i) = cur[j];
  }
  if (threadIdx.x == 0) {
    int32_t *codes = h.codes + row * h.codes_row + (size_t)st->frame * h.groups;
    codes[h.code] = tok;
    if (h.first) codes[0] = st->semantic;
  }
}

// HO = greedy token hand-off (AttnArgs::h): the q/k/v row comes from a table indexed by the
// token the previous group's LM head chose; workgroup (0, 0) also does the hand-off's stores.
// OPROJ = the output projection fused in, its K dimension split by KV head (one chunk, one
// stream): grid (kv_heads, wo_rows / kOprojRows).  Workgroup (h, b) computes KV head h's
// attention (every b alike), then opart[h][r] = sum over head h's G * D columns of
// wo[r][.] * attn for its kOprojRows rows r.  The consumer adds the kv_heads partials to the
// residual in head order (k_gemv with GemvArgs::parts).  Only b = 0 stores the K/V row at
// `pos` (and, with HO, the hand-off's rows); the others round it as the store would.
constexpr int kOprojRows = 32;

template <int D, int G, typename KVT, int CH, bool HO = false, bool OPROJ = false>
__global__ __launch_bounds__(256) void k_attn_split(AttnArgs a) {
  static_assert(D == 128, "lane layout assumes head_dim 128");
  static_assert(G >= 1 && G <= 2, "query heads per KV head");
  static_assert(CH % 16 == 0 && CH <= kAttnMaxChunk, "chunk length");
  static_assert(!OPROJ || CH <= 32, "the fused projection covers one chunk of at most 32 rows");
  // The Talker's form (no fused projection) reads each K/V row once per step: non-temporal
  // loads, as for the Talker's weights (the CodePredictor's form rereads its rows every group).
  constexpr bool KV_NT = !OPROJ;
  const int row = blockIdx.z;
  const SlotState *st = a.st + row;
  // A position given by the launch needs no state: the row mask and the stream state are
  // then checked after the loads below are issued (they are valid for any state).
  const bool frame_pos = a.pos_mode == POS_TALKER_FRAME;
  int frame = 0, prefill_steps = 0;
  if (frame_pos) {
    // the row mask and the state in one round trip (both addresses are known)
    const int on = a.row_on ? a.row_on[row] : 1;
    const SlotState sv = *st;
    if (!on || skip_state(sv, a.skip)) return;
    frame = sv.frame;
    prefill_steps = sv.prefill_steps;
  }
  const int h = blockIdx.x;
  const int c = OPROJ ? 0 : blockIdx.y;
  const int rb = OPROJ ? blockIdx.y : 0;  // output row block of the fused projection
  const int pos = frame_pos ? prefill_steps + frame : a.pos_const;
  if (pos < 0 || pos >= a.cap) return;  // host validates; never index outside the cache
  const int L = pos + 1;
  const int nchunks = (L + CH - 1) / CH;
  if (c >= nchunks) return;
  const int t0 = c * CH;
  const int t1 = min(L, t0 + CH);
  const int tpast = min(t1, pos);  // rows [t0, tpast) come from the cache
  const bool owns_pos = (c == nchunks - 1);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sub = lane & 15;
  const int grp = lane >> 4;
  const int q_out = a.q_heads * D;
  const int kv_out = a.kv_heads * D;
  KVT *kcache = reinterpret_cast<KVT *>(a.kcache) + row * a.kv_row;
  KVT *vcache = reinterpret_cast<KVT *>(a.vcache) + row * a.kv_row;
  const float *qkv = a.qkv + (size_t)row * a.ld_qkv;
  const KVT *kbase = kcache + (size_t)h * a.cap * D;
  const KVT *vbase = vcache + (size_t)h * a.cap * D;

  __shared__ float qs[G * D];
  __shared__ __align__(16) float ks[D], vs[D];
  __shared__ float sc[G][CH];
  __shared__ float red[4][G][D];
  __shared__ float stat[G][2];
  __shared__ float ao[OPROJ ? G * D : 1];

  // Loads first: this wave's head vector, then every cached K and V row the workgroup needs
  // (addresses clamped into the cache instead of branching), so the kernel waits on one
  // memory round trip.  Rows at or past `pos` are never used from these registers.  With the
  // hand-off, the head vector's row is known only once the keys (loaded first) are reduced.
  const int vec = wave;
  const bool has_vec = wave < G + 2 && (wave < G || owns_pos);
  const float *gain = vec < G ? a.gq : (vec == G ? a.gk : nullptr);
  float x0 = 0.f, x1 = 0.f, g0 = 0.f, g1 = 0.f;
  float2 cs = make_float2(0.f, 0.f);
  const int vec_off = vec < G ? (h * G + vec) * D : (vec == G ? q_out + h * D : q_out + kv_out + h * D);
  uint64_t kin[HO ? 4 : 1];
  int tok_in = 0;
  if constexpr (HO) {
    if (a.h.tok_in) {
      tok_in = *a.h.tok_in;
    } else {
      const uint64_t *keys = a.h.keys + row * a.h.keys_row;
#pragma unroll
      for (int j = 0; j < 4; ++j) kin[j] = keys[min(lane + 64 * j, a.h.n_keys - 1)];
    }
  }
  if (has_vec) {
    if constexpr (!HO) {
      x0 = qkv[vec_off + lane];
      x1 = qkv[vec_off + lane + 64];
    }
    if (gain) {
      g0 = gain[lane];
      g1 = gain[lane + 64];
      cs = a.rope[(size_t)pos * (D / 2) + lane];
    }
  }
  const int tmax = max(pos - 1, 0);
  float kpre[CH / 16][8];
#pragma unroll
  for (int i = 0; i < CH / 16; ++i) {
    const int t = min(t0 + wave * 4 + grp + 16 * i, tmax);
    KvIo<KVT>::template load8<KV_NT>(kbase + (size_t)t * D + sub * 8, kpre[i]);
  }
  // V rows two per load instruction: half-wave hf of wave w takes row t0 + 8 i + 2 w + hf,
  // lane q = lane % 32 of it dims 4q .. 4q + 3.
  const int hf = lane >> 5, q4 = (lane & 31) * 4;
  float4 vpre[CH / 8];
#pragma unroll
  for (int i = 0; i < CH / 8; ++i) {
    const int t = min(t0 + 8 * i + 2 * wave + hf, tmax);
    vpre[i] = KvIo<KVT>::template load4<KV_NT>(vbase + (size_t)t * D + q4);
  }
  // The fused projection's weights: wave w takes rows rb * kOprojRows + w * kOprojRows / 4 ..;
  // a row's G * D bf16 of head h are LPR lanes x 8, so one 16-byte load per lane covers RPL
  // rows.
  constexpr int LPR = G * D / 8;
  constexpr int RPL = 64 / LPR;
  constexpr int NWO = OPROJ ? kOprojRows / 4 / RPL : 1;
  uint4 wo[NWO];
  if constexpr (OPROJ) {
#pragma unroll
    for (int i = 0; i < NWO; ++i) {
      const int r = rb * kOprojRows + wave * (kOprojRows / 4) + i * RPL + lane / LPR;
      wo[i] = *reinterpret_cast<const uint4 *>(a.wo + (size_t)r * q_out + h * G * D + (lane % LPR) * 8);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  if (!frame_pos) {  // workgroup-uniform: no barrier has been reached yet
    if (a.row_on && !a.row_on[row]) return;
    if (skip_work(st, a.skip)) return;
  }
  // Hand-off: the token, its q/k/v row, and (workgroup (0, 0)) the rows the hand-off stores,
  // loaded here and stored after the attention output.
  int tok = 0;
  float4 side_e[2], side_s[2], side_c[2];
  if constexpr (HO) {
    tok = a.h.tok_in ? tok_in : key_token(wave_max_u64(umax64(umax64(kin[0], kin[1]), umax64(kin[2], kin[3]))));
    if (has_vec) {
      const float *src = a.qkv_table + (size_t)tok * a.ld_table + vec_off;
      x0 = src[lane];
      x1 = src[lane + 64];
    }
    if (h == 0 && c == 0 && rb == 0 && a.h.emb) handoff_load(a.h, row, tok, side_e, side_s, side_c);
  }

  // 1: q heads (waves 0..G-1); k and v (waves G, G+1) only where row `pos` is stored.
  if (has_vec) {
    if (gain) {
      const float ss = wave_sum(fmaf(x0, x0, x1 * x1));
      const float inv = 1.0f / sqrtf(ss / (float)D + a.eps);
      x0 = (x0 * inv) * g0;
      x1 = (x1 * inv) * g1;
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
      if (rb == 0) {
        keep[lane] = KvIo<KVT>::store(cache + row + lane, x0);
        keep[lane + 64] = KvIo<KVT>::store(cache + row + lane + 64, x1);
      } else {
        keep[lane] = KvIo<KVT>::round(x0);
        keep[lane + 64] = KvIo<KVT>::round(x1);
      }
    }
  }
  __syncthreads();

  // 2a: scores of this chunk.  The stored row's slice is read from LDS unconditionally, once:
  // read under the row test, it became a branch and a masked scalar LDS read per element.
  float kown[8];
  {
    const float4 a0 = *reinterpret_cast<const float4 *>(&ks[sub * 8]);
    const float4 a1 = *reinterpret_cast<const float4 *>(&ks[sub * 8 + 4]);
    kown[0] = a0.x; kown[1] = a0.y; kown[2] = a0.z; kown[3] = a0.w;
    kown[4] = a1.x; kown[5] = a1.y; kown[6] = a1.z; kown[7] = a1.w;
  }
#pragma unroll
  for (int i = 0; i < CH / 16; ++i) {
    const int t = t0 + wave * 4 + grp + 16 * i;
    if (t0 + wave * 4 + 16 * i >= t1) break;  // wave-uniform
    float kv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) kv[j] = (t < tpast) ? kpre[i][j] : ((t == pos) ? kown[j] : 0.f);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float sacc = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) sacc = fmaf(qs[g * D + sub * 8 + j], kv[j], sacc);
      sacc = row16_sum(sacc);
      if (sub == 0 && t < t1) sc[g][t - t0] = sacc * a.scale;
    }
  }
  __syncthreads();

  // 2b: chunk max and exp (wave g handles query head g, 64 rows per pass).
  const int n = t1 - t0;
  if (wave < G) {
    float m = -FLT_MAX;
    for (int i = lane; i < n; i += 64) m = fmaxf(m, sc[wave][i]);
    m = wave_max(m);
    float l = 0.f;
    for (int i = lane; i < n; i += 64) {
      const float p = expf(sc[wave][i] - m);
      sc[wave][i] = p;
      l += p;
    }
    l = wave_sum(l);
    if (lane == 0) {
      stat[wave][0] = m;
      stat[wave][1] = l;
    }
  }
  __syncthreads();

  // 2c: acc = sum_t p_t V_t over the rows of the loads above (value g * 4 + k: query head g,
  // dim 4q + k).  The two half-waves' sums are then folded by one lane swap per pair of
  // values: lanes 0-31 keep values 0 .. 2G - 1, lanes 32-63 values 2G .. 4G - 1.
  constexpr int NV = 4 * G;
  float acc[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) acc[v] = 0.f;
  const float4 vown = *reinterpret_cast<const float4 *>(&vs[q4]);
#pragma unroll
  for (int i = 0; i < CH / 8; ++i) {
    if (t0 + 8 * i + 2 * wave >= t1) break;  // wave-uniform
    const int t = t0 + 8 * i + 2 * wave + hf;
    const float4 v = (t < tpast) ? vpre[i] : ((t == pos) ? vown : make_float4(0.f, 0.f, 0.f, 0.f));
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float p = (t < t1) ? sc[g][min(t - t0, CH - 1)] : 0.f;
      acc[g * 4 + 0] = fmaf(p, v.x, acc[g * 4 + 0]);
      acc[g * 4 + 1] = fmaf(p, v.y, acc[g * 4 + 1]);
      acc[g * 4 + 2] = fmaf(p, v.z, acc[g * 4 + 2]);
      acc[g * 4 + 3] = fmaf(p, v.w, acc[g * 4 + 3]);
    }
  }
#pragma unroll
  for (int k = 0; k < NV / 2; ++k) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[k]), __float_as_uint(acc[k + NV / 2]),
                                                    false, false);
    const int v = hf * (NV / 2) + k;
    red[wave][v / 4][q4 + v % 4] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  __syncthreads();

  if constexpr (HO) {
    if (h == 0 && c == 0 && rb == 0 && a.h.emb) handoff_store(a.h, row, tok, st, side_e, side_s, side_c);
  }

  if constexpr (OPROJ) {
    // 3': this head's attention output to LDS, then its slice of the projection.  Rows of
    // LPR = 32 lanes are summed across their two 16-lane rows by row_bcast:15 (a VALU lane
    // permute), which leaves each row's sum in lanes 16..31 (and 48..63).
    const int o = threadIdx.x;
    if (o < G * D) {
      const int g_o = o / D, d_o = o % D;
      const float v_o = ((red[0][g_o][d_o] + red[1][g_o][d_o]) + red[2][g_o][d_o]) + red[3][g_o][d_o];
      ao[o] = v_o / stat[g_o][1];
    }
    __syncthreads();
    // every row's sum first, then the stores: with no store (and its lane mask) between
    // them, the NWO independent dot / DPP chains share one basic block and interleave
    float sum[NWO];
#pragma unroll
    for (int i = 0; i < NWO; ++i) {
      sum[i] = row16_sum(dot8(wo[i], ao + (lane % LPR) * 8));
      if constexpr (LPR == 32) sum[i] += dpp_f<0x142, 0xa>(sum[i], 0.f);
    }
    if (lane % LPR == LPR - 1) {
#pragma unroll
      for (int i = 0; i < NWO; ++i)
        a.opart[(size_t)h * a.wo_rows + rb * kOprojRows + wave * (kOprojRows / 4) + i * RPL + lane / LPR] = sum[i];
    }
    return;
  }

  // 3: final output (single chunk) or this chunk's partial.
  const int o = threadIdx.x;  // G * D <= 256 outputs
  if (o >= G * D) return;
  const int g_o = o / D, d_o = o % D;
  const float v_o = ((red[0][g_o][d_o] + red[1][g_o][d_o]) + red[2][g_o][d_o]) + red[3][g_o][d_o];
  if (!a.partial_out) {
    const int k = (h * G + g_o) * D + d_o;
    a.out[a.out_t16 ? t16_index(row, k) : (size_t)row * a.ld_out + k] = v_o / stat[g_o][1];
    return;
  }
  float *my = a.part + row * a.part_row + (((size_t)h * a.part_chunks + c) * G + g_o) * (D + 2);
  my[2 + d_o] = v_o;
  if (d_o == 0) {
    my[0] = stat[g_o][0];
    my[1] = stat[g_o][1];
  }
}

// Merges the attention partials of all query heads into xs[q_heads * D] (LDS), in chunk
// order: out = sum_c e^(m_c - M) acc_c / sum_c e^(m_c - M) l_c.  256 threads, 8 dims each.
__device__ void merge_attention(const GemvArgs &a, float *xs) {
  for (int base = threadIdx.x * 8; base < a.K; base += 256 * 8) {
    MergeRegs r;
    merge_load(a, base, r);
    merge_finish(a, base, r, xs);
  }
}

// The Talker's decode attention with its O projection fused in, one stream (no partials, no
// merge, no second launch).  Grid (kv_heads, N / ROWS), 16 waves.  Workgroup (h, b) runs KV
// head h's whole attention over key rows [0, pos] and multiplies its G query heads' outputs by
// head h's G * D columns of W_o for output rows ROWS * b ..: out[h][r] = that share of
// (W_o attn)[r], summed into the residual by the gate/up GEMV (GemvArgs::parts).
//   - Block id = h + kv_heads * b, and workgroup i runs on XCD i mod 8: with 8 KV heads every
//     workgroup of head h is on XCD h, so the head's K/V rows come from HBM once and from
//     that XCD's L2 for the other workgroups.
//   - Loads before the state: the W_o slice (streamed), the q/k/v head vectors and the norm
//     gains.  After it: the RoPE row and the first kFusedRows key rows' K and V (one round
//     trip); longer caches take one more round trip per further kFusedRows rows.
//   - Only b = 0 stores the K/V row at `pos`; every workgroup computes it (same arithmetic).
//   - Scores of every row go to LDS (wave w: rows 4w + (lane >> 4) + 64 i, 16 lanes x 8 dims
//     per row), then one softmax over all rows (wave g: query head g), then P.V summed over
//     the 16 waves in wave order: fp32 caches (V4) load V rows two per 16-byte load (half-wave
//     h of wave w: row 2 (16 i + w) + h, lane: 4 dims), the half-waves' sums folded by
//     v_permlane32_swap; bf16 caches one row per load (wave w: rows w + 16 i, lane: dims
//     2 lane, 2 lane + 1), which measured faster for them.
constexpr int kFusedWaves = 16;
constexpr int kFusedRows = 256;      // key rows per register pass
constexpr int kFusedMaxCap = 1024;   // longest cache (score rows in LDS)

template <int G, typename KVT, bool V4 = sizeof(KVT) == 4>
__global__ __launch_bounds__(64 * kFusedWaves) void k_attn_oproj_full(AttnArgs a) {
  constexpr int D = 128, NW = kFusedWaves, BL = kFusedRows;
  constexpr int KI = BL / (NW * 4);  // K rows per lane per pass
  constexpr int VI = BL / NW;        // V rows per wave per pass
  constexpr int LPR = G * D / 8;     // lanes per W_o row slice
  constexpr int RPL = 64 / LPR;      // W_o rows per wave load
  constexpr int ROWS = NW * RPL;     // W_o rows per workgroup
  static_assert(G >= 1 && G <= 2, "query heads per KV head");
  const int h = blockIdx.x, rb = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane & 15, grp = lane >> 4;
  const int q_out = a.q_heads * D, kv_out = a.kv_heads * D;
  KVT *kcache = reinterpret_cast<KVT *>(a.kcache);
  KVT *vcache = reinterpret_cast<KVT *>(a.vcache);
  const KVT *kbase = kcache + (size_t)h * a.cap * D;
  const KVT *vbase = vcache + (size_t)h * a.cap * D;

  __shared__ float qs[G * D];
  __shared__ __align__(16) float ks[D], vs[D];
  __shared__ float sc[G][kFusedMaxCap];
  __shared__ float red[NW][G][D];
  __shared__ float stat[G][2];
  __shared__ float ao[G * D];

  // 1. Everything that does not depend on the position.
  const int orow = rb * ROWS + wave * RPL + lane / LPR;
  const uint4 wo = load_w<true>(reinterpret_cast<const u32x4 *>(a.wo + (size_t)orow * q_out + h * G * D +
                                                                  (lane % LPR) * 8));
  const int vec = wave;  // waves 0..G-1: q heads; G: k; G+1: v
  const bool has_vec = wave < G + 2;
  const float *gain = vec < G ? a.gq : (vec == G ? a.gk : nullptr);
  const int vec_off = vec < G ? (h * G + vec) * D : (vec == G ? q_out + h * D : q_out + kv_out + h * D);
  float x0 = 0.f, x1 = 0.f, g0 = 0.f, g1 = 0.f;
  if (has_vec) {
    x0 = a.qkv[vec_off + lane];
    x1 = a.qkv[vec_off + lane + 64];
    if (gain) {
      g0 = gain[lane];
      g1 = gain[lane + 64];
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // 2. The position (stream state, or the launch's), then the first pass's K/V rows.
  int pos = a.pos_const;
  if (a.pos_mode == POS_TALKER_FRAME) {
    const SlotState sv = *a.st;
    if (skip_state(sv, a.skip)) return;
    pos = sv.prefill_steps + sv.frame;
  } else if (skip_work(a.st, a.skip)) {
    return;
  }
  if (pos < 0 || pos >= a.cap) return;  // host validates; never index outside the cache
  const int L = pos + 1;
  const int tmax = max(pos - 1, 0);
  float2 cs = make_float2(0.f, 0.f);
  if (has_vec && gain) cs = a.rope[(size_t)pos * (D / 2) + lane];
  // fp32 caches: only the row groups that hold rows below L are loaded (wave-uniform tests):
  // every load instruction costs the CU the same load-path time, used or not, and a short
  // cache needs a fraction of them.  bf16 caches load every group (clamped): there the tests
  // measured slower from half the cache on.  Each lane of an fp32 K row takes dims 4 sub ..
  // 4 sub + 3 and 64 + 4 sub .. (KvIo::load8_split), so one instruction covers 256
  // contiguous bytes per row.
  constexpr bool GUARD = sizeof(KVT) == 4;
  float kreg[KI][8];
  float2 vreg[V4 ? 1 : VI];
  // V4: V rows two per 16-byte load, half-wave hf of wave w taking row p0 + 2 (NW i + w) + hf,
  // lane q = lane % 32 dims 4q .. 4q + 3
  const int hf = lane >> 5, q4 = (lane & 31) * 4;
  float4 vreg4[V4 ? VI / 2 : 1];
  auto load_k = [&](int p0) {
#pragma unroll
    for (int i = 0; i < KI; ++i) {
      if (GUARD && p0 + wave * 4 + 64 * i >= L) break;
      const int t = min(p0 + wave * 4 + grp + 64 * i, tmax);
      KvIo<KVT>::load8_split(kbase + (size_t)t * D, sub, kreg[i]);
    }
  };
  auto load_v = [&](int p0) {
    if constexpr (V4) {
#pragma unroll
      for (int i = 0; i < VI / 2; ++i) {
        if (GUARD && p0 + 2 * (NW * i + wave) >= L) break;
        const int t = min(p0 + 2 * (NW * i + wave) + hf, tmax);
        vreg4[i] = KvIo<KVT>::load4(vbase + (size_t)t * D + q4);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < VI; ++i) {
      if (GUARD && p0 + wave + NW * i >= L) break;
      const int t = min(p0 + wave + NW * i, tmax);
      vreg[i] = KvIo<KVT>::load2(vbase + (size_t)t * D + 2 * lane);
    }
  };
  load_k(0);
  load_v(0);

  // 3. q heads (waves 0..G-1), k and v (waves G, G+1): norm, RoPE, the row at `pos`.
  if (has_vec) {
    if (gain) {
      const float ss = wave_sum(fmaf(x0, x0, x1 * x1));
      const float inv = 1.0f / sqrtf(ss / (float)D + a.eps);
      x0 = (x0 * inv) * g0;
      x1 = (x1 * inv) * g1;
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
      const size_t r = ((size_t)h * a.cap + pos) * D;
      if (rb == 0) {
        keep[lane] = KvIo<KVT>::store(cache + r + lane, x0);
        keep[lane + 64] = KvIo<KVT>::store(cache + r + lane + 64, x1);
      } else {
        keep[lane] = KvIo<KVT>::round(x0);
        keep[lane + 64] = KvIo<KVT>::round(x1);
      }
    }
  }
  __syncthreads();

  // 4. Scores of every row [0, L) (the dims of load8_split).
  float kown[8];
  {
    const float4 a0 = *reinterpret_cast<const float4 *>(&ks[KvIo<KVT>::split_dim(sub, 0)]);
    const float4 a1 = *reinterpret_cast<const float4 *>(&ks[KvIo<KVT>::split_dim(sub, 4)]);
    kown[0] = a0.x; kown[1] = a0.y; kown[2] = a0.z; kown[3] = a0.w;
    kown[4] = a1.x; kown[5] = a1.y; kown[6] = a1.z; kown[7] = a1.w;
  }
  for (int p0 = 0; p0 < L; p0 += BL) {
    if (p0 > 0) load_k(p0);
#pragma unroll
    for (int i = 0; i < KI; ++i) {
      const int t = p0 + wave * 4 + grp + 64 * i;
      if (p0 + wave * 4 + 64 * i >= L) break;  // wave-uniform
      float kv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) kv[j] = (t < pos) ? kreg[i][j] : ((t == pos) ? kown[j] : 0.f);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float sacc = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) sacc = fmaf(qs[g * D + KvIo<KVT>::split_dim(sub, j)], kv[j], sacc);
        sacc = row16_sum(sacc);
        if (sub == 0 && t < L) sc[g][t] = sacc * a.scale;
      }
    }
  }
  __syncthreads();

  // 5. Softmax over all rows (wave g: query head g).
  if (wave < G) {
    float m = -FLT_MAX;
    for (int i = lane; i < L; i += 64) m = fmaxf(m, sc[wave][i]);
    m = wave_max(m);
    float l = 0.f;
    for (int i = lane; i < L; i += 64) {
      const float p = expf(sc[wave][i] - m);
      sc[wave][i] = p;
      l += p;
    }
    l = wave_sum(l);
    if (lane == 0) {
      stat[wave][0] = m;
      stat[wave][1] = l;
    }
  }
  __syncthreads();

  // 6. P.V, per wave, then the 16 waves' sums in wave order.
  if constexpr (V4) {
    // value g * 4 + k: query head g, dim 4q + k; the half-waves' sums folded by one lane swap
    // per pair of values (lanes 0-31 keep values 0 .. 2G - 1, lanes 32-63 the rest)
    constexpr int NV = 4 * G;
    float acc[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) acc[v] = 0.f;
    const float4 vown = *reinterpret_cast<const float4 *>(&vs[q4]);
    for (int p0 = 0; p0 < L; p0 += BL) {
      if (p0 > 0) load_v(p0);
#pragma unroll
      for (int i = 0; i < VI / 2; ++i) {
        if (p0 + 2 * (NW * i + wave) >= L) break;  // wave-uniform
        const int t = p0 + 2 * (NW * i + wave) + hf;
        const float4 v = (t < pos) ? vreg4[i] : ((t == pos) ? vown : make_float4(0.f, 0.f, 0.f, 0.f));
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float p = (t < L) ? sc[g][min(t, L - 1)] : 0.f;
          acc[g * 4 + 0] = fmaf(p, v.x, acc[g * 4 + 0]);
          acc[g * 4 + 1] = fmaf(p, v.y, acc[g * 4 + 1]);
          acc[g * 4 + 2] = fmaf(p, v.z, acc[g * 4 + 2]);
          acc[g * 4 + 3] = fmaf(p, v.w, acc[g * 4 + 3]);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < NV / 2; ++k) {
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[k]), __float_as_uint(acc[k + NV / 2]),
                                                      false, false);
      const int v = hf * (NV / 2) + k;
      red[wave][v / 4][q4 + v % 4] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
  } else {
    float acc[G][2];
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g][0] = acc[g][1] = 0.f;
    for (int p0 = 0; p0 < L; p0 += BL) {
      if (p0 > 0) load_v(p0);
#pragma unroll
      for (int i = 0; i < VI; ++i) {
        const int t = p0 + wave + NW * i;
        if (t >= L) break;  // wave-uniform
        const float2 v = (t < pos) ? vreg[i] : make_float2(vs[2 * lane], vs[2 * lane + 1]);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float p = sc[g][t];
          acc[g][0] = fmaf(p, v.x, acc[g][0]);
          acc[g][1] = fmaf(p, v.y, acc[g][1]);
        }
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      red[wave][g][2 * lane] = acc[g][0];
      red[wave][g][2 * lane + 1] = acc[g][1];
    }
  }
  __syncthreads();
  if (threadIdx.x < G * D) {
    const int g_o = threadIdx.x / D, d_o = threadIdx.x % D;
    float v_o = red[0][g_o][d_o];
#pragma unroll
    for (int w = 1; w < NW; ++w) v_o += red[w][g_o][d_o];
    ao[threadIdx.x] = v_o / stat[g_o][1];
  }
  __syncthreads();

  // 7. This workgroup's rows of head h's share of W_o attn.
  float sum = row16_sum(dot8(wo, ao + (lane % LPR) * 8));
  if constexpr (LPR == 32) sum += dpp_f<0x142, 0xa>(sum, 0.f);
  if (lane % LPR == LPR - 1) a.opart[(size_t)h * a.wo_rows + orow] = sum;
}

// Stream-row form of merge_attention for the batched frame: workgroup (h, r) merges KV head
// h's G query heads of row r (thread = two adjacent output elements), in chunk order as in
// merge_attention.
// NC = chunk slots loaded (a multiple of 8 >= part_chunks): every partial of every slot is
// loaded before the stream state is read, so the merge waits on one memory round trip.
template <int NC>
__global__ __launch_bounds__(128) void k_attn_merge(AttnMergeArgs a) {
  constexpr int D = 128;
  const int h = blockIdx.x;
  const int row = blockIdx.y;
  const int G = a.q_heads / a.kv_heads;
  if (2 * (int)threadIdx.x >= G * D) return;
  const int g = 2 * threadIdx.x / D, d = 2 * threadIdx.x % D;  // two output elements per thread
  const float *p0 = a.part + row * a.part_row + (((size_t)h * a.part_chunks) * G + g) * (D + 2);
  const size_t stride = (size_t)G * (D + 2);
  float mv[NC], lv[NC];
  float2 av[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const float *pc = p0 + min(c, a.part_chunks - 1) * stride;
    const float2 ml = *reinterpret_cast<const float2 *>(pc);  // records of D + 2 floats: 8-byte aligned
    mv[c] = ml.x;
    lv[c] = ml.y;
    av[c] = *reinterpret_cast<const float2 *>(pc + 2 + d);
  }
  __builtin_amdgcn_sched_barrier(0);
  if (a.row_on && !a.row_on[row]) return;
  const SlotState *st = a.st + row;
  if (skip_work(st, a.skip)) return;
  const int pos = (a.pos_mode == POS_TALKER_FRAME) ? st->prefill_steps + st->frame : a.pos_const;
  const int nchunks = min((pos + a.chunk) / a.chunk, a.part_chunks);
  // max, then the weighted sums in chunk order
  float M = -FLT_MAX;
#pragma unroll
  for (int c = 0; c < NC; ++c)
    if (c < nchunks) M = fmaxf(M, mv[c]);
  float den = 0.f, num0 = 0.f, num1 = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
    if (c < nchunks) {
      const float w = expf(mv[c] - M);
      den = fmaf(w, lv[c], den);
      num0 = fmaf(w, av[c].x, num0);
      num1 = fmaf(w, av[c].y, num1);
    }
  const int k = (h * G + g) * D + d;  // even: k, k + 1 adjacent in both layouts
  *reinterpret_cast<float2 *>(a.out + (a.out_t16 ? t16_index(row, k) : (size_t)row * a.ld_out + k)) =
      make_float2(num0 / den, num1 / den);
}

// ---------------------------------------------------------------------------------------
// Y[M][N] = X[M][K] . W[N][K]^T on the bf16 matrix cores (v_mfma_f32_16x16x32_bf16).
// W is the bf16 weight as stored; X is fp32 and enters the matrix cores as three bf16 terms
// (three MFMAs per k-block, smallest term first, fp32 accumulation).  Optional per-row scale
// and per-column gain on X (the RMSNorm of the rows) are applied while converting.
// Wave tile: (16 * MB) rows x (16 * NB) columns, no LDS: every lane loads its own A fragment
// (8 consecutive k of one row, fp32) and B fragment (8 consecutive k of one weight row, bf16).
// Operand layouts of the 16x16x32 instruction: A[i][k] in lane i + 16 (k / 8), element k % 8;
// B[k][j] in lane j + 16 (k / 8), element k % 8; C[i][j] in lane j + 16 (i / 4), element i % 4.
// SwiGLU: the first NB/2 column tiles are gate rows, the last NB/2 the matching up rows.
// ---------------------------------------------------------------------------------------
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// x = hi + mid + lo, each a bf16: 24 significant bits, so every product with a bf16 weight
// is exact and the GEMM matches an fp32 GEMV up to the order of the fp32 additions.
// hi = bf16(x) (round to nearest even, v_cvt_pk_bf16_f32 on two lanes at a time); x - hi is
// exact in fp32 and holds the remaining 16 bits, split the same way into mid and lo.
__device__ __forceinline__ void split_bf16x8(const float *x, bf16x8_t &hi, bf16x8_t &mid, bf16x8_t &lo) {
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const f32x2_t v = {x[e], x[e + 1]};
    const bf16x2_t h = __builtin_convertvector(v, bf16x2_t);
    const f32x2_t r1 = v - __builtin_convertvector(h, f32x2_t);
    const bf16x2_t m = __builtin_convertvector(r1, bf16x2_t);
    const f32x2_t r2 = r1 - __builtin_convertvector(m, f32x2_t);
    const bf16x2_t l = __builtin_convertvector(r2, bf16x2_t);
    hi[e] = h[0]; hi[e + 1] = h[1];
    mid[e] = m[0]; mid[e + 1] = m[1];
    lo[e] = l[0]; lo[e + 1] = l[1];
  }
}

// split_bf16x8 without contraction: the residual is taken from the rounded x even where x is
// a product computed just before (otherwise the compiler may fuse that product into x - hi).
__device__ __forceinline__ void split_bf16x8_nc(const float *x, bf16x8_t &hi, bf16x8_t &mid, bf16x8_t &lo) {
#pragma clang fp contract(off)
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const f32x2_t v = {x[e], x[e + 1]};
    const bf16x2_t h = __builtin_convertvector(v, bf16x2_t);
    const f32x2_t r1 = v - __builtin_convertvector(h, f32x2_t);
    const bf16x2_t m = __builtin_convertvector(r1, bf16x2_t);
    const f32x2_t r2 = r1 - __builtin_convertvector(m, f32x2_t);
    const bf16x2_t l = __builtin_convertvector(r2, bf16x2_t);
    hi[e] = h[0]; hi[e + 1] = h[1];
    mid[e] = m[0]; mid[e + 1] = m[1];
    lo[e] = l[0]; lo[e + 1] = l[1];
  }
}

// Offset of X element (m, k) in the matrix-core GEMMs (k a multiple of 4 inside one 32-wide
// k step, which never straddles an X segment).
__device__ __forceinline__ size_t gemm_x_offset(const GemmArgs &a, int m, int k) {
  size_t o = (size_t)m * a.ldx;
  if (a.xseg_len > 0) o += (size_t)(k / a.xseg_len) * a.xseg_stride + k % a.xseg_len;
  else o += k;
  return o;
}

// Epilogues of the matrix-core GEMMs for element (m, n) with accumulated value v (not SwiGLU).
template <int EPI>
__device__ __forceinline__ float gemm_epilogue(const GemmArgs &a, int m, int n, float v) {
  if constexpr (EPI == EPI_RESIDUAL) v = a.res[(size_t)m * a.ldr + n] + v;
  if constexpr (EPI == EPI_BIAS) v = v + a.bias[n];
  if constexpr (EPI == EPI_AFFINE_RES) {
    if (a.bias) v = v + a.bias[n];
    if (a.scale) v = v * a.scale[n];
    v = a.res[(size_t)m * a.ldr + n] + v;
  }
  if constexpr (EPI == EPI_BIAS_GELU) {
    v = v + a.bias[n];
    v = 0.5f * v * (1.0f + erff(v * 0.7071067811865476f));
  }
  return v;
}

// gemm_epilogue with its operands loaded beforehand: r = res[m][n], b = bias[n] (when
// given), c = scale[n] (when given); the same arithmetic in the same order.
template <int EPI>
__device__ __forceinline__ float gemm_epilogue_ops(const GemmArgs &a, float v, float r, float b, float c) {
  if constexpr (EPI == EPI_RESIDUAL) v = r + v;
  if constexpr (EPI == EPI_BIAS) v = v + b;
  if constexpr (EPI == EPI_AFFINE_RES) {
    if (a.bias) v = v + b;
    if (a.scale) v = v * c;
    v = r + v;
  }
  if constexpr (EPI == EPI_BIAS_GELU) {
    v = v + b;
    v = 0.5f * v * (1.0f + erff(v * 0.7071067811865476f));
  }
  return v;
}

template <int EPI, int MB, int NB>
__global__ __launch_bounds__(256) void k_gemm_mfma(GemmArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15;   // row (A) / column (B, C) within a 16-tile
  const int kb = lane >> 4;   // k-block of 8 within the 32-wide k step
  constexpr int NTILE = (EPI == EPI_SWIGLU) ? NB / 2 : NB;  // output column tiles
  const int m0 = blockIdx.y * 16 * MB;
  const int n0 = (blockIdx.x * 4 + wave) * 16 * NTILE;  // first output column of this wave
  if (n0 >= a.N) return;
  // split z of gridDim.z: k steps [kt0, kt1) of 32
  const int KT = a.K / 32, nsplit = gridDim.z, z = blockIdx.z;
  const int kt0 = (int)((int64_t)KT * z / nsplit), kt1 = (int)((int64_t)KT * (z + 1) / nsplit);

  f32x4_t acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // rows / weight rows this lane feeds (clamped into range; padding results are not stored)
  int arow[MB];
  float rscale[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    arow[i] = min(m0 + 16 * i + li, a.M - 1);
    rscale[i] = a.row_scale ? a.row_scale[arow[i]] : 1.f;
  }
  int wrow[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    int col;
    if constexpr (EPI == EPI_SWIGLU)
      col = (j < NTILE) ? n0 + 16 * j + li : a.N + n0 + 16 * (j - NTILE) + li;
    else
      col = n0 + 16 * j + li;
    const int lim = (EPI == EPI_SWIGLU) ? 2 * a.N : a.N;
    wrow[j] = min(col, lim - 1);
  }

  for (int k0 = kt0 * 32; k0 < kt1 * 32; k0 += 32) {
    const int k = k0 + 8 * kb;
    float xa[MB][8];
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      const float4 *px = reinterpret_cast<const float4 *>(a.X + gemm_x_offset(a, arow[i], k));
      const float4 p0 = px[0], p1 = px[1];
      xa[i][0] = p0.x; xa[i][1] = p0.y; xa[i][2] = p0.z; xa[i][3] = p0.w;
      xa[i][4] = p1.x; xa[i][5] = p1.y; xa[i][6] = p1.z; xa[i][7] = p1.w;
    }
    uint4 wb[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) wb[j] = *reinterpret_cast<const uint4 *>(a.W + (size_t)wrow[j] * a.K + k);
    float g[8];
    if (a.gamma) {
      const float4 *pg = reinterpret_cast<const float4 *>(a.gamma + k);
      const float4 g0 = pg[0], g1 = pg[1];
      g[0] = g0.x; g[1] = g0.y; g[2] = g0.z; g[3] = g0.w; g[4] = g1.x; g[5] = g1.y; g[6] = g1.z; g[7] = g1.w;
    }
    bf16x8_t ahi[MB], amid[MB], alo[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      if (a.gamma) {
#pragma unroll
        for (int e = 0; e < 8; ++e) xa[i][e] = (xa[i][e] * rscale[i]) * g[e];
      } else if (a.row_scale) {
#pragma unroll
        for (int e = 0; e < 8; ++e) xa[i][e] = xa[i][e] * rscale[i];
      }
      split_bf16x8(xa[i], ahi[i], amid[i], alo[i]);
    }
    // term-major (lo, mid, hi over all tiles): independent accumulations between two that depend
    // on each other
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int i = 0; i < MB; ++i)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(alo[i], __builtin_bit_cast(bf16x8_t, wb[j]), acc[i][j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int i = 0; i < MB; ++i)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(amid[i], __builtin_bit_cast(bf16x8_t, wb[j]), acc[i][j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int i = 0; i < MB; ++i)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ahi[i], __builtin_bit_cast(bf16x8_t, wb[j]), acc[i][j], 0, 0, 0);
  }

  // epilogue: lane holds C[4 * kb + e][li] of every tile
  // The epilogue's operands are loaded before the first store (Y may be the residual itself:
  // a load after a store that may alias it would wait for that store).
  constexpr bool RES = EPI == EPI_RESIDUAL || EPI == EPI_AFFINE_RES;
  constexpr bool BIAS = EPI == EPI_BIAS || EPI == EPI_AFFINE_RES || EPI == EPI_BIAS_GELU;
  constexpr bool OPS = RES || BIAS;
  float rv[OPS ? MB : 1][OPS ? NTILE : 1][4], bv[OPS ? NTILE : 1], cv[OPS ? NTILE : 1];
  if constexpr (OPS) {
    if (nsplit == 1) {
#pragma unroll
      for (int j = 0; j < NTILE; ++j) {
        const int nc = min(n0 + 16 * j + li, a.N - 1);
        bv[j] = (BIAS && (EPI != EPI_AFFINE_RES || a.bias)) ? a.bias[nc] : 0.f;
        cv[j] = (EPI == EPI_AFFINE_RES && a.scale) ? a.scale[nc] : 1.f;
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            rv[i][j][e] = RES ? a.res[(size_t)min(m0 + 16 * i + 4 * kb + e, a.M - 1) * a.ldr + nc] : 0.f;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NTILE; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + 16 * i + 4 * kb + e;
        const int n = n0 + 16 * j + li;
        if (m >= a.M || n >= a.N) continue;
        float v = acc[i][j][e];
        if constexpr (EPI == EPI_SWIGLU) {
          const float u = acc[i][j + NTILE][e];
          if (nsplit > 1) {  // raw gate and up sums: [split][M][2N], up at N + n
            float *w = a.split_ws + ((size_t)z * a.M + m) * 2 * a.N;
            w[n] = v;
            w[a.N + n] = u;
            continue;
          }
          v = v / (1.0f + expf(-v)) * u;
        } else {
          if (nsplit > 1) {
            a.split_ws[((size_t)z * a.M + m) * a.N + n] = v;
            continue;
          }
          if constexpr (OPS) v = gemm_epilogue_ops<EPI>(a, v, rv[i][j][e], bv[j], cv[j]);
        }
        a.Y[(size_t)m * a.ldy + n] = v;
      }
}

// ---------------------------------------------------------------------------------------
// Skinny GEMM for M <= 16 rows (one row per stream in batched decode): one 1024-thread
// workgroup per 16-column output tile (a gate tile + up tile pair for SwiGLU); its 16 waves
// split K into contiguous ranges, issue every load of their range up front, run the three
// bf16-term MFMAs, and the 16 partial tiles are summed in wave order through LDS.  With
// NORM the rows' RMSNorm is computed from the same loads (sum of squares reduced across the
// workgroup) and applied before the split.
// ---------------------------------------------------------------------------------------
// ---------------------------------------------------------------------------------------
// Prefill GEMM, LDS-tiled: Y[M][N] = f(X)[M][K] . W[N][K]^T for many rows.
// Block tile 128 rows x 128 weight rows, k step 32; four waves, each 32 rows x 128 weight rows
// (2 x 8 tiles of v_mfma_f32_16x16x32_bf16), two blocks per CU.  Each wave's X rows are its
// own: it loads them from global memory in matrix-core fragment order, scales them by the
// row's 1/rms and the gain, and splits them in registers into the hi/mid/lo bf16 terms of
// k_gemm_mfma.  Only the weight tile, shared by the four waves, goes through LDS (double
// buffered, in fragment order: conflict-free 16-byte reads).  Global loads of the next k step
// are in flight while the matrix cores work on this one.  SwiGLU blocks hold 64 gate rows and
// the matching 64 up rows (64 outputs).  Requires K % 32 == 0 (and N % 64 == 0 for SwiGLU); a
// partial last block of columns computes clamped weight rows and stores only columns below N.
// XS: bit 0 = GemmArgs::row_scale given, bit 1 = gamma given (compile-time, so that the k
// loop is one basic block).  BW = 96 (not SwiGLU): 96-column blocks, for N a multiple of 96
// but not of 128 (the codec's 96- and 192-channel convolutions), where 128-column blocks
// would leave a quarter of the matrix-core work on padding columns.
// ---------------------------------------------------------------------------------------
template <int EPI, int XS, int BW = 128>
__global__ __launch_bounds__(256, 2) void k_gemm_lds(GemmArgs a) {
  constexpr int BM = 128, BK = 32;
  constexpr bool SW = EPI == EPI_SWIGLU;
  static_assert(BW == 128 || (BW == 96 && !SW), "column block");
  constexpr int NU = BW / 16;  // 16-column tiles per block
  constexpr bool RS = XS & 1, GM = XS & 2;
  // weight tile u (rows 16 u .. 16 u + 15 of the block) at Bs[buf][u]; lane li + 16 kb reads
  // row 16 u + li, k = 8 kb .. 8 kb + 7, from entry 16 kb + (li ^ 4 kb).  The xor spreads the
  // stores (four lanes of one row, k = 0 .. 31, see below) over distinct banks while every 16
  // lanes of a read still cover all 16 bank groups.
  __shared__ bf16x8_t Bs[2][BW / 16][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, kb = lane >> 4;
  // Block tile (mb, nb).  Workgroups go to the 8 XCDs round robin (linear id % 8), each with its
  // own L2.  With few column blocks (gridDim.x <= 8) that would send every row block of one
  // column block to the same XCD, which would then read all of X; instead each XCD takes a
  // contiguous range of row-major tiles (all column blocks of its row blocks), so its L2 reads
  // only its own X rows, once for all column blocks.
  int mb = blockIdx.y, nb = blockIdx.x;
  if (gridDim.x <= 8) {
    const int total = gridDim.x * gridDim.y, L = blockIdx.y * gridDim.x + blockIdx.x;
    const int xcd = L % 8, local = L / 8, C = (total + 7) / 8, r = total % 8;
    const int t = (r == 0 || xcd < r) ? xcd * C + local : r * C + (xcd - r) * (C - 1) + local;
    mb = t / gridDim.x;
    nb = t % gridDim.x;
  }
  const int m0 = mb * BM + wave * 32;  // this wave's rows m0 .. m0 + 31
  // split z of gridDim.z: k tiles [kt0, kt1)
  const int KT = a.K / BK, nsplit = gridDim.z, z = blockIdx.z;
  const int kt0 = (int)((int64_t)KT * z / nsplit), kt1 = (int)((int64_t)KT * (z + 1) / nsplit);

  // weight row of block row r (a partial last block of a non-SwiGLU GEMM repeats the last row;
  // its columns are not stored)
  auto wrow = [&](int r) -> int {
    if constexpr (SW) return r < 64 ? nb * 64 + r : a.N + nb * 64 + (r - 64);
    else return min(nb * BW + r, a.N - 1);
  };
  // X: lane (li, kb) reads rows m0 + 16 t + li, k = 8 kb .. 8 kb + 7 (two float4 per tile t).
  // W: thread tid reads block rows (tid + 256 i) / 4, k = 8 ((tid + 256 i) % 4) .. + 7 (four
  // consecutive lanes read one row's 64 contiguous bytes).
  // NCH 16-byte weight chunks per k step, NB per thread (the last one partial for BW = 96)
  constexpr int NCH = BW * BK / 8, NB = (NCH + 255) / 256, CB = BK / 8;
  const float *xp[2];
  float rs[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int m = min(m0 + 16 * t + li, a.M - 1);
    xp[t] = a.X + (size_t)m * a.ldx + 8 * kb;
    rs[t] = RS ? a.row_scale[m] : 1.0f;
  }
  const uint16_t *wp[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int idx = tid + 256 * i, row = idx / CB, c = idx % CB;
    wp[i] = a.W + (size_t)wrow(row) * a.K + 8 * c;
  }
  const float *gp = GM ? a.gamma + 8 * kb : nullptr;
  // X offset of the current k step and the k left in its segment (X rows in segments of
  // xseg_len, xseg_stride apart; a 32-wide step never straddles two): advanced per step
  int xk, xleft;
  {
    const int k = kt0 * BK;
    if (a.xseg_len > 0) {
      xk = (k / a.xseg_len) * a.xseg_stride + k % a.xseg_len;
      xleft = a.xseg_len - k % a.xseg_len;
    } else {
      xk = k;
      xleft = 1 << 30;
    }
  }
  float4 rx[2][2];  // X of the loaded step, [tile][half]
  float4 rg[2];     // gain of the loaded step
  bf16x8_t rb[NB];  // a native vector (a uint4 struct copy stays a memcpy through scratch in the IR)
  auto gload = [&](int k0) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int h = 0; h < 2; ++h) rx[t][h] = *reinterpret_cast<const float4 *>(xp[t] + xk + 4 * h);
    if constexpr (GM) {
      rg[0] = *reinterpret_cast<const float4 *>(gp + k0);
      rg[1] = *reinterpret_cast<const float4 *>(gp + k0 + 4);
    }
#pragma unroll
    for (int i = 0; i < NB; ++i)
      if (NCH % 256 == 0 || tid + 256 * i < NCH) rb[i] = *reinterpret_cast<const bf16x8_t *>(wp[i] + k0);
    const bool wrap = xleft == BK;
    xk += wrap ? BK + a.xseg_stride - a.xseg_len : BK;
    xleft = wrap ? a.xseg_len : xleft - BK;
  };
  bf16x8_t aq[3][2];  // [lo, mid, hi][tile] of the step the matrix cores work on next
  auto split = [&]() {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      float xv[8] = {rx[t][0].x, rx[t][0].y, rx[t][0].z, rx[t][0].w,
                     rx[t][1].x, rx[t][1].y, rx[t][1].z, rx[t][1].w};
      if constexpr (RS) {
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[e] *= rs[t];
      }
      if constexpr (GM) {
        const float gv[8] = {rg[0].x, rg[0].y, rg[0].z, rg[0].w, rg[1].x, rg[1].y, rg[1].z, rg[1].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[e] *= gv[e];
      }
      split_bf16x8_nc(xv, aq[2][t], aq[1][t], aq[0][t]);
    }
  };
  auto bstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int idx = tid + 256 * i, row = idx / CB, c = idx % CB;
      if (NCH % 256 == 0 || idx < NCH) Bs[buf][row >> 4][16 * c + ((row & 15) ^ (4 * c))] = rb[i];
    }
  };

  f32x4_t acc[2][NU];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int u = 0; u < NU; ++u) acc[t][u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto mma = [&](int buf) {
    bf16x8_t bq[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) bq[u] = Bs[buf][u][16 * kb + (li ^ (4 * kb))];
    // term-major: 16 independent accumulations between two that depend on each other;
    // each accumulator still adds lo, mid, hi in that order.
#pragma unroll
    for (int q = 0; q < 3; ++q)
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int u = 0; u < NU; ++u)
          acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aq[q][t], bq[u], acc[t][u], 0, 0, 0);
  };

  gload(kt0 * BK);
  split();
  bstore(0);
  __syncthreads();
  // all but the last k step: load the next step's operands, multiply this one, split and store
  // the next
  int buf = 0;
  for (int kt = kt0; kt < kt1 - 1; ++kt) {
    // without the fences the scheduler sinks the loads among the MFMAs and waits for them there
    gload((kt + 1) * BK);
    __builtin_amdgcn_sched_barrier(0);
    mma(buf);
    __builtin_amdgcn_sched_barrier(0);
    split();
    bstore(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }
  mma(buf);

  // C[i][j] of a tile sits in lane j + 16 (i / 4), element i % 4.
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = m0 + t * 16 + 4 * kb + e;
      if (m >= a.M) continue;
      if constexpr (SW) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int n = nb * 64 + u * 16 + li;
          const float g = acc[t][u][e], up = acc[t][u + 4][e];
          if (nsplit > 1) {  // raw gate and up sums: [split][M][2N], up at N + n
            float *w = a.split_ws + ((size_t)z * a.M + m) * 2 * a.N;
            w[n] = g;
            w[a.N + n] = up;
          } else {
            a.Y[(size_t)m * a.ldy + n] = g / (1.0f + expf(-g)) * up;
          }
        }
      } else if (nsplit > 1) {
#pragma unroll
        for (int u = 0; u < NU; ++u) {
          const int n = nb * BW + u * 16 + li;
          if (n < a.N) a.split_ws[((size_t)z * a.M + m) * a.N + n] = acc[t][u][e];
        }
      }
    }
  if constexpr (!SW) {
    if (nsplit > 1) return;
    // Every epilogue operand is loaded before the first store: Y may be the residual itself
    // (each element read and written by this lane only), and a load after a store that may
    // alias it would wait for that store, one memory round trip per element.
    constexpr bool RES = EPI == EPI_RESIDUAL || EPI == EPI_AFFINE_RES;
    constexpr bool BIAS = EPI == EPI_BIAS || EPI == EPI_AFFINE_RES || EPI == EPI_BIAS_GELU;
    float rv[2][4][RES ? NU : 1], bv[BIAS ? NU : 1], cv[EPI == EPI_AFFINE_RES ? NU : 1];
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int nc = min(nb * BW + u * 16 + li, a.N - 1);
      if constexpr (BIAS) bv[u] = (EPI != EPI_AFFINE_RES || a.bias) ? a.bias[nc] : 0.f;
      if constexpr (EPI == EPI_AFFINE_RES) cv[u] = a.scale ? a.scale[nc] : 1.f;
    }
    if constexpr (RES) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int u = 0; u < NU; ++u) {
            const int mc = min(m0 + t * 16 + 4 * kb + e, a.M - 1), nc = min(nb * BW + u * 16 + li, a.N - 1);
            rv[t][e][u] = a.res[(size_t)mc * a.ldr + nc];
          }
    }
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + t * 16 + 4 * kb + e;
        if (m >= a.M) continue;
#pragma unroll
        for (int u = 0; u < NU; ++u) {
          const int n = nb * BW + u * 16 + li;
          if (n >= a.N) continue;
          a.Y[(size_t)m * a.ldy + n] = gemm_epilogue_ops<EPI>(a, acc[t][u][e], RES ? rv[t][e][RES ? u : 0] : 0.f,
                                                              BIAS ? bv[BIAS ? u : 0] : 0.f,
                                                              EPI == EPI_AFFINE_RES ? cv[EPI == EPI_AFFINE_RES ? u : 0] : 1.f);
        }
      }
  }
}

// KEYS (EPI_STORE): store per-row argmax keys (GemmArgs::keys_out) instead of Y.  XT16: X is
// a T16 block (else row-major with leading dimension ldx).  W is always in k_pack_w's layout,
// in whole 16-column tiles (the last one padded).
// Both operand layouts are compile-time so that the load phase has no branch: a branch there
// makes the first MFMA wait for every load of the pass (vmcnt(0)) instead of its own step's.
// SPLIT (GemmArgs::split2): grid y = 2 halves of K, KS = K / (2 * 16 * 32); the halves meet
// in fp32 atomic adds on a zeroed T16 Y.
// MB = 2 (GemmArgs::mb): two 16-row blocks against one pass over W, the two positions of the
// same stream rows (row m of block b is stream row m, masked by row_on[m]).  T16 operands of
// block b start 16 * K (X) or 16 * N (Y, res, res_zero) elements after block 0; row-major ones
// x_blk / r_blk / y_blk elements after.
template <int EPI, bool NORM, int KS, bool KEYS = false, bool XT16 = true, bool SPLIT = false, int MB = 1,
          bool WNT = false>
__global__ __launch_bounds__(1024) void k_gemm_skinny(GemmArgs a) {
  static_assert(!KEYS || EPI == EPI_STORE, "keys replace the plain store");
  static_assert(!SPLIT || (EPI == EPI_RESIDUAL && !NORM && XT16), "the split GEMM is the T16 residual form");
  static_assert(MB == 1 || (MB == 2 && !KEYS), "two row blocks: no key store");
  constexpr int T = (EPI == EPI_SWIGLU) ? 2 : 1;
  constexpr int KW = KS * 32;  // k range per wave
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;  // 0..15
  const int li = lane & 15, kb = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int kbase = (SPLIT ? blockIdx.y * (a.K >> 1) : 0) + wave * KW;
  const int arow = min(li, a.M - 1);
  __shared__ f32x4_t part[16][MB * T][64];
  __shared__ float ssq[16][MB * 16];

  // Output (ob, om, on) of this thread's epilogue (threads 0 .. 256 MB - 1, one output each:
  // block ob, row om, column on).  Its residual / bias / row mask are loaded first so that the
  // epilogue waits on nothing.
  const int ot = threadIdx.x;
  const int ob = min(ot >> 8, MB - 1);
  const int ol = (ot & 255) >> 2, oe = ot & 3;
  const int om = 4 * (ol >> 4) + oe, on = n0 + (ol & 15);
  const int cm = min(om, a.M - 1), cn = min(on, a.N - 1);
  // A global load (never a flat one: a pending flat load makes every later wait a vmcnt(0)).
  int oflag = 1;
  if (a.row_on) oflag = a.row_on[cm];
  float oadd = 0.f;
  if constexpr (EPI == EPI_RESIDUAL)
    oadd = a.res[a.r_t16 ? (size_t)ob * 16 * a.N + t16_index(cm, cn) : (size_t)cm * a.ldr + (size_t)ob * a.r_blk + cn];
  if constexpr (EPI == EPI_BIAS) oadd = a.bias[cn];

  // k steps in passes of KP (all loads of a pass in flight together): registers for
  // KP <= 6 steps, so K = 512 * {8, 12} runs as two passes instead of spilling.
  constexpr int KP = KS <= 6 ? KS : (KS % 6 == 0 ? 6 : 4);
  static_assert(KS % KP == 0, "pass length");
  static_assert(!NORM || KS <= 4, "the fused RMSNorm keeps the whole row slice in registers");
  f32x4_t acc[MB][T];
#pragma unroll
  for (int b = 0; b < MB; ++b)
#pragma unroll
    for (int t = 0; t < T; ++t) acc[b][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // The RMSNorm gain of this wave's k range (KW <= 128 values): one load per lane and 64
  // values; each lane then takes its 8 values per k step by lane permutes (the 16 lanes of a
  // row share them), not by two 16-byte loads per step.
  constexpr int GL = NORM ? (KW + 63) / 64 : 1;
  float gl[GL];
  if constexpr (NORM) {
#pragma unroll
    for (int j = 0; j < GL; ++j) gl[j] = (64 * j + lane < KW) ? a.gamma[kbase + 64 * j + lane] : 0.f;
  }
#pragma unroll
  for (int p0 = 0; p0 < KS; p0 += KP) {
    float xa[MB][KP][8];
    float ga[NORM ? KP : 1][8];
    uint4 wb[KP][T];
#pragma unroll
    for (int st = 0; st < KP; ++st) {
      const int k0 = kbase + (p0 + st) * 32;
      const int k = k0 + 8 * kb;
#pragma unroll
      for (int b = 0; b < MB; ++b) {
        const float4 *px = reinterpret_cast<const float4 *>(
            XT16 ? a.X + (size_t)b * 16 * a.K + ((size_t)(k0 >> 5) * 64 + lane) * 8
                 : a.X + (size_t)arow * a.ldx + (size_t)b * a.x_blk + k);
        const float4 x0 = px[0], x1 = px[1];
        xa[b][st][0] = x0.x; xa[b][st][1] = x0.y; xa[b][st][2] = x0.z; xa[b][st][3] = x0.w;
        xa[b][st][4] = x1.x; xa[b][st][5] = x1.y; xa[b][st][6] = x1.z; xa[b][st][7] = x1.w;
      }
#pragma unroll
      for (int t = 0; t < T; ++t) {  // tile blockIdx.x (+ N / 16 for the up rows), k step k0 / 32
        const size_t tile = blockIdx.x + (size_t)t * (a.N >> 4);
        wb[st][t] = load_w<WNT>(reinterpret_cast<const u32x4 *>(a.W + ((tile * (a.K >> 5) + (k0 >> 5)) * 64 + lane) * 8));
      }
    }
    __builtin_amdgcn_sched_barrier(0);

    if constexpr (NORM) {  // single pass: this wave holds its whole k range of every row
#pragma unroll
      for (int st = 0; st < KP; ++st) {
        const int r = (p0 + st) * 32;  // this step's first value in the wave's range
#pragma unroll
        for (int e = 0; e < 8; ++e) ga[st][e] = __shfl(gl[(r + 8 * kb + e) >> 6], (r + 8 * kb + e) & 63, 64);
      }
      // RMSNorm(x) W^T = r (x * g) W^T with r = 1 / rms(x) one scalar per row: the products
      // take x * g, and r multiplies the sums in the epilogue.  Each wave leaves its rows'
      // sums of squares in ssq; the reduction's barrier then covers them too, so no wave
      // waits for the others' activation loads before its matrix-core work.
#pragma unroll
      for (int b = 0; b < MB; ++b) {
        float ss = 0.f;
#pragma unroll
        for (int st = 0; st < KP; ++st)
#pragma unroll
          for (int e = 0; e < 8; ++e) ss = fmaf(xa[b][st][e], xa[b][st][e], ss);
        ss = pair16_sum(ss);  // the four lanes of a row (kb = 0..3)
        ss = pair32_sum(ss);
        if (kb == 0) ssq[wave][b * 16 + li] = ss;
#pragma unroll
        for (int st = 0; st < KP; ++st)
#pragma unroll
          for (int e = 0; e < 8; ++e) xa[b][st][e] = xa[b][st][e] * ga[st][e];
      }
    }

#pragma unroll
    for (int st = 0; st < KP; ++st) {
#pragma unroll
      for (int b = 0; b < MB; ++b) {
        bf16x8_t hi, mid, lo;
        split_bf16x8(xa[b][st], hi, mid, lo);
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const bf16x8_t w = __builtin_bit_cast(bf16x8_t, wb[st][t]);
          acc[b][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo, w, acc[b][t], 0, 0, 0);
          acc[b][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mid, w, acc[b][t], 0, 0, 0);
          acc[b][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi, w, acc[b][t], 0, 0, 0);
        }
      }
    }
  }
#pragma unroll
  for (int b = 0; b < MB; ++b)
#pragma unroll
    for (int t = 0; t < T; ++t) part[wave][b * T + t][lane] = acc[b][t];
  __syncthreads();
  if (ot >= 256 * MB) return;
  // Sum of the 16 waves' k ranges in wave order (C[i][j] sits in lane j + 16 (i / 4),
  // element i % 4: this thread's (om, on) is lane ol, element oe).
  float v[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    float sacc = part[0][ob * T + t][ol][oe];
#pragma unroll
    for (int w = 1; w < 16; ++w) sacc += part[w][ob * T + t][ol][oe];
    v[t] = sacc;
  }
  if constexpr (NORM) {  // the row's 1 / rms from the 16 waves' sums of squares, in wave order
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < 16; ++w) tot += ssq[w][ob * 16 + cm];
    const float r = 1.0f / sqrtf(tot / (float)a.K + a.eps);
#pragma unroll
    for (int t = 0; t < T; ++t) v[t] *= r;
  }
  if constexpr (KEYS) {
    // The 16 columns of row om sit in lanes oe + 4c (c = 0..15) of one wave: their largest
    // key, in every one of those lanes, then stored by lane oe.
    uint64_t key = (om < a.M && on < a.N) ? order_key(v[0], on) : 0;
    key = umax64(key, lane_xor_u64<4>(key));
    key = umax64(key, lane_xor_u64<8>(key));
    key = umax64(key, lane_xor_u64<16>(key));
    key = umax64(key, lane_xor_u64<32>(key));
    if ((ol & 15) == 0 && om < a.M && oflag) a.keys_out[om * a.keys_row + blockIdx.x] = key;
    return;
  }
  if (om >= a.M || on >= a.N || !oflag) return;
  float y = v[0];
  if constexpr (SPLIT) {
    const size_t oi = (size_t)ob * 16 * a.N + t16_index(om, on);
    if (blockIdx.y == 0) {
      y = oadd + y;
      a.res_zero[oi] = 0.f;  // after this thread's own residual read (res_zero may be res)
    }
    unsafeAtomicAdd(a.Y + oi, y);
    return;
  }
  if constexpr (EPI == EPI_SWIGLU) {
    y = y / (1.0f + expf(-y)) * v[T - 1];
  } else if constexpr (EPI == EPI_RESIDUAL || EPI == EPI_BIAS) {
    y = (EPI == EPI_RESIDUAL) ? oadd + y : y + oadd;
  }
  a.Y[a.y_t16 ? (size_t)ob * 16 * a.N + t16_index(om, on) : (size_t)om * a.ldy + (size_t)ob * a.y_blk + on] = y;
}

// inv_rms[m] = 1 / sqrt(mean(X[m]^2) + eps), one wave per row.
__global__ __launch_bounds__(256) void k_row_rms(const float *X, int ldx, int M, int K, float eps, float *inv_rms) {
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= M) return;
  float ss = 0.f;
  for (int k = lane; k < K; k += 64) ss = fmaf(X[(size_t)m * ldx + k], X[(size_t)m * ldx + k], ss);
  ss = wave_sum(ss);
  if (lane == 0) inv_rms[m] = 1.0f / sqrtf(ss / (float)K + eps);
}

// ---------------------------------------------------------------------------------------
// Prompt prefill attention over every stream's prompt rows at once, rows at positions
// 0..P-1 of their stream (decode.rs:1077-1298 with the cache written first and read back, the
// same values the decode steps read).  Segment s holds rows row0[s] .. row0[s] + P[s] - 1.
//   k_prefill_qkv: per (row, head vector): q/k head RMSNorm + RoPE at the row's position
//     (q written back in place), K and V stored into the row's stream cache.  One wave per
//     vector.
//   k_attn_prefill: per (stream, query head, 16-row query block): causal attention over
//     the stream's cache rows on the fp32 matrix cores, one wave per unit.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ int prefill_segment(const PrefillBatchArgs &a, int row) {
  int s = 0;
  while (s + 1 < a.nseg && row >= a.row0[s + 1]) ++s;
  return s;
}

template <typename KVT>
__global__ __launch_bounds__(256) void k_prefill_qkv(PrefillBatchArgs a) {
  constexpr int D = 128;
  const int lane = threadIdx.x & 63;
  const int vec = blockIdx.x * 4 + (threadIdx.x >> 6);  // q heads, then k heads, then v heads
  const int r = blockIdx.y;
  const int nvec = a.q_heads + 2 * a.kv_heads;
  if (vec >= nvec || r >= a.M) return;
  const int sg = prefill_segment(a, r);
  const int pos = r - a.row0[sg];
  float *row = a.qkv + (size_t)r * a.ldq;
  float *v = row + vec * D;
  float x0 = v[lane], x1 = v[lane + 64];
  if (vec < a.q_heads + a.kv_heads) {
    const float *gain = vec < a.q_heads ? a.gq : a.gk;
    const float ss = wave_sum(fmaf(x0, x0, x1 * x1));
    const float inv = 1.0f / sqrtf(ss / (float)D + a.eps);
    x0 = (x0 * inv) * gain[lane];
    x1 = (x1 * inv) * gain[lane + 64];
    const float2 cs = a.rope[(size_t)pos * (D / 2) + lane];
    const float r0 = x0 * cs.x - x1 * cs.y, r1 = x1 * cs.x + x0 * cs.y;
    x0 = r0;
    x1 = r1;
  }
  if (vec < a.q_heads) {
    v[lane] = x0;
    v[lane + 64] = x1;
  } else {
    const bool is_k = vec < a.q_heads + a.kv_heads;
    const int h = is_k ? vec - a.q_heads : vec - a.q_heads - a.kv_heads;
    KVT *cache = reinterpret_cast<KVT *>(is_k ? a.kcache[sg] : a.vcache[sg]) + ((size_t)h * a.cap + pos) * D;
    KvIo<KVT>::store(cache + lane, x0);
    KvIo<KVT>::store(cache + lane + 64, x1);
  }
}

// Prefill of a few rows at positions 0 .. P-1 (the CodePredictor's 2-row prefix) in one
// workgroup per KV head: q/k head RMSNorm + RoPE, K/V stores, then each row's causal
// attention over rows 0..p with the values just stored (rounded to the cache type).  The
// P * (G + 2) head vectors are spread over the 4 waves, loads first.
// OPROJ: the output projection fused in as in k_attn_split (grid (kv_heads, wo_rows / 32));
// row p's per-head shares go to opart + p * opart_row + h * wo_rows.  Only row block 0 stores
// the K/V rows.
// ROWS: stream rows (PrefillAttnArgs::ld_pos ..), grid (kv_heads, 1, rows); the output goes to
// T16 blocks, one per position.
template <int G, typename KVT, int P, bool OPROJ = false, bool ROWS = false>
__global__ __launch_bounds__(256) void k_attn_prefix(PrefillAttnArgs a) {
  static_assert(!(OPROJ && ROWS), "stream rows take the unfused form");
  constexpr int D = 128, NV = P * (G + 2), VPW = (NV + 3) / 4;
  const int h = blockIdx.x;
  const int rb = OPROJ ? blockIdx.y : 0;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = ROWS ? blockIdx.z : 0;
  if constexpr (ROWS) {
    a.qkv += (size_t)row * a.ldq;
    a.kcache = reinterpret_cast<KVT *>(a.kcache) + row * a.kv_row;
    a.vcache = reinterpret_cast<KVT *>(a.vcache) + row * a.kv_row;
  }
  const int64_t ld_pos = ROWS ? a.ld_pos : a.ldq;
  __shared__ float qs[P][G][D], ks[P][D], vs[P][D];
  __shared__ float sc[P][G][P];
  __shared__ float ao[OPROJ ? P : 1][G * D];
  constexpr int LPR = G * D / 8;
  constexpr int RPL = 64 / LPR;
  constexpr int NWO = OPROJ ? kOprojRows / 4 / RPL : 1;
  uint4 wo[NWO];
  if constexpr (OPROJ) {
#pragma unroll
    for (int i = 0; i < NWO; ++i) {
      const int r = rb * kOprojRows + wave * (kOprojRows / 4) + i * RPL + lane / LPR;
      wo[i] = *reinterpret_cast<const uint4 *>(a.wo + (size_t)r * a.q_heads * D + h * G * D + (lane % LPR) * 8);
    }
  }
  float x0[VPW], x1[VPW], g0[VPW], g1[VPW];
  float2 cs[VPW];
#pragma unroll
  for (int i = 0; i < VPW; ++i) {
    const int vi = min(wave + 4 * i, NV - 1);  // vector vi: row vi / (G + 2), kind vi % (G + 2)
    const int p = vi / (G + 2), kind = vi % (G + 2);
    const int off = kind < G ? (h * G + kind) * D
                             : (kind == G ? a.q_heads * D + h * D : (a.q_heads + a.kv_heads) * D + h * D);
    const float *src = a.qkv + (size_t)p * ld_pos + off;
    x0[i] = src[lane];
    x1[i] = src[lane + 64];
    const float *gain = kind < G ? a.gq : a.gk;  // unused for v
    g0[i] = gain[lane];
    g1[i] = gain[lane + 64];
    cs[i] = a.rope[(size_t)p * (D / 2) + lane];
  }
  if constexpr (ROWS) {  // workgroup-uniform, after the loads (valid for any state)
    if (a.row_on && !a.row_on[row]) return;
    if (skip_work(a.st + row, SKIP_DONE)) return;
  }
#pragma unroll
  for (int i = 0; i < VPW; ++i) {
    const int vi = wave + 4 * i;
    if (vi >= NV) break;  // wave-uniform
    const int p = vi / (G + 2), kind = vi % (G + 2);
    float y0 = x0[i], y1 = x1[i];
    if (kind <= G) {
      const float ss = wave_sum(fmaf(y0, y0, y1 * y1));
      const float inv = 1.0f / sqrtf(ss / (float)D + a.eps);
      y0 = (y0 * inv) * g0[i];
      y1 = (y1 * inv) * g1[i];
      const float r0 = y0 * cs[i].x - y1 * cs[i].y, r1 = y1 * cs[i].x + y0 * cs[i].y;
      y0 = r0;
      y1 = r1;
    }
    if (kind < G) {
      qs[p][kind][lane] = y0;
      qs[p][kind][lane + 64] = y1;
    } else {
      KVT *cache = reinterpret_cast<KVT *>(kind == G ? a.kcache : a.vcache) + ((size_t)h * a.cap + p) * D;
      float *keep = kind == G ? ks[p] : vs[p];
      if (rb == 0) {
        keep[lane] = KvIo<KVT>::store(cache + lane, y0);
        keep[lane + 64] = KvIo<KVT>::store(cache + lane + 64, y1);
      } else {
        keep[lane] = KvIo<KVT>::round(y0);
        keep[lane + 64] = KvIo<KVT>::round(y1);
      }
    }
  }
  __syncthreads();
  // scores: 16 lanes per (row, head, key) triple, 8 dims each
  constexpr int NT = P * G * P;
  const int sub = lane & 15, grp = (int)threadIdx.x >> 4;
  for (int tr = grp; tr < NT; tr += 16) {
    const int p = tr / (G * P), g = (tr / P) % G, t = tr % P;
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc = fmaf(qs[p][g][sub * 8 + j], ks[t][sub * 8 + j], acc);
    acc = row16_sum(acc);
    if (sub == 0) sc[p][g][t] = acc * a.scale;
  }
  __syncthreads();
  // outputs: row p, head g, dim d; softmax over keys 0..p in key order
  for (int o = threadIdx.x; o < P * G * D; o += 256) {
    const int p = o / (G * D), g = (o / D) % G, d = o % D;
    float m = -FLT_MAX;
    for (int t = 0; t <= p; ++t) m = fmaxf(m, sc[p][g][t]);
    float l = 0.f, acc = 0.f;
    for (int t = 0; t <= p; ++t) {
      const float w = expf(sc[p][g][t] - m);
      l += w;
      acc = fmaf(w, vs[t][d], acc);
    }
    if constexpr (OPROJ)
      ao[p][g * D + d] = acc / l;
    else if constexpr (ROWS)
      a.out[(size_t)p * 16 * a.ldo + t16_index(row, (h * G + g) * D + d)] = acc / l;
    else
      a.out[(size_t)p * a.ldo + (h * G + g) * D + d] = acc / l;
  }
  if constexpr (OPROJ) {
    __syncthreads();
    // every (row, position) sum first, then the stores (one basic block: the chains interleave)
    float sum[NWO][P];
#pragma unroll
    for (int i = 0; i < NWO; ++i)
#pragma unroll
      for (int p = 0; p < P; ++p) {
        sum[i][p] = row16_sum(dot8(wo[i], ao[p] + (lane % LPR) * 8));
        if constexpr (LPR == 32) sum[i][p] += dpp_f<0x142, 0xa>(sum[i][p], 0.f);
      }
    if (lane % LPR == LPR - 1) {
#pragma unroll
      for (int i = 0; i < NWO; ++i) {
        const int r = rb * kOprojRows + wave * (kOprojRows / 4) + i * RPL + lane / LPR;
#pragma unroll
        for (int p = 0; p < P; ++p) a.opart[p * a.opart_row + (size_t)h * a.wo_rows + r] = sum[i][p];
      }
    }
  }
}

// One wave per unit (stream s, query head hq, query rows q0 .. q0 + 15), units in
// PrefillBatchArgs::unit0 order: per stream, the last query block first (the longest causal
// range).  v_mfma_f32_16x16x4_f32 (fp32 products and sums):
//   S^T = K Q^T per 16-key tile: lane (li, kk) supplies key row li and query row li, dims
//     32 kk + s at step s (32 steps: the four lane groups cover the 128 dims in quarters), and
//     holds scores of keys 4 kk + e (e = 0..3) for query li.
//   O^T += V^T P^T: step s' takes keys 4 kk + s' (lane group kk), so each lane's own score
//     e = s' is its B operand; A row i of output tile t is dim 8 i + t, so a lane reads 8
//     consecutive floats of a value row and ends up holding dims 32 kk .. 32 kk + 31 of query li.
//   Online softmax per query over 16-key tiles: the tile max over the four lane groups by lane
//     exchanges, per-lane partial sums of p (added across the groups at the end).
template <typename KVT>
__global__ __launch_bounds__(256) void k_attn_prefill(PrefillBatchArgs a) {
  constexpr int D = 128;
  const int lane = threadIdx.x & 63, li = lane & 15, kk = lane >> 4;
  const int u = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (u >= a.unit0[a.nseg]) return;
  int sg = 0;
  while (sg + 1 < a.nseg && u >= a.unit0[sg + 1]) ++sg;
  const int P = a.P[sg], local = u - a.unit0[sg];
  const int nqb = (P + 15) / 16;
  const int hq = local % a.q_heads, q0 = 16 * (nqb - 1 - local / a.q_heads);
  const int kvh = hq / (a.q_heads / a.kv_heads);
  const float *qkv = a.qkv + (size_t)a.row0[sg] * a.ldq;
  const KVT *kb = reinterpret_cast<const KVT *>(a.kcache[sg]) + (size_t)kvh * a.cap * D;
  const KVT *vb = reinterpret_cast<const KVT *>(a.vcache[sg]) + (size_t)kvh * a.cap * D;

  float q[32];
  {
    const float *qp = qkv + (size_t)min(q0 + li, P - 1) * a.ldq + hq * D + 32 * kk;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4 x0 = reinterpret_cast<const float4 *>(qp + 8 * c)[0];
      const float4 x1 = reinterpret_cast<const float4 *>(qp + 8 * c)[1];
      q[8 * c] = x0.x; q[8 * c + 1] = x0.y; q[8 * c + 2] = x0.z; q[8 * c + 3] = x0.w;
      q[8 * c + 4] = x1.x; q[8 * c + 5] = x1.y; q[8 * c + 6] = x1.z; q[8 * c + 7] = x1.w;
    }
  }
  f32x4_t o[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) o[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -FLT_MAX, l_part = 0.f;
  const int qrow = q0 + li;                      // this lane's query (rows >= P are not stored)
  const int nkt = (min(q0 + 16, P) + 15) / 16;   // key tiles up to the block's last row
  for (int kt = 0; kt < nkt; ++kt) {
    float kv[32];
    {
      const KVT *kp = kb + (size_t)min(16 * kt + li, P - 1) * D + 32 * kk;
#pragma unroll
      for (int c = 0; c < 4; ++c) KvIo<KVT>::load8(kp + 8 * c, kv + 8 * c);
    }
    float vv[4][8];
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2) KvIo<KVT>::load8(vb + (size_t)min(16 * kt + 4 * kk + s2, P - 1) * D + 8 * li, vv[s2]);
    f32x4_t st = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s1 = 0; s1 < 32; ++s1) st = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[s1], q[s1], st, 0, 0, 0);
    float p[4], mt = -FLT_MAX;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int key = 16 * kt + 4 * kk + e;
      p[e] = (key <= qrow && key < P) ? st[e] * a.scale : -FLT_MAX;
      mt = fmaxf(mt, p[e]);
    }
    mt = fmaxf(mt, __builtin_bit_cast(float, lane_xor_u32<16>(__builtin_bit_cast(uint32_t, mt))));
    mt = fmaxf(mt, __builtin_bit_cast(float, lane_xor_u32<32>(__builtin_bit_cast(uint32_t, mt))));
    const float m_new = fmaxf(m_run, mt);
    const float corr = expf(m_run - m_new);
    float ps = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      p[e] = p[e] == -FLT_MAX ? 0.f : expf(p[e] - m_new);
      ps += p[e];
    }
    l_part = l_part * corr + ps;
    m_run = m_new;
#pragma unroll
    for (int t = 0; t < 8; ++t) o[t] *= corr;
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2)
#pragma unroll
      for (int t = 0; t < 8; ++t) o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[s2][t], p[s2], o[t], 0, 0, 0);
  }
  float l = l_part;
  l += __builtin_bit_cast(float, lane_xor_u32<16>(__builtin_bit_cast(uint32_t, l)));
  l += __builtin_bit_cast(float, lane_xor_u32<32>(__builtin_bit_cast(uint32_t, l)));
  if (qrow >= P) return;
  const float inv = 1.0f / l;
  float *op = a.out + (size_t)(a.row0[sg] + qrow) * a.ldo + hq * D + 32 * kk;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    reinterpret_cast<float4 *>(op + 8 * e)[0] = make_float4(o[0][e] * inv, o[1][e] * inv, o[2][e] * inv, o[3][e] * inv);
    reinterpret_cast<float4 *>(op + 8 * e)[1] = make_float4(o[4][e] * inv, o[5][e] * inv, o[6][e] * inv, o[7][e] * inv);
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

struct alignas(16) SelectShared {
  float lg[kMaxVocab];
  float cv[kMaxVocab];
  int ci[kMaxVocab];
  float sv[kMaxVocab];
  int si[kMaxVocab];
  uint32_t hist[256];
  uint32_t whist[16][256];  // per-wave histograms of a radix pass
  uint32_t skey[64];        // the keys of a radix bin resolved directly
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

// Inclusive prefix sums across a wave (lane order).
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t o = (uint32_t)__shfl_up((int)v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

__device__ __forceinline__ float wave_incl_scan(float v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const float o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

// ---- top-k sampling for 1 <= top_k <= 64 and V <= 2048 (the CodePredictor's heads) ----
// Candidate key: (value's order bits << 32) | (2^32 - 1 - index) for a finite value (-0 as
// +0), 0 otherwise, so that larger keys rank first by (value desc, index asc), the order
// block_sample ranks candidates in.
__device__ __forceinline__ uint64_t sample_key(float v, int idx) {
  if (!isfinite(v)) return 0;
  uint32_t u = __float_as_uint(v);
  if (u == 0x80000000u) u = 0;
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | (uint64_t)(0xffffffffu - (uint32_t)idx);
}
__device__ __forceinline__ float sample_key_value(uint64_t key) {
  const uint32_t u = (uint32_t)(key >> 32);
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}
// Compare-exchange across lanes l and l ^ J: keep the larger key where keep_max.
template <int J>
__device__ __forceinline__ uint64_t wave_cx_u64(uint64_t v, bool keep_max) {
  const uint64_t o = lane_xor_u64<J>(v);
  return keep_max ? (v > o ? v : o) : (v < o ? v : o);
}
__device__ __forceinline__ uint64_t wave_cx_u64(uint64_t v, int j, bool keep_max) {
  switch (j) {
    case 1: return wave_cx_u64<1>(v, keep_max);
    case 2: return wave_cx_u64<2>(v, keep_max);
    case 4: return wave_cx_u64<4>(v, keep_max);
    case 8: return wave_cx_u64<8>(v, keep_max);
    case 16: return wave_cx_u64<16>(v, keep_max);
    default: return wave_cx_u64<32>(v, keep_max);
  }
}
// Bitonic sort of the wave's E * 64 keys (key[e] of lane l at position e * 64 + l), descending.
template <int E>
__device__ void wave_sort_desc(uint64_t (&key)[E]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 2; k <= 64 * E; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j >= 1; j >>= 1) {
      if (j >= 64) {  // partners in the same lane
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const int je = j >> 6;
          if (e & je) continue;
          const bool desc = ((e * 64 + lane) & k) == 0;
          const uint64_t x = key[e], y = key[e | je];
          key[e] = (x > y) == desc ? x : y;
          key[e | je] = (x > y) == desc ? y : x;
        }
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const bool desc = ((e * 64 + lane) & k) == 0;
          key[e] = wave_cx_u64(key[e], j, ((lane & j) == 0) == desc);
        }
      }
    }
  }
}
// The 64 largest of two descending 64-key lists a (lane i: a[i]) and b (lane i: b[63 - i]),
// descending: max(a[i], b[63 - i]) is a bitonic sequence holding them, then a bitonic merge.
__device__ __forceinline__ uint64_t wave_merge_top64(uint64_t a, uint64_t b_rev) {
  const int lane = threadIdx.x & 63;
  uint64_t v = a > b_rev ? a : b_rev;
#pragma unroll
  for (int j = 32; j >= 1; j >>= 1) v = wave_cx_u64(v, j, (lane & j) == 0);
  return v;
}

// block_sample for 1 <= top_k <= 64, V <= 2048 (1024 threads): each wave sorts its 128 keys,
// a four-level merge tree keeps the 64 largest, and wave 0 draws from the first k as
// block_sample does (the same weights, the same prefix sums in the same order, the same
// top-p cut and inverse CDF), so it returns the same token for the same u.
__device__ int block_sample_top64(SelectShared &sh, int V, const SamplingParams &sp, float u) {
  constexpr int E = 2;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint64_t key[E];
  int nf = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = (wave * E + e) * 64 + lane;
    key[e] = i < V ? sample_key(sh.lg[i], i) : 0;
    nf += key[e] != 0;
  }
  wave_sort_desc<E>(key);
  uint64_t *buf = reinterpret_cast<uint64_t *>(sh.cv);  // [2][16][64] ping-pong lists
  buf[wave * 64 + lane] = key[0];
  nf = (int)wave_incl_scan((uint32_t)nf);
  if (lane == 63) sh.wi[wave] = nf;
  __syncthreads();
  int src = 0;
  uint64_t top = 0;
#pragma unroll
  for (int lists = 8; lists >= 1; lists >>= 1) {
    if (wave < lists) {
      const uint64_t *A = buf + (src * 16 + 2 * wave) * 64;
      top = wave_merge_top64(A[lane], A[64 + 63 - lane]);
      if (lists > 1) buf[((src ^ 1) * 16 + wave) * 64 + lane] = top;
    }
    if (lists > 1) __syncthreads();
    src ^= 1;
  }
  if (wave == 0) {
    int n_finite = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) n_finite += sh.wi[w];
    int tok = 0;
    if (n_finite > 0) {
      const int k_eff = min(sp.top_k, n_finite);
      const float v = sample_key_value(top);
      const float vmax = __shfl(v, 0, 64);
      const float p = lane < k_eff ? expf((v - vmax) / sp.temperature) : 0.f;
      const float c = wave_incl_scan(p);
      const float total = __shfl(c, k_eff - 1, 64);
      int kept = k_eff;
      if (sp.top_p < 1.0f) {
        const uint64_t hit = __ballot(lane < k_eff && c >= sp.top_p * total);
        if (hit) kept = min(kept, (int)__ffsll((unsigned long long)hit));
      }
      const float target = u * __shfl(c, kept - 1, 64);
      const uint64_t hit = __ballot(lane < kept && target <= c);
      const int pick = hit ? __ffsll((unsigned long long)hit) - 1 : kept - 1;
      tok = (int)(0xffffffffu - (uint32_t)__shfl((int)(uint32_t)top, pick, 64));
    }
    if (lane == 0) sh.misc[0] = tok;
  }
  __syncthreads();
  return sh.misc[0];
}

// Top-k / temperature / top-p sampling over the finite entries of lg[0..V).
// k-th largest found by an 8-bit radix select on order keys; the candidates are ranked by
// (value desc, index asc); inverse CDF over the kept prefix with target = u * sum(p).  The
// bin scans and the CDF are wave-parallel prefix sums.
__device__ int block_sample(SelectShared &sh, int V, const SamplingParams &sp, float u) {
  if (V <= 2048 && sp.top_k >= 1 && sp.top_k <= 64) return block_sample_top64(sh, V, sp, u);
  const int tid = threadIdx.x, wave = tid >> 6;
  if (tid == 0) sh.misc[2] = 0;  // candidate count
  int local = 0;
  for (int i = tid; i < V; i += 1024) local += isfinite(sh.lg[i]) ? 1 : 0;
  local = (int)wave_incl_scan((uint32_t)local);  // lane 63: the wave's count
  if ((tid & 63) == 63) sh.wi[wave] = local;
  __syncthreads();
  int n_finite = 0;
#pragma unroll
  for (int w = 0; w < 16; ++w) n_finite += sh.wi[w];
  if (n_finite == 0) return 0;
  const int k_eff = (sp.top_k > 0 && sp.top_k < n_finite) ? sp.top_k : n_finite;

  uint32_t thresh = 0;  // keys >= thresh are candidates
  if (k_eff < n_finite) {
    uint32_t prefix = 0, mask = 0;
    int remaining = k_eff;
    // each wave counts into its own histogram (keys of a pass share few digits, so one shared
    // histogram serialises on its hot bins), then the 16 are added per bin by the thread
    // that also clears that bin for the next pass
#pragma unroll
    for (int j = 0; j < 4; ++j) (&sh.whist[0][0])[tid + 1024 * j] = 0;
    __syncthreads();
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int i = tid; i < V; i += 1024) {
        const float v = sh.lg[i];
        if (!isfinite(v)) continue;
        const uint32_t key = order_key(v);
        if ((key & mask) == prefix) atomicAdd(&sh.whist[wave][(key >> shift) & 255u], 1u);
      }
      __syncthreads();
      if (tid < 256) {
        uint32_t t = 0;
#pragma unroll
        for (int w = 0; w < 16; ++w) {
          t += sh.whist[w][tid];
          sh.whist[w][tid] = 0;
        }
        sh.hist[tid] = t;
      }
      __syncthreads();
      if (tid < 64) {
        // bins from the top: lane l holds 255 - 4l - j, j = 0..3; the first bin where the count
        // of keys in it and above reaches `remaining` is the k-th largest key's digit
        const int lane = tid;
        uint32_t c[4], tot = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          c[j] = sh.hist[255 - 4 * lane - j];
          tot += c[j];
        }
        uint32_t run = wave_incl_scan(tot) - tot;  // keys in the bins of earlier lanes
        int found = -1;
        uint32_t at = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (found < 0 && run + c[j] >= (uint32_t)remaining) {
            found = j;
            at = run;
          }
          run += c[j];
        }
        const uint64_t hit = __ballot(found >= 0);
        const int first = hit ? __ffsll((unsigned long long)hit) - 1 : 63;
        if (lane == first) {
          const int sel = found >= 0 ? 255 - 4 * lane - found : 0;
          sh.misc[3] = remaining - (int)(found >= 0 ? at : run);
          sh.umisc[0] = prefix | ((uint32_t)sel << shift);
          uint32_t nb = 0;  // keys in the selected bin
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (j == found) nb = c[j];
          sh.misc[6] = found >= 0 ? (int)nb : 1 << 30;
          sh.misc[7] = 0;
        }
      }
      __syncthreads();
      // read by every thread; the next writes to these come after two more barriers
      remaining = sh.misc[3];
      prefix = sh.umisc[0];
      mask |= 255u << shift;
      const int nbin = sh.misc[6];
      if (shift > 0 && nbin <= 64) {
        // Few keys share the prefix: collect them and take the remaining-th largest directly
        // (the same key the later passes would reach).  Ranks are unique: ties by slot.
        for (int i = tid; i < V; i += 1024) {
          const float v = sh.lg[i];
          if (!isfinite(v)) continue;
          const uint32_t key = order_key(v);
          if ((key & mask) == prefix) sh.skey[atomicAdd(&sh.misc[7], 1)] = key;
        }
        __syncthreads();
        if (tid < nbin) {
          const uint32_t kt = sh.skey[tid];
          int rank = 0;
          for (int o = 0; o < nbin; ++o) {
            const uint32_t ko = sh.skey[o];
            rank += (ko > kt || (ko == kt && o < tid)) ? 1 : 0;
          }
          if (rank == remaining - 1) sh.umisc[0] = kt;
        }
        __syncthreads();
        prefix = sh.umisc[0];
        break;
      }
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
  // pad to a multiple of 4 with entries that never outrank a candidate, then rank each
  // candidate against the others four at a time
  const int n_pad = (n_cand + 3) & ~3;  // <= kMaxVocab
  if (tid < n_pad - n_cand) {
    sh.cv[n_cand + tid] = -INFINITY;
    sh.ci[n_cand + tid] = 0x7fffffff;
  }
  __syncthreads();
  for (int c = tid; c < n_cand; c += 1024) {
    const float v = sh.cv[c];
    const int idx = sh.ci[c];
    int rank = 0;
    for (int o = 0; o < n_pad; o += 4) {
      const float4 ov = *reinterpret_cast<const float4 *>(&sh.cv[o]);
      const int4 oi = *reinterpret_cast<const int4 *>(&sh.ci[o]);
      rank += (ov.x > v || (ov.x == v && oi.x < idx)) ? 1 : 0;
      rank += (ov.y > v || (ov.y == v && oi.y < idx)) ? 1 : 0;
      rank += (ov.z > v || (ov.z == v && oi.z < idx)) ? 1 : 0;
      rank += (ov.w > v || (ov.w == v && oi.w < idx)) ? 1 : 0;
    }
    if (rank < k_eff) {
      sh.sv[rank] = v;
      sh.si[rank] = idx;
    }
  }
  __syncthreads();
  // cv[i] = sum of p over ranks 0..i, p = exp((v - vmax) / T): wave 0, 64 ranks per step
  if (tid < 64) {
    const float vmax = sh.sv[0];
    float carry = 0.f;
    for (int base = 0; base < k_eff; base += 64) {
      const int i = base + tid;
      const float p = i < k_eff ? expf((sh.sv[i] - vmax) / sp.temperature) : 0.f;
      const float c = wave_incl_scan(p) + carry;
      if (i < k_eff) sh.cv[i] = c;
      carry = __shfl(c, 63, 64);
    }
    if (tid == 0) {
      sh.misc[4] = k_eff;  // kept = first rank reaching top_p * sum, plus one
      sh.misc[5] = 0x7fffffff;
    }
  }
  __syncthreads();
  const float total = sh.cv[k_eff - 1];
  if (sp.top_p < 1.0f) {
    const float cut = sp.top_p * total;
    for (int i = tid; i < k_eff; i += 1024)
      if (sh.cv[i] >= cut) atomicMin(&sh.misc[4], i + 1);
  }
  __syncthreads();
  const int kept = sh.misc[4];
  const float target = u * sh.cv[kept - 1];
  for (int i = tid; i < kept; i += 1024)
    if (target <= sh.cv[i]) atomicMin(&sh.misc[5], i);
  __syncthreads();
  const int pick = sh.misc[5] == 0x7fffffff ? kept - 1 : sh.misc[5];
  return sh.si[pick];
}

// Ends a frame (advance = 1) or checks the token drawn after the prefill (advance = 0):
// frame counter, then EOS (the frame's semantic token) or max_frames.
__device__ __forceinline__ void end_frame(SlotState *st, const SlotParams *prm, int advance) {
  if (st->done) return;
  const int f = st->frame + advance;
  st->frame = f;
  if (st->semantic == prm->codec_eos)
    st->done = 1;
  else if (f >= st->max_frames)
    st->done = 2;
}

__global__ __launch_bounds__(1024) void k_select_talker(SelectTalkerArgs a) {
  const int row = blockIdx.x;
  if (a.row_on && !a.row_on[row]) return;
  a.st += row;
  a.prm += row;
  if (a.after_frame && skip_work(a.st, SKIP_TALKER)) {  // no Talker step after the last frame
    if (a.end_frame && threadIdx.x == 0) end_frame(a.st, a.prm, 1);
    return;
  }
  a.logits += (size_t)row * a.V;
  if (!a.x_t16) a.x += (size_t)row * a.H;
  a.cp_prefix += (size_t)row * 2 * a.H;
  a.codes += row * a.codes_row;
  if (a.trace) a.trace += row * a.trace_row;
  __shared__ SelectShared sh;
  __shared__ uint32_t seen[kMaxVocab];  // history occurrences of each token
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
      if (t >= 0 && t < a.V) {
        if (prm.penalty_per_occurrence) atomicAdd(&seen[t], 1u);
        else seen[t] = 1;
      }
    }
    __syncthreads();
  }
  // Once per distinct token (HF), or once per occurrence in sequence (the crate's GPU kernel,
  // kernels.rs:408-426): the same fp32 operation repeated, so both orders give one result.
  const float pen = prm.repetition_penalty;
  for (int i = tid; i < a.V; i += 1024) {
    float l = a.logits[i];
    if (a.trace) a.trace[(size_t)step * a.V + i] = l;
    const uint32_t times = hist ? seen[i] : 0u;
    for (uint32_t r = 0; r < times; ++r) l = (l < 0.0f) ? l * pen : l / pen;
    if (i >= a.V - 1024 && i != prm.codec_eos) l = -INFINITY;
    sh.lg[i] = l;
  }
  __syncthreads();
  const int tok = prm.talker.do_sample ? block_sample(sh, a.V, prm.talker, sampler_uniform(prm, step, 0))
                                       : block_argmax(sh, a.V);
  if (tid == 0) a.st->semantic = tok;

  // CodePredictor prefix: [RMSNorm(x) * gamma ; codec_emb[tok]]
  auto xv = [&](int i) { return a.x_t16 ? a.x[t16_index(row, i)] : a.x[i]; };
  float ss = 0.f;
  for (int i = tid; i < a.H; i += 1024) ss = fmaf(xv(i), xv(i), ss);
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
  for (int w = 0; w < 16; ++w) tot += red[w];
  const float inv = 1.0f / sqrtf(tot / (float)a.H + a.eps);
  for (int i = tid; i < a.H; i += 1024) {
    a.cp_prefix[i] = (xv(i) * inv) * a.gamma[i];
    a.cp_prefix[a.H + i] = bf16_to_f32(a.codec_emb[(size_t)tok * a.H + i]);
  }
  // every thread read the loop state at entry (before the first barrier); thread 0 wrote
  // the semantic token itself
  if (a.end_frame && tid == 0) end_frame(a.st, a.prm, a.after_frame);
}

// Loads first, in two dependent steps: the logits and the row's running embedding sum (their
// addresses need no state), then the state and, for the last group, the semantic token's
// codec embedding row and the trailing text row.  Only the chosen token's embedding row waits
// for the selection.  Vc <= kMaxVocab and Ht <= 2048 (launch_select_cp).
__global__ __launch_bounds__(1024) void k_select_cp(SelectCpArgs a) {
  constexpr int LV = kMaxVocab / 1024;
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const float *logits = a.logits + (size_t)row * a.Vc;
  float *emb_sum = a.emb_sum + (size_t)row * a.Ht;
  float lv[LV], es[2];
#pragma unroll
  for (int j = 0; j < LV; ++j) {
    const int i = tid + 1024 * j;
    lv[j] = i < a.Vc ? logits[i] : 0.f;
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int i = tid + 1024 * j;
    es[j] = (a.group > 0 && i < a.Ht) ? emb_sum[i] : 0.f;
  }
  if (a.row_on && !a.row_on[row]) return;
  a.st += row;
  a.prm += row;
  if (skip_work(a.st, SKIP_DONE)) return;
  a.cur += (size_t)row * a.Ht;
  a.talker_in += (size_t)row * a.Ht;
  a.codes += row * a.codes_row;
  a.trailing += row * a.trailing_row;
  if (a.trace) a.trace += row * a.trace_row;
  __shared__ SelectShared sh;
  const SlotParams prm = *a.prm;
  const int frame = a.st->frame;
  const int semantic = a.st->semantic;
  const bool last = a.group == a.groups - 2;
  float ce[2] = {0.f, 0.f}, tr[2] = {0.f, 0.f};
  if (last) {
    const int trow = min(frame, a.st->trailing_rows);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int i = tid + 1024 * j;
      if (i < a.Ht) {
        ce[j] = bf16_to_f32(a.codec_emb[(size_t)semantic * a.Ht + i]);
        tr[j] = a.trailing[(size_t)trow * a.Ht + i];
      }
    }
  }
#pragma unroll
  for (int j = 0; j < LV; ++j) {
    const int i = tid + 1024 * j;
    if (i < a.Vc) {
      if (a.trace) a.trace[((size_t)frame * (a.groups - 1) + a.group) * a.Vc + i] = lv[j];
      sh.lg[i] = lv[j];
    }
  }
  __syncthreads();
  const int tok = prm.cp.do_sample ? block_sample(sh, a.Vc, prm.cp, sampler_uniform(prm, frame, 1 + a.group))
                                   : block_argmax(sh, a.Vc);
  if (tid == 0) {
    a.codes[(size_t)frame * a.groups + 1 + a.group] = tok;
    if (a.group == 0) a.codes[(size_t)frame * a.groups] = semantic;
    if (a.tok_out) *a.tok_out = tok;
  }
  if (a.token_only) return;  // the next group's hand-off attention stores the rows
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int i = tid + 1024 * j;
    if (i < a.Ht) {
      const float e = bf16_to_f32(a.emb[(size_t)tok * a.Ht + i]);
      a.cur[i] = e;
      const float sum = (a.group == 0) ? e : es[j] + e;
      emb_sum[i] = sum;
      if (last) a.talker_in[i] = (ce[j] + sum) + tr[j];
    }
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

// dst = src [rows][K] repacked for the skinny GEMM: [rows / 16][K / 32][64 lanes][8], lane
// j + 16 kb of (tile, step) holding src[16 tile + j][32 step + 8 kb .. + 8].
__global__ void k_pack_w(const uint16_t *src, uint16_t *dst, int rows, int K) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int ksteps = K >> 5;
  if (i >= (size_t)(rows >> 4) * ksteps * 64) return;
  const int lane = (int)(i & 63);
  const size_t rest = i >> 6;
  const int step = (int)(rest % ksteps);
  const size_t tile = rest / ksteps;
  const int j = lane & 15, kb = lane >> 4;
  *reinterpret_cast<uint4 *>(dst + i * 8) =
      *reinterpret_cast<const uint4 *>(src + (tile * 16 + j) * (size_t)K + step * 32 + kb * 8);
}

// ---------------------------------------------------------------------------------------
// Prompt preparation (text.rs:516-603): text-embedding rows through the text projection
// (fc1, SiLU, fc2; the GEMMs run on the matrix-core path), plus codec embedding rows, placed
// into the prefill, trailing-text and tts_pad rows.
// ---------------------------------------------------------------------------------------
// X[m] = table[ids[m]] (bf16 -> fp32), one workgroup per row.
__global__ void k_text_gather(const uint16_t *table, int width, const int32_t *ids, float *X) {
  const int m = blockIdx.x;
  const uint16_t *src = table + (size_t)ids[m] * width;
  float *dst = X + (size_t)m * width;
  for (int i = threadIdx.x; i < width; i += blockDim.x) dst[i] = bf16_to_f32(src[i]);
}

// x = x / (1 + e^-x) (text.rs:705-707).
__global__ void k_silu(float *x, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] = x[i] / (1.0f + expf(-x[i]));
}

// Row m of Y (+ codec_emb[codec[m]] where codec[m] >= 0, + xvec where codec[m] ==
// kTextSpeakerRow) to its destination dst[m]: (kind << 24) | row, kind 0 = prefill row,
// 1 = trailing row, 2 = the tts_pad row, 3 = none.
__global__ void k_text_assemble(const float *Y, int H, const int32_t *codec, const uint16_t *codec_emb,
                                const float *xvec, const int32_t *dst, float *prefill, float *trailing,
                                float *pad) {
  const int m = blockIdx.x;
  const int kind = dst[m] >> 24, row = dst[m] & 0xffffff;
  if (kind == 3) return;
  float *out = kind == 0 ? prefill + (size_t)row * H : (kind == 1 ? trailing + (size_t)row * H : pad);
  const int c = codec[m];
  const float *y = Y + (size_t)m * H;
  if (c == kTextSpeakerRow) {
    for (int i = threadIdx.x; i < H; i += blockDim.x) out[i] = y[i] + xvec[i];
    return;
  }
  for (int i = threadIdx.x; i < H; i += blockDim.x)
    out[i] = c >= 0 ? y[i] + bf16_to_f32(codec_emb[(size_t)c * H + i]) : y[i];
}

__global__ void k_bf16_to_f32(const uint16_t *src, float *dst, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = bf16_to_f32(src[i]);
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

template <typename K, typename... Args>
static void launch_timed(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t s, const LaunchTiming *t,
                         Args... args) {
  if (t && t->start)
    hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, s, t->start, t->stop, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, lds, s, args...);
}

// Weight loads in flight per lane are capped at kMaxLoads (4 VGPRs each) for streamed
// weights, and at kMaxLoadsCached for cache-resident ones.
constexpr int kMaxLoads = 8;
constexpr int kMaxLoadsCached = 4;

// Rows per wave: spread the matrix over ~256 workgroups (one per CU, one wave per SIMD)
// with every weight load of the launch issued up front; when that needs more than the load
// cap per lane, use more workgroups instead.  The result is one of 1, 2, 3, 4, 6 that fits
// the cap (or 1).
// The cap depends on where the weights come from.  Streamed (non-temporal, read once per
// frame from HBM) matrices keep up to 8 loads per lane: since the input vector reaches the
// waves through LDS once per workgroup, more workgroups with fewer rows each cost little
// (the 1.7B gate/up at 1 row per wave instead of 3, its down at 1 instead of 2: config 4
// 490.2 -> 497.7 frames/s; 24 was best while every lane loaded the whole vector).  The
// CodePredictor's matrices, reread from the last-level cache 15 times per frame, keep 4:
// its gate/up GEMV at 3 workgroups per CU with 4 loads per lane instead of 1 with 12 took
// the 0.6B frame from 524 to 535 frames/s and the 1.7B frame from 435 to 448.
static int gemv_rows_per_wave(int N, int KC, int epi, bool streaming) {
  const int pu = (epi == EPI_SWIGLU) ? 2 : 1;
  const int cap = streaming ? kMaxLoads : kMaxLoadsCached;
  int rw = (N + 1023) / 1024;
  const int cap_rw = cap / (pu * KC);
  if (rw > cap_rw) rw = std::max(1, cap_rw);
  if (rw == 5) rw = 6;
  if (rw > 6) rw = 6;
  while (rw > 1 && rw * pu * KC > cap) rw = rw == 6 ? 4 : rw - 1;
  return rw;
}

static int gemv_grid(int N, int K, int epi, bool streaming) {
  const int waves = K / 512 >= kXldsWideKC ? kXldsWideWaves : 4;  // the one-row forms' workgroups
  const int units = waves * gemv_rows_per_wave(N, K / 512, epi, streaming);
  return (N + units - 1) / units;
}

int gemv_grid_for(int N, int K) { return gemv_grid(N, K, EPI_STORE, false); }

template <int EPI, bool NORM, int KC, int RW, bool NT>
static void gemv_launch(const GemvArgs &a, hipStream_t s, const LaunchTiming *t) {
  const int units = 4 * RW;
  const dim3 grid((a.N + units - 1) / units);
  // Hand-off producer: the CodePredictor's LM heads (store + norm).
  if constexpr (!NT && KC <= 4 && KC != 3 && EPI == EPI_STORE && NORM) {
    if (a.keys_out) {
      if (grid.x > (unsigned)kHandoffKeys) return;  // launch_gemv checked the grid
      launch_timed(k_gemv<EPI, NORM, KC, RW, NT, IN_XLDS, 1, true>, grid, dim3(256), 0, s, t, a);
      return;
    }
  }
  // The Talker's layer-0 QKV GEMV taking its input from the last CodePredictor group.
  if constexpr (EPI == EPI_STORE && NORM && NT && (KC == 1 || KC == 2 || KC == 4)) {
    if (a.tin.keys) {
      launch_timed(k_gemv<EPI, NORM, KC, RW, NT, IN_TALKER>, grid, dim3(256), 0, s, t, a);
      return;
    }
  }
  if constexpr (EPI == EPI_RESIDUAL && !NORM && KC <= 8) {
    if (a.attn_part) {
      launch_timed(k_gemv<EPI, NORM, KC, RW, NT, IN_ATTN>, grid, dim3(256), 0, s, t, a);
      return;
    }
  }
  // The per-head partials of a head-split O projection: the gate/up GEMV after it (one
  // output per wave, launched with RW = 1).
  if constexpr (EPI == EPI_SWIGLU && NORM && RW == 1 && (KC == 1 || KC == 2)) {
    if (a.parts) {
      const dim3 grid_p((a.N + kPartsWaves * RW - 1) / (kPartsWaves * RW));
      if constexpr (!NT) {
        if (a.rows == 2) {  // the CodePredictor's prefix pass
          launch_timed(k_gemv<EPI, NORM, KC, RW, NT, IN_PARTS, 2>, grid_p, dim3(64 * kPartsWaves), 0, s, t, a);
          return;
        }
      }
      launch_timed(k_gemv<EPI, NORM, KC, RW, NT, IN_PARTS>, grid_p, dim3(64 * kPartsWaves), 0, s, t, a);
      return;
    }
  }
  if constexpr (!NT && KC <= 6) {  // two input rows: the CodePredictor's prefix pass
    if (a.rows == 2) {
      launch_timed(k_gemv<EPI, NORM, KC, RW, NT, IN_X, 2>, grid, dim3(256), 0, s, t, a);
      return;
    }
  }
  constexpr int xw = gemv_waves<IN_XLDS, KC>();
  const dim3 grid_x((a.N + xw * RW - 1) / (xw * RW));
  launch_timed(k_gemv<EPI, NORM, KC, RW, NT, IN_XLDS>, grid_x, dim3(64 * xw), 0, s, t, a);
}

template <int EPI, bool NORM, int KC, bool NT>
static hipError_t gemv_rw(const GemvArgs &a, hipStream_t s, const LaunchTiming *t) {
  constexpr int pu = (EPI == EPI_SWIGLU) ? 2 : 1;
  if (a.parts) {  // kPartsWaves-wave workgroups, one output per wave
    gemv_launch<EPI, NORM, KC, 1, NT>(a, s, t);
    return hipGetLastError();
  }
  switch (gemv_rows_per_wave(a.N, KC, EPI, NT)) {
    case 6:
      if constexpr (6 * pu * KC <= kMaxLoads) { gemv_launch<EPI, NORM, KC, 6, NT>(a, s, t); break; }
      [[fallthrough]];
    case 4:
      if constexpr (4 * pu * KC <= kMaxLoads) { gemv_launch<EPI, NORM, KC, 4, NT>(a, s, t); break; }
      [[fallthrough]];
    case 3:
      if constexpr (3 * pu * KC <= kMaxLoads) { gemv_launch<EPI, NORM, KC, 3, NT>(a, s, t); break; }
      [[fallthrough]];
    case 2:
      if constexpr (2 * pu * KC <= kMaxLoads) { gemv_launch<EPI, NORM, KC, 2, NT>(a, s, t); break; }
      [[fallthrough]];
    default:
      gemv_launch<EPI, NORM, KC, 1, NT>(a, s, t);
  }
  return hipGetLastError();
}

template <int EPI, bool NORM, bool NT>
static hipError_t gemv_k(const GemvArgs &a, hipStream_t s, const LaunchTiming *t) {
  switch (a.K / 512) {
    case 1: return gemv_rw<EPI, NORM, 1, NT>(a, s, t);
    case 2: return gemv_rw<EPI, NORM, 2, NT>(a, s, t);
    case 3: return gemv_rw<EPI, NORM, 3, NT>(a, s, t);
    case 4: return gemv_rw<EPI, NORM, 4, NT>(a, s, t);
    case 6: return gemv_rw<EPI, NORM, 6, NT>(a, s, t);
    case 8: return gemv_rw<EPI, NORM, 8, NT>(a, s, t);
    case 12: return gemv_rw<EPI, NORM, 12, NT>(a, s, t);
  }
  return hipErrorInvalidValue;
}

template <bool NT>
static hipError_t gemv_epi(int epi, bool norm, const GemvArgs &a, hipStream_t s, const LaunchTiming *t) {
  switch (epi) {
    case EPI_STORE: return norm ? gemv_k<EPI_STORE, true, NT>(a, s, t) : gemv_k<EPI_STORE, false, NT>(a, s, t);
    case EPI_RESIDUAL: return norm ? hipErrorInvalidValue : gemv_k<EPI_RESIDUAL, false, NT>(a, s, t);
    case EPI_SWIGLU: return norm ? gemv_k<EPI_SWIGLU, true, NT>(a, s, t) : hipErrorInvalidValue;
    case EPI_BIAS: return norm ? hipErrorInvalidValue : gemv_k<EPI_BIAS, false, NT>(a, s, t);
  }
  return hipErrorInvalidValue;
}

static bool handoff_ok(const TokenHandoff &h) {
  return h.keys && h.n_keys >= 1 && h.n_keys <= kHandoffKeys && h.emb && h.emb_width > 0 && h.emb_width % 8 == 0 &&
         h.cur && h.sum && h.codes && h.code >= 1 && h.code < h.groups &&
         (!h.cur_table || (h.cur_width > 0 && h.cur_width % 4 == 0));
}

hipError_t launch_gemv(int epi, bool norm, bool streaming, const GemvArgs &a, hipStream_t s,
                       const LaunchTiming *t) {
  if (!gemv_supports_k(a.K) || a.N <= 0) return hipErrorInvalidValue;
  if (a.keys_out) {
    const bool ok = !streaming && a.rows <= 1 && !a.attn_part && (a.K == 512 || a.K == 1024 || a.K == 2048) &&
                    a.st && epi == EPI_STORE && norm && gemv_grid(a.N, a.K, epi, false) <= kHandoffKeys;
    if (!ok) return hipErrorInvalidValue;
  }
  if (a.rows > 1 && (a.rows != 2 || streaming || a.attn_part || a.K > 6 * 512 || a.ldx_r % 4 ||
                     (epi == EPI_RESIDUAL && !a.ldr_r) || !a.ldo_r))
    return hipErrorInvalidValue;
  if (a.parts && a.rows == 2 && (a.ldp_r % 4 || a.ldp_r < a.n_parts * a.ld_parts || (a.x_store && a.ldxs_r < a.K) ||
                                 a.ldxs_r % 4))
    return hipErrorInvalidValue;
  if (a.tin.keys) {
    const TokenHandoff &h = a.tin;
    const bool ok = epi == EPI_STORE && norm && streaming && a.rows <= 1 && !a.attn_part && !a.parts &&
                    !a.keys_out && (a.K == 512 || a.K == 1024 || a.K == 2048) && h.emb_width == a.K &&
                    h.n_keys >= 1 && h.n_keys <= kHandoffKeys && h.emb && h.sum && h.codes && h.groups > 1 &&
                    h.code >= 1 && h.code < h.groups && a.tin_codec_emb && a.tin_trailing && a.tin_x && a.st &&
                    a.skip != SKIP_NEVER;
    if (!ok) return hipErrorInvalidValue;
  }
  if (a.parts && (epi != EPI_SWIGLU || !norm || a.attn_part || a.keys_out ||
                  (a.K != 512 && a.K != 1024) || a.n_parts < 1 || a.n_parts > kMaxParts ||
                  a.ld_parts < a.K || a.ld_parts % 4 || !a.x))
    return hipErrorInvalidValue;
  return streaming ? gemv_epi<true>(epi, norm, a, s, t) : gemv_epi<false>(epi, norm, a, s, t);
}

int attn_chunk_len(int cap) {
  // 16 rows for a cache of at most 16 (the CodePredictor's), else 32, 64 or 128: at most
  // kAttnMaxChunks chunks up to a 1024-row cache
  if (cap <= 16) return 16;
  int c = 32;
  while (c < kAttnMaxChunk && c * kAttnMaxChunks < cap) c *= 2;
  return c;
}

int attn_chunks(int cap) { return (cap + attn_chunk_len(cap) - 1) / attn_chunk_len(cap); }

int attn_rows_chunk_len(int cap) {
  if (cap <= 16) return 16;
  int c = 32;
  while (c < kAttnMaxChunk && c * kAttnMergeMaxChunks < cap) c *= 2;
  return c;
}

int attn_max_cache_steps(int q_heads, int kv_heads) {
  (void)q_heads;
  (void)kv_heads;
  return kAttnMaxChunk * kAttnMergeMaxChunks;  // the merge's most partials, of the longest chunks
}

hipError_t launch_attn_decode(const AttnArgs &a, int head_dim, hipStream_t s, const LaunchTiming *t, int rows) {
  if (head_dim != 128 || a.kv_heads <= 0 || a.q_heads % a.kv_heads) return hipErrorInvalidValue;
  if (rows < 1 || rows > kMaxRows || (rows > 1 && (!a.row_on || a.ld_qkv <= 0 || a.kv_row <= 0))) return hipErrorInvalidValue;
  if (rows > 1 && (a.partial_out ? a.part_row <= 0 : a.ld_out <= 0)) return hipErrorInvalidValue;
  const int G = a.q_heads / a.kv_heads;
  // chunk: attn_chunk_len(cap) for one stream (the O GEMV merges at most kAttnMaxChunks
  // partials); any of 32 / 64 / 128 for stream rows (merged by k_attn_merge).
  if (a.cap > attn_max_cache_steps(a.q_heads, a.kv_heads)) return hipErrorInvalidValue;
  if (rows == 1 ? a.chunk != attn_chunk_len(a.cap) : a.chunk != attn_rows_chunk_len(a.cap))
    return hipErrorInvalidValue;
  const int nch = (a.cap + a.chunk - 1) / a.chunk;
  if (a.partial_out ? a.part_chunks < nch : nch != 1) return hipErrorInvalidValue;
  const dim3 grid(a.kv_heads, nch, rows), block(256);
  if (a.h.keys) {
    // the hand-off: one chunk (16 or 32 rows), a position given by the launch; stream rows store
    // through their own slices (no overlap between rows)
    const int qkv_rows = (a.q_heads + 2 * a.kv_heads) * head_dim;
    const TokenHandoff &h = a.h;
    const bool rows_ok = rows == 1 || (h.keys_row >= h.n_keys && h.sum_row >= h.emb_width &&
                                       h.cur_row >= (h.cur_table ? h.cur_width : h.emb_width) &&
                                       h.codes_row >= h.groups);
    if (!rows_ok || a.partial_out || (a.chunk != 16 && a.chunk != 32) || a.pos_mode != POS_CONST || !a.qkv_table ||
        a.ld_table < qkv_rows || !handoff_ok(h) || h.emb_width > 2048 || h.emb_width % 4 ||
        (h.cur_table && h.cur_width > 2048) || !a.st)
      return hipErrorInvalidValue;
#define Q3T_HO_CASE(GG, TT, CC) \
  if (G == GG && a.chunk == CC) launch_timed(k_attn_split<128, GG, TT, CC, true>, grid, block, 0, s, t, a);
    if (a.kv_bf16) {
      Q3T_HO_CASE(1, uint16_t, 16) Q3T_HO_CASE(2, uint16_t, 16) Q3T_HO_CASE(1, uint16_t, 32) Q3T_HO_CASE(2, uint16_t, 32)
    } else {
      Q3T_HO_CASE(1, float, 16) Q3T_HO_CASE(2, float, 16) Q3T_HO_CASE(1, float, 32) Q3T_HO_CASE(2, float, 32)
    }
#undef Q3T_HO_CASE
    return hipGetLastError();
  }
#define Q3T_ATTN_CASE(GG, TT, CC) \
  if (G == GG && a.chunk == CC) {  \
    launch_timed(k_attn_split<128, GG, TT, CC>, grid, block, 0, s, t, a); \
    return hipGetLastError();     \
  }
  if (a.kv_bf16) {
    Q3T_ATTN_CASE(1, uint16_t, 16) Q3T_ATTN_CASE(1, uint16_t, 32) Q3T_ATTN_CASE(1, uint16_t, 64)
    Q3T_ATTN_CASE(1, uint16_t, 128)
    Q3T_ATTN_CASE(2, uint16_t, 16) Q3T_ATTN_CASE(2, uint16_t, 32) Q3T_ATTN_CASE(2, uint16_t, 64)
    Q3T_ATTN_CASE(2, uint16_t, 128)
  } else {
    Q3T_ATTN_CASE(1, float, 16) Q3T_ATTN_CASE(1, float, 32) Q3T_ATTN_CASE(1, float, 64) Q3T_ATTN_CASE(1, float, 128)
    Q3T_ATTN_CASE(2, float, 16) Q3T_ATTN_CASE(2, float, 32) Q3T_ATTN_CASE(2, float, 64) Q3T_ATTN_CASE(2, float, 128)
  }
#undef Q3T_ATTN_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_attn_oproj_full(const AttnArgs &a, int head_dim, hipStream_t s, const LaunchTiming *t) {
  if (head_dim != 128 || a.kv_heads <= 0 || a.kv_heads > kMaxParts || a.q_heads % a.kv_heads) return hipErrorInvalidValue;
  const int G = a.q_heads / a.kv_heads;
  const int rows = kFusedWaves * (64 / (G * 16));  // W_o rows per workgroup
  if (G < 1 || G > 2 || a.cap < 1 || a.cap > kFusedMaxCap || a.row_on || a.h.keys || a.h.tok_in ||
      (a.pos_mode != POS_TALKER_FRAME && a.pos_mode != POS_CONST) || !a.wo || !a.opart || !a.st ||
      a.wo_rows <= 0 || a.wo_rows % rows)
    return hipErrorInvalidValue;
  const dim3 grid(a.kv_heads, a.wo_rows / rows, 1), block(64 * kFusedWaves);
  if (a.kv_bf16) {
    if (G == 1) launch_timed(k_attn_oproj_full<1, uint16_t>, grid, block, 0, s, t, a);
    else launch_timed(k_attn_oproj_full<2, uint16_t>, grid, block, 0, s, t, a);
  } else {
    if (G == 1) launch_timed(k_attn_oproj_full<1, float>, grid, block, 0, s, t, a);
    else launch_timed(k_attn_oproj_full<2, float>, grid, block, 0, s, t, a);
  }
  return hipGetLastError();
}

int attn_oproj_full_rows(int q_heads, int kv_heads) {
  const int G = kv_heads > 0 ? q_heads / kv_heads : 0;
  return (G == 1 || G == 2) ? kFusedWaves * (64 / (G * 16)) : 0;
}


hipError_t launch_attn_oproj(const AttnArgs &a, int head_dim, hipStream_t s, const LaunchTiming *t) {
  if (head_dim != 128 || a.kv_heads <= 0 || a.q_heads % a.kv_heads || a.kv_heads > kMaxParts) return hipErrorInvalidValue;
  const int G = a.q_heads / a.kv_heads;
  if (G < 1 || G > 2 || a.cap < 1 || a.cap > 32 || a.chunk != attn_chunk_len(a.cap) || a.partial_out || a.row_on ||
      a.pos_mode != POS_CONST || !a.wo || !a.opart || a.wo_rows <= 0 || a.wo_rows % kOprojRows || !a.st)
    return hipErrorInvalidValue;
  const dim3 grid(a.kv_heads, a.wo_rows / kOprojRows, 1), block(256);
  if (a.h.keys || a.h.tok_in) {
    const int qkv_rows = (a.q_heads + 2 * a.kv_heads) * head_dim;
    const TokenHandoff &h = a.h;
    if (!a.qkv_table || a.ld_table < qkv_rows) return hipErrorInvalidValue;
    // tok_in: the token's table row (the caller validates the token's range: the selection
    // kernel that stores it draws from the table's vocabulary), and with emb the stores
    const bool stores_ok = h.emb && h.emb_width > 0 && h.emb_width <= 2048 && h.emb_width % 8 == 0 && h.cur &&
                           h.sum && h.codes && h.code >= 1 && h.code < h.groups;
    if (h.tok_in ? (h.keys != nullptr || h.cur_table != nullptr || (h.emb && !stores_ok))
                 : (!handoff_ok(h) || h.emb_width > 2048 || h.emb_width % 4 || (h.cur_table && h.cur_width > 2048)))
      return hipErrorInvalidValue;
#define Q3T_OP_CASE(GG, TT, CC, HH) \
  if (G == GG && a.chunk == CC) launch_timed(k_attn_split<128, GG, TT, CC, HH, true>, grid, block, 0, s, t, a);
    if (a.kv_bf16) {
      Q3T_OP_CASE(1, uint16_t, 16, true) Q3T_OP_CASE(2, uint16_t, 16, true)
      Q3T_OP_CASE(1, uint16_t, 32, true) Q3T_OP_CASE(2, uint16_t, 32, true)
    } else {
      Q3T_OP_CASE(1, float, 16, true) Q3T_OP_CASE(2, float, 16, true)
      Q3T_OP_CASE(1, float, 32, true) Q3T_OP_CASE(2, float, 32, true)
    }
    return hipGetLastError();
  }
  if (a.kv_bf16) {
    Q3T_OP_CASE(1, uint16_t, 16, false) Q3T_OP_CASE(2, uint16_t, 16, false)
    Q3T_OP_CASE(1, uint16_t, 32, false) Q3T_OP_CASE(2, uint16_t, 32, false)
  } else {
    Q3T_OP_CASE(1, float, 16, false) Q3T_OP_CASE(2, float, 16, false)
    Q3T_OP_CASE(1, float, 32, false) Q3T_OP_CASE(2, float, 32, false)
  }
#undef Q3T_OP_CASE
  return hipGetLastError();
}

// Sum of the K splits in split order, then the epilogue: Y[m][n] = f(sum_z ws[z][m][n])
// (SwiGLU: silu(sum_z gate) * sum_z up).
template <int EPI>
__global__ __launch_bounds__(256) void k_gemm_split_reduce(GemmArgs a, int nsplit) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t mn = (size_t)a.M * a.N;
  if (i >= mn) return;
  const int m = (int)(i / a.N), n = (int)(i % a.N);
  if constexpr (EPI == EPI_SWIGLU) {  // gate and up sums, each added in split order
    const size_t gi = (size_t)m * 2 * a.N + n;
    float g = a.split_ws[gi], u = a.split_ws[gi + a.N];
    for (int z = 1; z < nsplit; ++z) {
      g += a.split_ws[(size_t)z * 2 * mn + gi];
      u += a.split_ws[(size_t)z * 2 * mn + gi + a.N];
    }
    a.Y[(size_t)m * a.ldy + n] = g / (1.0f + expf(-g)) * u;
    return;
  }
  float v = a.split_ws[i];
  for (int z = 1; z < nsplit; ++z) v += a.split_ws[(size_t)z * mn + i];
  a.Y[(size_t)m * a.ldy + n] = gemm_epilogue<EPI>(a, m, n, v);
}

// K splits for a launch of `blocks` workgroups: enough to reach ~256 workgroups, at least
// 4 k steps of 32 per split, at most 16 splits, within the workspace.
static int gemm_splits(const GemmArgs &a, int blocks, bool swiglu) {
  if (!a.split_ws || blocks >= 128) return 1;
  int sp = std::min(std::min((256 + blocks - 1) / blocks, a.K / 32 / 4), 16);
  // SwiGLU keeps the gate and the up sums apart until the reduction
  while (sp > 1 && (int64_t)sp * a.M * a.N * (swiglu ? 2 : 1) > a.split_cap) --sp;
  return std::max(sp, 1);
}

template <int EPI>
static hipError_t gemm_epi(const GemmArgs &a, hipStream_t s) {
  // 16-row tiles for short M (batched decode), 32-row tiles otherwise; 64 output columns
  // per wave (2 x 32 for SwiGLU gate/up pairs).
  constexpr int NB = 4;
  constexpr int NT = (EPI == EPI_SWIGLU) ? NB / 2 : NB;
  const int cols_per_wg = 4 * 16 * NT;
  dim3 grid;
  int path;
  // 96-column blocks where N is a multiple of 96 but not of 128
  const bool bw96 = EPI != EPI_SWIGLU && a.N % 128 != 0 && a.N % 96 == 0;
  if (a.M >= 128 && a.K % 32 == 0 && (EPI != EPI_SWIGLU || a.N % 64 == 0) && a.ldx % 4 == 0) {
    const int nout = EPI == EPI_SWIGLU ? 64 : (bw96 ? 96 : 128);
    grid = dim3((a.N + nout - 1) / nout, (a.M + 127) / 128);
    path = 0;
  } else if (a.M <= 16) {
    grid = dim3((a.N + cols_per_wg - 1) / cols_per_wg, (a.M + 15) / 16);
    path = 1;
  } else {
    grid = dim3((a.N + cols_per_wg - 1) / cols_per_wg, (a.M + 31) / 32);
    path = 2;
  }
  grid.z = gemm_splits(a, (int)(grid.x * grid.y), EPI == EPI_SWIGLU);
  if (path == 0) {
    const int xs = (a.row_scale ? 1 : 0) | (a.gamma ? 2 : 0);
    bool launched = false;
    if constexpr (EPI != EPI_SWIGLU) {
      if (bw96) {
        switch (xs) {
          case 0: hipLaunchKernelGGL((k_gemm_lds<EPI, 0, 96>), grid, dim3(256), 0, s, a); break;
          case 1: hipLaunchKernelGGL((k_gemm_lds<EPI, 1, 96>), grid, dim3(256), 0, s, a); break;
          case 2: hipLaunchKernelGGL((k_gemm_lds<EPI, 2, 96>), grid, dim3(256), 0, s, a); break;
          default: hipLaunchKernelGGL((k_gemm_lds<EPI, 3, 96>), grid, dim3(256), 0, s, a); break;
        }
        launched = true;
      }
    }
    if (!launched) {
      switch (xs) {
        case 0: hipLaunchKernelGGL((k_gemm_lds<EPI, 0>), grid, dim3(256), 0, s, a); break;
        case 1: hipLaunchKernelGGL((k_gemm_lds<EPI, 1>), grid, dim3(256), 0, s, a); break;
        case 2: hipLaunchKernelGGL((k_gemm_lds<EPI, 2>), grid, dim3(256), 0, s, a); break;
        default: hipLaunchKernelGGL((k_gemm_lds<EPI, 3>), grid, dim3(256), 0, s, a); break;
      }
    }
  }
  else if (path == 1) hipLaunchKernelGGL((k_gemm_mfma<EPI, 1, NB>), grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL((k_gemm_mfma<EPI, 2, NB>), grid, dim3(256), 0, s, a);
  if (grid.z > 1) {
    const size_t mn = (size_t)a.M * a.N;
    hipLaunchKernelGGL((k_gemm_split_reduce<EPI>), dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, s, a,
                       (int)grid.z);
  }
  return hipGetLastError();
}

template <int EPI, bool NORM, bool XT16, bool WNT>
static hipError_t skinny_ks(const GemmArgs &a, hipStream_t s) {
  const dim3 grid((a.N + 15) / 16), block(1024);
  switch (a.K / 512) {
    case 1: hipLaunchKernelGGL((k_gemm_skinny<EPI, NORM, 1, false, XT16, false, 1, WNT>), grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((k_gemm_skinny<EPI, NORM, 2, false, XT16, false, 1, WNT>), grid, block, 0, s, a); break;
    case 3: hipLaunchKernelGGL((k_gemm_skinny<EPI, NORM, 3, false, XT16, false, 1, WNT>), grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL((k_gemm_skinny<EPI, NORM, 4, false, XT16, false, 1, WNT>), grid, block, 0, s, a); break;
    case 6:
      if constexpr (NORM) return hipErrorInvalidValue;
      else hipLaunchKernelGGL((k_gemm_skinny<EPI, NORM, 6, false, XT16, false, 1, WNT>), grid, block, 0, s, a);
      break;
    case 8:
      if constexpr (NORM) return hipErrorInvalidValue;
      else hipLaunchKernelGGL((k_gemm_skinny<EPI, NORM, 8, false, XT16, false, 1, WNT>), grid, block, 0, s, a);
      break;
    case 12:
      if constexpr (NORM) return hipErrorInvalidValue;
      else hipLaunchKernelGGL((k_gemm_skinny<EPI, NORM, 12, false, XT16, false, 1, WNT>), grid, block, 0, s, a);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int EPI, bool NORM>
static hipError_t skinny_ks(const GemmArgs &a, hipStream_t s) {
  if (a.w_nt) return a.x_t16 ? skinny_ks<EPI, NORM, true, true>(a, s) : skinny_ks<EPI, NORM, false, true>(a, s);
  return a.x_t16 ? skinny_ks<EPI, NORM, true, false>(a, s) : skinny_ks<EPI, NORM, false, false>(a, s);
}

// The K-split residual GEMM (GemmArgs::split2): 2 x N / 16 workgroups, each half of K.
template <int MB, bool WNT = false>
static hipError_t skinny_split2(const GemmArgs &a, hipStream_t s) {
  const dim3 grid((a.N + 15) / 16, 2), block(1024);
  switch (a.K / 1024) {
    case 1: hipLaunchKernelGGL((k_gemm_skinny<EPI_RESIDUAL, false, 1, false, true, true, MB, WNT>), grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((k_gemm_skinny<EPI_RESIDUAL, false, 2, false, true, true, MB, WNT>), grid, block, 0, s, a); break;
    case 3: hipLaunchKernelGGL((k_gemm_skinny<EPI_RESIDUAL, false, 3, false, true, true, MB, WNT>), grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL((k_gemm_skinny<EPI_RESIDUAL, false, 4, false, true, true, MB, WNT>), grid, block, 0, s, a); break;
    case 6: hipLaunchKernelGGL((k_gemm_skinny<EPI_RESIDUAL, false, 6, false, true, true, MB, WNT>), grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Two row blocks (GemmArgs::mb = 2), the forms the CodePredictor's two-position prefix pass
// runs: QKV (RMSNorm, T16 or row-major input), gate/up (RMSNorm, SwiGLU), the projection
// (bias, row-major input); K = 512 * {1, 2, 4}.
template <int EPI, bool NORM, bool XT16>
static hipError_t skinny_mb2_ks(const GemmArgs &a, hipStream_t s) {
  const dim3 grid((a.N + 15) / 16), block(1024);
  switch (a.K / 512) {
    case 1: hipLaunchKernelGGL((k_gemm_skinny<EPI, NORM, 1, false, XT16, false, 2>), grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((k_gemm_skinny<EPI, NORM, 2, false, XT16, false, 2>), grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL((k_gemm_skinny<EPI, NORM, 4, false, XT16, false, 2>), grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

static hipError_t skinny_mb2(int epi, bool norm, const GemmArgs &a, hipStream_t s) {
  if (epi == EPI_STORE && norm) return a.x_t16 ? skinny_mb2_ks<EPI_STORE, true, true>(a, s)
                                                : skinny_mb2_ks<EPI_STORE, true, false>(a, s);
  if (epi == EPI_SWIGLU && norm && a.x_t16) return skinny_mb2_ks<EPI_SWIGLU, true, true>(a, s);
  if (epi == EPI_BIAS && !norm && !a.x_t16) return skinny_mb2_ks<EPI_BIAS, false, false>(a, s);
  return hipErrorInvalidValue;
}

bool gemm_skinny_split2_supports(int K) { return K % 1024 == 0 && (K / 1024 <= 4 || K / 1024 == 6); }

// The greedy hand-off producer (LM heads over stream rows, T16 input): per-row argmax keys, no Y.
static hipError_t skinny_keys(const GemmArgs &a, hipStream_t s) {
  if (!a.x_t16) return hipErrorInvalidValue;
  const dim3 grid((a.N + 15) / 16), block(1024);
  switch (a.K / 512) {
    case 1: hipLaunchKernelGGL((k_gemm_skinny<EPI_STORE, true, 1, true>), grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((k_gemm_skinny<EPI_STORE, true, 2, true>), grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL((k_gemm_skinny<EPI_STORE, true, 4, true>), grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

bool gemm_skinny_supports(int M, int K, bool norm) {
  return M >= 1 && M <= 16 && gemv_supports_k(K) && (!norm || K <= 2048);
}

hipError_t launch_gemm_skinny(int epi, bool norm, const GemmArgs &a, hipStream_t s) {
  if (!gemm_skinny_supports(a.M, a.K, norm) || a.N <= 0 || a.ldx % 4 || (norm && (!a.gamma || a.row_scale)))
    return hipErrorInvalidValue;
  // T16 output / residual needs N % 32 (whole k steps).  The weights must be packed
  // (launch_pack_weights) in whole 16-column tiles, the last one padded; SwiGLU's up tiles
  // start at tile N / 16, so it needs N % 16 == 0.
  if (((a.y_t16 || a.r_t16) && a.N % 32) || !a.w_packed || (epi == EPI_SWIGLU && a.N % 16))
    return hipErrorInvalidValue;
  if (a.keys_out) {
    if (epi != EPI_STORE || !norm || a.keys_row < (a.N + 15) / 16 || a.mb == 2) return hipErrorInvalidValue;
    return skinny_keys(a, s);
  }
  if (a.mb != 0 && a.mb != 1 && a.mb != 2) return hipErrorInvalidValue;
  if (a.split2) {
    if (epi != EPI_RESIDUAL || norm || !a.x_t16 || !a.y_t16 || !a.res_zero || !gemm_skinny_split2_supports(a.K))
      return hipErrorInvalidValue;
    if (a.mb == 2) return skinny_split2<2>(a, s);
    return a.w_nt ? skinny_split2<1, true>(a, s) : skinny_split2<1>(a, s);
  }
  if (a.mb == 2) return skinny_mb2(epi, norm, a, s);
  switch (epi) {
    case EPI_STORE: return norm ? skinny_ks<EPI_STORE, true>(a, s) : skinny_ks<EPI_STORE, false>(a, s);
    case EPI_RESIDUAL: return norm ? hipErrorInvalidValue : skinny_ks<EPI_RESIDUAL, false>(a, s);
    case EPI_SWIGLU: return norm ? skinny_ks<EPI_SWIGLU, true>(a, s) : skinny_ks<EPI_SWIGLU, false>(a, s);
    case EPI_BIAS: return norm ? hipErrorInvalidValue : skinny_ks<EPI_BIAS, false>(a, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_pack_weights(const uint16_t *src, uint16_t *dst, int rows, int K, hipStream_t s) {
  if (rows <= 0 || rows % 16 || K <= 0 || K % 32 || !src || !dst) return hipErrorInvalidValue;
  const size_t n = (size_t)(rows / 16) * (K / 32) * 64;
  hipLaunchKernelGGL(k_pack_w, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src, dst, rows, K);
  return hipGetLastError();
}

hipError_t launch_gemm(int epi, const GemmArgs &a, hipStream_t s) {
  if (a.M <= 0 || a.N <= 0 || a.K <= 0 || a.K % 32 || a.ldx % 4) return hipErrorInvalidValue;
  if (a.xseg_len && (a.xseg_len < 0 || a.xseg_len % 32 || a.K % a.xseg_len || a.xseg_stride % 4))
    return hipErrorInvalidValue;
  switch (epi) {
    case EPI_STORE: return gemm_epi<EPI_STORE>(a, s);
    case EPI_RESIDUAL: return gemm_epi<EPI_RESIDUAL>(a, s);
    case EPI_SWIGLU: return gemm_epi<EPI_SWIGLU>(a, s);
    case EPI_BIAS: return gemm_epi<EPI_BIAS>(a, s);
    case EPI_AFFINE_RES: return a.res ? gemm_epi<EPI_AFFINE_RES>(a, s) : hipErrorInvalidValue;
    case EPI_BIAS_GELU: return a.bias ? gemm_epi<EPI_BIAS_GELU>(a, s) : hipErrorInvalidValue;
  }
  return hipErrorInvalidValue;
}

hipError_t launch_text_gather(const uint16_t *table, int width, const int32_t *ids, int M, float *X, hipStream_t s) {
  if (M <= 0 || width <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_text_gather, dim3(M), dim3(256), 0, s, table, width, ids, X);
  return hipGetLastError();
}

hipError_t launch_silu(float *x, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_silu, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, n);
  return hipGetLastError();
}

hipError_t launch_text_assemble(const float *Y, int H, int M, const int32_t *codec, const uint16_t *codec_emb,
                                const float *xvec, const int32_t *dst, float *prefill, float *trailing, float *pad,
                                hipStream_t s) {
  if (M <= 0 || H <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_text_assemble, dim3(M), dim3(256), 0, s, Y, H, codec, codec_emb, xvec, dst, prefill, trailing,
                     pad);
  return hipGetLastError();
}

hipError_t launch_bf16_to_f32(const uint16_t *src, float *dst, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_bf16_to_f32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src, dst, n);
  return hipGetLastError();
}

hipError_t launch_row_rms(const float *X, int ldx, int M, int K, float eps, float *inv_rms, hipStream_t s) {
  if (M <= 0 || K <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_row_rms, dim3((M + 3) / 4), dim3(256), 0, s, X, ldx, M, K, eps, inv_rms);
  return hipGetLastError();
}

hipError_t launch_prefix_attention(const PrefillAttnArgs &a, hipStream_t s) {
  if (a.P != 2 || a.pos0 != 0 || a.kv_heads <= 0 || a.q_heads % a.kv_heads || a.cap < 2) return hipErrorInvalidValue;
  const int G = a.q_heads / a.kv_heads;
  if (G != 1 && G != 2) return hipErrorInvalidValue;
  if (a.wo) {  // fused output projection
    if (!a.opart || a.wo_rows <= 0 || a.wo_rows % kOprojRows || a.kv_heads > kMaxParts ||
        a.opart_row < (int64_t)a.kv_heads * a.wo_rows)
      return hipErrorInvalidValue;
    const dim3 grid_o(a.kv_heads, a.wo_rows / kOprojRows), block_o(256);
    if (a.kv_bf16) {
      if (G == 1) hipLaunchKernelGGL((k_attn_prefix<1, uint16_t, 2, true>), grid_o, block_o, 0, s, a);
      else hipLaunchKernelGGL((k_attn_prefix<2, uint16_t, 2, true>), grid_o, block_o, 0, s, a);
    } else {
      if (G == 1) hipLaunchKernelGGL((k_attn_prefix<1, float, 2, true>), grid_o, block_o, 0, s, a);
      else hipLaunchKernelGGL((k_attn_prefix<2, float, 2, true>), grid_o, block_o, 0, s, a);
    }
    return hipGetLastError();
  }
  const dim3 grid(a.kv_heads), block(256);
  if (a.kv_bf16) {
    if (G == 1) hipLaunchKernelGGL((k_attn_prefix<1, uint16_t, 2>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_attn_prefix<2, uint16_t, 2>), grid, block, 0, s, a);
  } else {
    if (G == 1) hipLaunchKernelGGL((k_attn_prefix<1, float, 2>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_attn_prefix<2, float, 2>), grid, block, 0, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_prefix_attention_rows(const PrefillAttnArgs &a, int rows, hipStream_t s) {
  if (a.P != 2 || a.pos0 != 0 || a.kv_heads <= 0 || a.q_heads % a.kv_heads || a.cap < 2 || a.wo || rows < 1 ||
      rows > kMaxRows || !a.st || a.ldo != a.q_heads * 128 || a.ldo % 32 || (rows > 1 && a.kv_row <= 0))
    return hipErrorInvalidValue;
  const int G = a.q_heads / a.kv_heads;
  if (G != 1 && G != 2) return hipErrorInvalidValue;
  const dim3 grid(a.kv_heads, 1, rows), block(256);
  if (a.kv_bf16) {
    if (G == 1) hipLaunchKernelGGL((k_attn_prefix<1, uint16_t, 2, false, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_attn_prefix<2, uint16_t, 2, false, true>), grid, block, 0, s, a);
  } else {
    if (G == 1) hipLaunchKernelGGL((k_attn_prefix<1, float, 2, false, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_attn_prefix<2, float, 2, false, true>), grid, block, 0, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_prefill_attention(const PrefillBatchArgs &a, hipStream_t s) {
  if (a.nseg < 1 || a.nseg > kMaxPrefillSegs || a.kv_heads <= 0 || a.q_heads % a.kv_heads || a.ldq % 4 ||
      a.ldo % 4 || a.unit0[0] != 0)
    return hipErrorInvalidValue;
  int rows = 0;
  for (int i = 0; i < a.nseg; ++i) {
    if (a.P[i] < 1 || a.P[i] > a.cap || a.row0[i] != rows || !a.kcache[i] || !a.vcache[i] ||
        a.unit0[i + 1] != a.unit0[i] + (a.P[i] + 15) / 16 * a.q_heads)
      return hipErrorInvalidValue;
    rows += a.P[i];
  }
  if (rows != a.M) return hipErrorInvalidValue;
  const dim3 g1((a.q_heads + 2 * a.kv_heads + 3) / 4, a.M), g2((a.unit0[a.nseg] + 3) / 4), block(256);
  if (a.kv_bf16) {
    hipLaunchKernelGGL(k_prefill_qkv<uint16_t>, g1, block, 0, s, a);
    hipLaunchKernelGGL(k_attn_prefill<uint16_t>, g2, block, 0, s, a);
  } else {
    hipLaunchKernelGGL(k_prefill_qkv<float>, g1, block, 0, s, a);
    hipLaunchKernelGGL(k_attn_prefill<float>, g2, block, 0, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_attn_merge(const AttnMergeArgs &a, int rows, hipStream_t s) {
  if (rows < 1 || rows > kMaxRows || a.kv_heads <= 0 || a.q_heads % a.kv_heads || a.chunk <= 0 ||
      a.part_chunks <= 0 || a.q_heads * 128 > a.ld_out || (rows > 1 && (!a.row_on || a.part_row <= 0)))
    return hipErrorInvalidValue;
  if ((a.q_heads / a.kv_heads) * 128 > 256 || a.part_chunks > kAttnMergeMaxChunks) return hipErrorInvalidValue;
  // (m, l) and output pairs: 8-byte aligned records and rows
  if ((a.part_row & 1) || (reinterpret_cast<uintptr_t>(a.part) & 7) || (reinterpret_cast<uintptr_t>(a.out) & 7) ||
      (!a.out_t16 && (a.ld_out & 1)))
    return hipErrorInvalidValue;
  const dim3 grid(a.kv_heads, rows), block(128);
  if (a.part_chunks <= 8) hipLaunchKernelGGL(k_attn_merge<8>, grid, block, 0, s, a);
  else if (a.part_chunks <= 16) hipLaunchKernelGGL(k_attn_merge<16>, grid, block, 0, s, a);
  else if (a.part_chunks <= 24) hipLaunchKernelGGL(k_attn_merge<24>, grid, block, 0, s, a);
  else if (a.part_chunks <= 32) hipLaunchKernelGGL(k_attn_merge<32>, grid, block, 0, s, a);
  else if (a.part_chunks <= 48) hipLaunchKernelGGL(k_attn_merge<48>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(k_attn_merge<64>, grid, block, 0, s, a);
  return hipGetLastError();
}

hipError_t launch_select_talker(const SelectTalkerArgs &a, hipStream_t s, int rows) {
  if (a.V > kMaxVocab || a.V < 1024) return hipErrorInvalidValue;
  if (rows < 1 || rows > kMaxRows || (rows > 1 && (!a.row_on || a.codes_row <= 0 || (a.trace && a.trace_row <= 0))))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_select_talker, dim3(rows), dim3(1024), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_select_cp(const SelectCpArgs &a, hipStream_t s, int rows) {
  if (a.Vc < 1 || a.Vc > kMaxVocab || a.Ht < 1 || a.Ht > 2048) return hipErrorInvalidValue;
  if (a.token_only && (rows != 1 || !a.tok_out || a.group >= a.groups - 2)) return hipErrorInvalidValue;
  if (rows < 1 || rows > kMaxRows ||
      (rows > 1 && (!a.row_on || a.codes_row <= 0 || a.trailing_row <= 0 || (a.trace && a.trace_row <= 0) ||
                    a.tok_out)))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_select_cp, dim3(rows), dim3(1024), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_sample_draws(const float *logits, int V, const SamplingParams &sp, uint64_t seed, int kind, int n,
                               int32_t *out, hipStream_t s) {
  if (V <= 0 || V > kMaxVocab || n <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_sample_draws, dim3(n), dim3(1024), 0, s, logits, V, sp, (uint32_t)(seed & 0xffffffffu),
                     (uint32_t)(seed >> 32), kind, out);
  return hipGetLastError();
}

// The no-allocation scratch.  Each GPU holds its own copy of the array, at its own address,
// until the process ends.  In host code `scratch` names a host-side stand-in, never a device
// address: host code uses only the pointer hipGetSymbolAddress returns for the device.
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};
}  // namespace

hipError_t noalloc_scratch_setup(int device) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device]) return hipSuccess;
  int current = -1;
  hipError_t err = hipGetDevice(&current);
  if (err != hipSuccess) return err;
  if (current != device) return hipErrorInvalidDevice;
  void *ptr = nullptr;
  err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (err != hipSuccess) return err;
  if (!ptr) return hipErrorInvalidSymbol;
  g_scratch_ptr[device] = ptr;
  return hipSuccess;
}

void *noalloc_scratch(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  return g_scratch_ptr[device];
}

}  // namespace q3t
