// The Gated DeltaNet layer's neighbour ops for gfx950: GatedDeltaRuleGates, GatedRmsNorm, SigmoidMul, CausalConv1d and
// the recurrent-state copies (ROOST_OP_GATED_DELTA_RULE_GATES, _GATED_RMS_NORM, _SIGMOID_MUL, _CAUSAL_CONV1D,
// _RECURRENT_STATE_COPY, _RECURRENT_STATE_SNAPSHOT).
//
// Semantics: src/Starlings.Roost.Ops/CpuOps.Gating.cs:21-101 and CpuOps.Hybrid.cs:160-263 (the formulas and element
// types), with the reference entry points' refusal rules (kernels/src/ops/gating.cu:110-268, causal_conv1d.cu:122-175,
// recurrent_state.cu:58-108). Every element is computed in fp32 and rounded once into its span's type.
//
// All of them are HBM-bound streams (a few flops per byte). The kernels read each input element once with 16-byte
// vector loads where the layout allows, reduce in a fixed order (deterministic and batch invariant: no result depends
// on another row, token or sequence), allocate nothing and use only the caller's stream (graph capturable).

#include <cmath>

#include "common.h"
#include "gdn_layer.h"

namespace {

using namespace roost_dev;

__device__ __forceinline__ void StoreF(void* p, uint32_t dt, int64_t i, float v) {
  if (dt == ROOST_DTYPE_BF16) {
    static_cast<uint16_t*>(p)[i] = F32ToBf16(v);
  } else {
    static_cast<float*>(p)[i] = v;
  }
}

// ---- GatedDeltaRuleGates -------------------------------------------------------------------------------------------
// g = -exp(a_log[h]) * softplus(a[t, h] + dt_bias[h]) (softplus(x) = x above 20), beta = sigmoid(b[t, h]). One thread per
// (token, head); a and b are row-strided column views.
__global__ void __launch_bounds__(256) GatesKernel(const void* a, const void* b, const void* a_log, const void* dt_bias,
                                                   void* g, void* beta, uint32_t a_t, uint32_t b_t, uint32_t alog_t,
                                                   uint32_t dtb_t, uint32_t g_t, uint32_t beta_t, uint64_t total,
                                                   uint32_t v_heads, uint64_t a_stride, uint64_t b_stride) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const uint64_t t = i / v_heads;
  const uint32_t h = static_cast<uint32_t>(i - t * v_heads);
  float gv, bv;
  GateValues(LoadF(a, a_t, static_cast<int64_t>(t * a_stride + h)), LoadF(dt_bias, dtb_t, h), LoadF(a_log, alog_t, h),
             LoadF(b, b_t, static_cast<int64_t>(t * b_stride + h)), gv, bv);
  StoreF(g, g_t, static_cast<int64_t>(i), gv);
  StoreF(beta, beta_t, static_cast<int64_t>(i), bv);
}

// ---- GatedRmsNorm --------------------------------------------------------------------------------------------------
// out = x * rsqrt(mean(x^2) + eps) * weight * silu(gate) per row. A row is served by G lanes (a power of two, G <= 64),
// 64 / G rows per wavefront; each lane takes kV consecutive elements at a time (16-byte loads when kVec). The sum of
// squares is reduced over the G lanes by a fixed xor butterfly.
// kV consecutive elements of a bf16 or f32 row as floats: one 16-byte load when kVec.
template <typename T, bool kVec>
__device__ __forceinline__ void LoadRun(const T* p, uint64_t k, float* v) {
  constexpr int kV = kVec ? 16 / static_cast<int>(sizeof(T)) : 1;
  if constexpr (kVec) {
    const uint4 q = *reinterpret_cast<const uint4*>(p + k);
    const uint32_t* qw = reinterpret_cast<const uint32_t*>(&q);
#pragma unroll
    for (int e = 0; e < kV; ++e) {
      v[e] = sizeof(T) == 2 ? ((e & 1) ? Bf16HiToF32(qw[e >> 1]) : Bf16LoToF32(qw[e >> 1])) : __uint_as_float(qw[e]);
    }
  } else {
    v[0] = sizeof(T) == 2 ? Bf16ToF32(reinterpret_cast<const uint16_t*>(p)[k]) : reinterpret_cast<const float*>(p)[k];
  }
}

template <typename T, bool kVec>
__device__ __forceinline__ void StoreRun(T* p, uint64_t k, const float* v) {
  constexpr int kV = kVec ? 16 / static_cast<int>(sizeof(T)) : 1;
  if constexpr (kVec) {
    uint4 q;
    uint32_t* qw = reinterpret_cast<uint32_t*>(&q);
#pragma unroll
    for (int w = 0; w < 4; ++w) qw[w] = sizeof(T) == 2 ? PackBf16Rne(v[2 * w], v[2 * w + 1]) : __float_as_uint(v[w]);
    *reinterpret_cast<uint4*>(p + k) = q;
  } else if constexpr (sizeof(T) == 2) {
    reinterpret_cast<uint16_t*>(p)[k] = F32ToBf16(v[0]);
  } else {
    reinterpret_cast<float*>(p)[k] = v[0];
  }
  (void)kV;
}

template <typename T, bool kVec>
__global__ void __launch_bounds__(256) GatedRmsNormKernel(const T* __restrict__ x, const T* __restrict__ gate,
                                                          const void* __restrict__ weight, uint32_t w_t,
                                                          T* __restrict__ out, uint64_t rows, uint32_t dim,
                                                          uint32_t lanes_per_row, float eps) {
  constexpr int kV = kVec ? 16 / static_cast<int>(sizeof(T)) : 1;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t sub = lane % lanes_per_row;
  const uint64_t row = (static_cast<uint64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * (64 / lanes_per_row) +
                       lane / lanes_per_row;
  const bool live = row < rows;
  const uint64_t base = (live ? row : 0) * dim;
  float ss = 0.0f;
  for (uint32_t i = sub * kV; i < dim; i += lanes_per_row * kV) {
    float v[kV];
    LoadRun<T, kVec>(x, base + i, v);
#pragma unroll
    for (int e = 0; e < kV; ++e) ss = fmaf(v[e], v[e], ss);
  }
  for (uint32_t m = 1; m < lanes_per_row; m <<= 1) ss += __shfl_xor(ss, static_cast<int>(m), 64);
  if (!live) return;
  const float inv = rsqrtf(ss / static_cast<float>(dim) + eps);
  for (uint32_t i = sub * kV; i < dim; i += lanes_per_row * kV) {
    float xv[kV], gv[kV], y[kV];
    LoadRun<T, kVec>(x, base + i, xv);
    LoadRun<T, kVec>(gate, base + i, gv);
#pragma unroll
    for (int e = 0; e < kV; ++e) y[e] = xv[e] * inv * LoadF(weight, w_t, i + e) * SiluF(gv[e]);
    StoreRun<T, kVec>(out, base + i, y);
  }
}

// Single-pass form for 16-byte vectors when one vector per lane covers the row (lanes_per_row * kV == dim, the Qwen
// head dims): each thread serves kR rows spaced one block-row apart, issues all of their x and gate loads before any
// arithmetic, keeps the row in registers (x is read once) and loads its kV weights once for all kR rows.
constexpr int kRmsRows = 4;

// LoadWords with the non-temporal hint, for rows read once in whole lines (the tiled convolution's input rows, the
// chunk layer's norm inputs).
template <int kBytes>
__device__ __forceinline__ void LoadWordsNt(const void* p, uint32_t* w) {
  typedef uint32_t v4 __attribute__((ext_vector_type(4)));
  typedef uint32_t v2 __attribute__((ext_vector_type(2)));
  if constexpr (kBytes == 16) {
    const v4 q = __builtin_nontemporal_load(static_cast<const v4*>(p));
    w[0] = q[0]; w[1] = q[1]; w[2] = q[2]; w[3] = q[3];
  } else if constexpr (kBytes == 8) {
    const v2 q = __builtin_nontemporal_load(static_cast<const v2*>(p));
    w[0] = q[0]; w[1] = q[1];
  } else {
    w[0] = __builtin_nontemporal_load(static_cast<const uint32_t*>(p));
  }
}
template <typename T, int kR, bool kStream = false>
__device__ __forceinline__ void GatedRmsNormRows(const T* __restrict__ x, const T* __restrict__ gate,
                                                 const void* __restrict__ weight, uint32_t w_t, T* __restrict__ out,
                                                 uint64_t rows, uint32_t dim, uint32_t lanes_per_row, float eps,
                                                 uint32_t block) {
  constexpr int kV = 16 / static_cast<int>(sizeof(T));
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t sub = lane % lanes_per_row;
  const uint64_t rows_per_pass = 4ull * (64 / lanes_per_row);  // rows one pass of the block covers
  const uint64_t row0 = static_cast<uint64_t>(block) * rows_per_pass * kR +
                        (threadIdx.x >> 6) * (64 / lanes_per_row) + lane / lanes_per_row;
  const uint32_t col = sub * kV;
  uint4 xq[kR], gq[kR];
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    const uint64_t row = row0 + r * rows_per_pass;
    const uint64_t at = (row < rows ? row : 0) * dim + col;
    if constexpr (kStream) {  // both streams read once, past the caches
      uint32_t t[4];
      LoadWordsNt<16>(x + at, t);
      xq[r] = make_uint4(t[0], t[1], t[2], t[3]);
      LoadWordsNt<16>(gate + at, t);
      gq[r] = make_uint4(t[0], t[1], t[2], t[3]);
    } else {
      xq[r] = *reinterpret_cast<const uint4*>(x + at);
      gq[r] = *reinterpret_cast<const uint4*>(gate + at);
    }
  }
  float wv[kV];
  if (w_t == ROOST_DTYPE_F32 && (reinterpret_cast<uintptr_t>(weight) & 15) == 0) {
    const float4* wp = reinterpret_cast<const float4*>(static_cast<const float*>(weight) + col);
#pragma unroll
    for (int q = 0; q < kV / 4; ++q) {
      const float4 f = wp[q];
      wv[4 * q] = f.x; wv[4 * q + 1] = f.y; wv[4 * q + 2] = f.z; wv[4 * q + 3] = f.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < kV; ++e) wv[e] = LoadF(weight, w_t, col + e);
  }
  auto unpack = [](const uint4& q, float* v) {
    const uint32_t* qw = reinterpret_cast<const uint32_t*>(&q);
#pragma unroll
    for (int e = 0; e < kV; ++e) {
      v[e] = sizeof(T) == 2 ? ((e & 1) ? Bf16HiToF32(qw[e >> 1]) : Bf16LoToF32(qw[e >> 1])) : __uint_as_float(qw[e]);
    }
  };
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    float xv[kV], gv[kV], y[kV];
    unpack(xq[r], xv);
    unpack(gq[r], gv);
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < kV; ++e) ss = fmaf(xv[e], xv[e], ss);
    for (uint32_t m = 1; m < lanes_per_row; m <<= 1) ss += __shfl_xor(ss, static_cast<int>(m), 64);
    const float inv = rsqrtf(ss / static_cast<float>(dim) + eps);
#pragma unroll
    for (int e = 0; e < kV; ++e) y[e] = xv[e] * inv * wv[e] * SiluF(gv[e]);
    const uint64_t row = row0 + r * rows_per_pass;
    if (row < rows) StoreRun<T, true>(out, row * dim + col, y);
  }
}
template <typename T, int kR, bool kStream = false>
__global__ void __launch_bounds__(256) GatedRmsNormRowKernel(const T* __restrict__ x, const T* __restrict__ gate,
                                                             const void* __restrict__ weight, uint32_t w_t,
                                                             T* __restrict__ out, uint64_t rows, uint32_t dim,
                                                             uint32_t lanes_per_row, float eps) {
  GatedRmsNormRows<T, kR, kStream>(x, gate, weight, w_t, out, rows, dim, lanes_per_row, eps, blockIdx.x);
}

// ---- SigmoidMul ----------------------------------------------------------------------------------------------------
// out = x * sigmoid(gate), kV elements per step (16-byte loads and stores when kVec), grid-stride.
template <typename T, bool kVec>
__global__ void __launch_bounds__(256) SigmoidMulKernel(const T* __restrict__ x, const T* __restrict__ gate,
                                                        T* __restrict__ out, uint64_t n) {
  constexpr int kV = kVec ? 16 / static_cast<int>(sizeof(T)) : 1;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x * kV;
  for (uint64_t i = (static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * kV; i < n; i += stride) {
    if constexpr (kVec) {
      const uint4 xv = *reinterpret_cast<const uint4*>(x + i);
      const uint4 gv = *reinterpret_cast<const uint4*>(gate + i);
      uint4 ov;
      const uint32_t* xw = reinterpret_cast<const uint32_t*>(&xv);
      const uint32_t* gw = reinterpret_cast<const uint32_t*>(&gv);
      uint32_t* ow = reinterpret_cast<uint32_t*>(&ov);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        if constexpr (sizeof(T) == 2) {
          ow[w] = GateMulBf16x2(xw[w], gw[w]);
        } else {
          ow[w] = __float_as_uint(GateMul(__uint_as_float(xw[w]), __uint_as_float(gw[w])));
        }
      }
      *reinterpret_cast<uint4*>(out + i) = ov;
    } else {
      out[i] = GateMul(x[i], gate[i]);
    }
  }
}

// ---- CausalConv1d --------------------------------------------------------------------------------------------------
// y_t = bias + sum_j w[c, j] * h_{t + j} over h = [conv state (width - 1, oldest first), the sequence's inputs], SiLU
// last when set. Workgroup column blockIdx.x is one token; its sequence is found by a binary search of cu_seqlens (uniform,
// scalar loads). A thread computes kV consecutive channels (8 bf16 / 4 f32 from one 16-byte load per tap when kVec);
// the taps re-read neighbouring tokens' inputs from cache. A slot outside the pool reads a zero history.
struct ConvArgs {
  const void* x;
  const void* w;
  const void* bias;  // NULL: none
  void* y;
  void* state;
  const int32_t* slots;
  const int32_t* cu;
  uint32_t act_t, state_t;
  uint32_t batch, tokens, channels, width, silu;
  uint64_t pool_slots;
};

__device__ __forceinline__ int32_t SeqOfToken(const int32_t* cu, uint32_t batch, int32_t t, uint32_t tokens) {
  // The sequence b with cu[b] <= t < cu[b + 1] (empty sequences are skipped by the upper-bound search). The search
  // starts from the sequence equal lengths would put t in (exact for a decode step, where every sequence is one
  // token), so a batch of even lengths costs two loads instead of log2(batch) dependent ones.
  uint32_t lo = 0, hi = batch;  // invariant: cu[lo] <= t, answer in [lo, hi)
  if (batch > 1 && tokens > 0) {
    const uint32_t g = static_cast<uint32_t>(min<uint64_t>(uint64_t(t) * batch / tokens, batch - 1));
    const int32_t at = cu[g], next = cu[g + 1];
    if (at <= t && t < next) return static_cast<int32_t>(g);
    if (at <= t) lo = g; else hi = g;
  }
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) >> 1;
    if (cu[mid] <= t) lo = mid; else hi = mid;
  }
  return static_cast<int32_t>(lo);
}

// A run of kBytes / sizeof(T) consecutive channels: one 4-, 8- or 16-byte load or store.
template <int kBytes>
__device__ __forceinline__ void LoadWords(const void* p, uint32_t* w) {
  if constexpr (kBytes == 16) {
    const uint4 q = *static_cast<const uint4*>(p);
    w[0] = q.x; w[1] = q.y; w[2] = q.z; w[3] = q.w;
  } else if constexpr (kBytes == 8) {
    const uint2 q = *static_cast<const uint2*>(p);
    w[0] = q.x; w[1] = q.y;
  } else {
    w[0] = *static_cast<const uint32_t*>(p);
  }
}
template <int kBytes>
__device__ __forceinline__ void StoreWords(void* p, const uint32_t* w) {
  if constexpr (kBytes == 16) {
    *static_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  } else if constexpr (kBytes == 8) {
    *static_cast<uint2*>(p) = make_uint2(w[0], w[1]);
  } else {
    *static_cast<uint32_t*>(p) = w[0];
  }
}
template <typename T, int kWords>
__device__ __forceinline__ void UnpackWords(const uint32_t* w, float* v) {
  constexpr int kV = kWords * 4 / static_cast<int>(sizeof(T));
#pragma unroll
  for (int e = 0; e < kV; ++e) {
    v[e] = sizeof(T) == 2 ? ((e & 1) ? Bf16HiToF32(w[e >> 1]) : Bf16LoToF32(w[e >> 1])) : __uint_as_float(w[e]);
  }
}
template <typename T, int kWords>
__device__ __forceinline__ void PackWords(const float* v, uint32_t* w) {
#pragma unroll
  for (int q = 0; q < kWords; ++q) w[q] = sizeof(T) == 2 ? PackBf16Rne(v[2 * q], v[2 * q + 1]) : __float_as_uint(v[q]);
}

// Tiled form for a compile-time width and channel vectors of kBytes (kV channels per thread). Workgroup b serves token
// tile b / cblocks (kConvTile tokens) and channel block b % cblocks (consecutive workgroups cover one row). A thread keeps
// the last kW - 1 inputs of its channels in registers, so every input row is read once plus a kW - 1 row halo per tile,
// and loads its kV x kW weights once. Narrow vectors (8 bytes for bf16) keep the register count low enough for eight
// waves per SIMD, which with long tiles keeps the halo small while the grid still fills the chip several times over.
// Zeros in device memory, read in place of an absent bias so that the request needs no branch.
__device__ __align__(16) uint32_t kConvZeros[4] = {0u, 0u, 0u, 0u};

constexpr int kConvTile = 32;
constexpr int kConvChunk = 4;  // rows requested ahead of the arithmetic

template <typename T, int kW, int kBytes>
__global__ void __launch_bounds__(256) ConvTileKernel(ConvArgs a, uint32_t cblocks) {
  constexpr int kWords = kBytes / 4;
  constexpr int kV = kBytes / static_cast<int>(sizeof(T));
  const uint32_t tile = blockIdx.x / cblocks;
  const int32_t t_begin = static_cast<int32_t>(tile) * kConvTile;
  const uint32_t c0 = ((blockIdx.x - tile * cblocks) * blockDim.x + threadIdx.x) * kV;
  if (c0 >= a.channels) return;
  const int32_t t_end = min(t_begin + kConvTile, static_cast<int32_t>(a.tokens));
  const T* x = static_cast<const T*>(a.x);
  auto row_at = [&](int32_t t, float* v) {
    uint32_t q[kWords];
    LoadWords<kBytes>(x + static_cast<uint64_t>(t) * a.channels + c0, q);
    UnpackWords<T, kWords>(q, v);
  };
  // Weights of channels c0 .. c0 + kV - 1: kV * kW consecutive elements, channel-major (kBytes-aligned: the launcher
  // checks the base). Weights and bias are requested as words without a branch (no bias: zeros from kConvZeros) and
  // unpacked after: a request inside a branch, used there, waited for everything before it.
  float w[kV][kW];
  float bias[kV];
  {
    uint32_t qw[kW][kWords], qb[kWords];
    const T* wrow = static_cast<const T*>(a.w) + static_cast<uint64_t>(c0) * kW;
#pragma unroll
    for (int q = 0; q < kW; ++q) LoadWords<kBytes>(wrow + q * kV, qw[q]);
    LoadWords<kBytes>(a.bias != nullptr ? static_cast<const T*>(a.bias) + c0 : reinterpret_cast<const T*>(kConvZeros),
                      qb);
    float flat[kV * kW];
#pragma unroll
    for (int q = 0; q < kW; ++q) UnpackWords<T, kWords>(qw[q], flat + q * kV);
#pragma unroll
    for (int e = 0; e < kV; ++e)
#pragma unroll
      for (int j = 0; j < kW; ++j) w[e][j] = flat[e * kW + j];
    UnpackWords<T, kWords>(qb, bias);
  }

  const int32_t seq0 = SeqOfToken(a.cu, a.batch, t_begin, a.tokens);
  const int32_t s0 = a.cu[seq0], s1 = a.cu[seq0 + 1];
  // Entry i of [state (kW - 1), inputs] of sequence `seq` (first token `first`) for channels c0.., as floats.
  auto history = [&](int32_t seq, int32_t first, int32_t i, float* v) {
    if (i < kW - 1) {
      const int32_t slot = a.slots[seq];
      const bool ok = slot >= 0 && static_cast<uint64_t>(slot) < a.pool_slots;
      const uint64_t so = static_cast<uint64_t>(ok ? slot : 0) * a.channels * (kW - 1);
#pragma unroll
      for (int e = 0; e < kV; ++e) v[e] = ok ? LoadF(a.state, a.state_t, so + (c0 + e) * (kW - 1) + i) : 0.0f;
    } else {
      row_at(first + i - (kW - 1), v);
    }
  };
  auto emit = [&](int32_t t, const float (*taps)[kV], const float* cur) {
    float y[kV];
#pragma unroll
    for (int e = 0; e < kV; ++e) {
      float acc = bias[e];
#pragma unroll
      for (int j = 0; j < kW - 1; ++j) acc = fmaf(w[e][j], taps[j][e], acc);
      acc = fmaf(w[e][kW - 1], cur[e], acc);
      y[e] = a.silu ? SiluF(acc) : acc;
    }
    uint32_t q[kWords];
    PackWords<T, kWords>(y, q);
    StoreWords<kBytes>(static_cast<T*>(a.y) + static_cast<uint64_t>(t) * a.channels + c0, q);
  };
  float h[kW - 1][kV];  // the window: h[kW - 2] is the newest input

  if (t_begin >= s0 && t_end <= s1) {
    // The whole tile lies in one sequence (every tile but those at sequence boundaries): one window load, then a
    // straight-line slide over the tile's rows, the next kConvChunk rows requested before the current ones are computed.
    // The rows stream in with the non-temporal hint (Qwen3.5's [16384, 6144] projection: 74.6 against 86.0 us); the
    // window's halo rows, which the tile before also reads, keep plain loads.
    auto fetch = [&](int32_t t0, uint32_t (*r)[kWords]) {
#pragma unroll
      for (int i = 0; i < kConvChunk; ++i) {
        LoadWordsNt<kBytes>(x + static_cast<uint64_t>(min(t0 + i, t_end - 1)) * a.channels + c0, r[i]);
      }
    };
    uint32_t rows[kConvChunk][kWords], next[kConvChunk][kWords];
    fetch(t_begin, rows);
#pragma unroll
    for (int j = 0; j < kW - 1; ++j) history(seq0, s0, t_begin - s0 + j, h[j]);
#pragma unroll 1
    for (int32_t tc = t_begin; tc < t_end; tc += kConvChunk) {
      if (tc + kConvChunk < t_end) fetch(tc + kConvChunk, next);
#pragma unroll
      for (int i = 0; i < kConvChunk; ++i) {
        const int32_t t = tc + i;
        if (t >= t_end) break;
        float cur[kV];
        UnpackWords<T, kWords>(rows[i], cur);
        emit(t, h, cur);
#pragma unroll
        for (int j = 0; j + 1 < kW - 1; ++j)
#pragma unroll
          for (int e = 0; e < kV; ++e) h[j][e] = h[j + 1][e];
#pragma unroll
        for (int e = 0; e < kV; ++e) h[kW - 2][e] = cur[e];
      }
#pragma unroll
      for (int i = 0; i < kConvChunk; ++i)
#pragma unroll
        for (int q = 0; q < kWords; ++q) rows[i][q] = next[i][q];
    }
    return;
  }
  // A tile that crosses a sequence boundary (or holds tokens outside every sequence): token by token, each tap read
  // directly from the state or the inputs (the sequence is uniform across the workgroup: every thread shares the token).
  int32_t seq = seq0;
#pragma unroll 1
  for (int32_t t = t_begin; t < t_end; ++t) {
    while (seq + 1 < static_cast<int32_t>(a.batch) && a.cu[seq + 1] <= t) ++seq;
    const int32_t first = a.cu[seq];
    if (t < first || t >= a.cu[seq + 1]) continue;  // a token outside every sequence: no output
    const int32_t rel = t - first;
#pragma unroll
    for (int j = 0; j < kW - 1; ++j) history(seq, first, rel + j, h[j]);
    float cur[kV];
    row_at(t, cur);
    emit(t, h, cur);
  }
}

// Short-sequence form (a decode step: tokens per sequence below a tile) for bf16 rows, widths 2-4 and 16-byte aligned
// buffers: one thread per (token, 8 channels), every operand one 16-byte vector -- the 8 channels' taps of weights, their
// bias, their state entries (contiguous per channel) and each needed input row -- with the weights requested before the
// token's sequence is looked up. Same arithmetic as the other forms.
template <int kW>
__global__ void __launch_bounds__(256) ConvShortKernel(ConvArgs a) {
  constexpr int kV = 8, sl = kW - 1;
  constexpr int kSq = sl > 0 ? 2 * sl : 1;  // 16-byte state words: sl for bf16, 2 sl for f32
  const int32_t t = static_cast<int32_t>(blockIdx.x);
  const uint32_t c0 = (blockIdx.y * blockDim.x + threadIdx.x) * kV;
  if (c0 >= a.channels) return;
  // Every operand is requested as raw words first (no bias: zeros from kConvZeros; the state and input words in
  // branches that do not use them) and unpacked after: a thread lives for a few round trips, and a request used
  // inside its own branch waited for everything requested before it.
  uint32_t wq[kW][4], bq[4];
  const auto* wp = static_cast<const uint16_t*>(a.w) + static_cast<uint64_t>(c0) * kW;
#pragma unroll
  for (int q = 0; q < kW; ++q) LoadWords<16>(wp + 8 * q, wq[q]);
  LoadWords<16>(a.bias != nullptr ? static_cast<const uint16_t*>(a.bias) + c0
                                  : reinterpret_cast<const uint16_t*>(kConvZeros),
                bq);
  const int32_t b = SeqOfToken(a.cu, a.batch, t, a.tokens);
  const int32_t t0 = a.cu[b];
  if (t < t0 || t >= a.cu[b + 1]) return;  // a token outside every sequence (cu does not cover it): no output
  const int32_t rel = t - t0;              // tap j of this token is entry rel + j of [state, inputs]
  const bool bf_state = a.state_t == ROOST_DTYPE_BF16;
  const int32_t slot = rel < sl ? a.slots[b] : -1;
  const bool ok = slot >= 0 && static_cast<uint64_t>(slot) < a.pool_slots;
  uint32_t sq[kSq][4] = {};
  if (rel < sl) {  // some taps come from the state: the 8 channels' entries are 8 x sl contiguous elements
    const uint64_t so = (static_cast<uint64_t>(ok ? slot : 0) * a.channels + c0) * sl;
    if (bf_state) {
#pragma unroll
      for (int q = 0; q < sl; ++q) LoadWords<16>(static_cast<const uint16_t*>(a.state) + so + 8 * q, sq[q]);
    } else {
#pragma unroll
      for (int q = 0; q < 2 * sl; ++q) LoadWords<16>(static_cast<const float*>(a.state) + so + 4 * q, sq[q]);
    }
  }
  const auto* x = static_cast<const uint16_t*>(a.x);
  uint32_t xq[kW][4] = {};
#pragma unroll
  for (int j = 0; j < kW; ++j) {
    const int32_t hi = rel + j;
    if (hi >= sl) LoadWords<16>(x + static_cast<uint64_t>(t0 + hi - sl) * a.channels + c0, xq[j]);
  }
  float w[kV][kW];
  {
    float flat[kV * kW];
#pragma unroll
    for (int q = 0; q < kW; ++q) UnpackWords<uint16_t, 4>(wq[q], flat + 8 * q);
#pragma unroll
    for (int e = 0; e < kV; ++e)
#pragma unroll
      for (int j = 0; j < kW; ++j) w[e][j] = flat[e * kW + j];
  }
  float acc[kV];
  UnpackWords<uint16_t, 4>(bq, acc);
  float st[kV][sl > 0 ? sl : 1];
  if (rel < sl) {
    float flat[kV * (sl > 0 ? sl : 1)];
    if (bf_state) {
#pragma unroll
      for (int q = 0; q < sl; ++q) UnpackWords<uint16_t, 4>(sq[q], flat + 8 * q);
    } else {
#pragma unroll
      for (int q = 0; q < 2 * sl; ++q) UnpackWords<float, 4>(sq[q], flat + 4 * q);
    }
#pragma unroll
    for (int e = 0; e < kV; ++e)
#pragma unroll
      for (int i = 0; i < sl; ++i) st[e][i] = ok ? flat[e * sl + i] : 0.0f;
  }
#pragma unroll
  for (int j = 0; j < kW; ++j) {
    const int32_t hi = rel + j;
    float tap[kV];
    if (hi < sl) {
#pragma unroll
      for (int e = 0; e < kV; ++e) tap[e] = st[e][hi < sl ? hi : 0];
    } else {
      UnpackWords<uint16_t, 4>(xq[j], tap);
    }
#pragma unroll
    for (int e = 0; e < kV; ++e) acc[e] = fmaf(w[e][j], tap[e], acc[e]);
  }
  float y[kV];
#pragma unroll
  for (int e = 0; e < kV; ++e) y[e] = a.silu ? SiluF(acc[e]) : acc[e];
  uint32_t q[4];
  PackWords<uint16_t, 4>(y, q);
  StoreWords<16>(static_cast<uint16_t*>(a.y) + static_cast<uint64_t>(t) * a.channels + c0, q);
}

// General form (any width, any channel count): one thread per (token, kV channels), taps loaded per output.
template <typename T, bool kVec>
__global__ void __launch_bounds__(256) ConvKernel(ConvArgs a) {
  constexpr int kV = kVec ? 16 / static_cast<int>(sizeof(T)) : 1;
  const int32_t t = static_cast<int32_t>(blockIdx.x);
  const uint32_t c0 = (blockIdx.y * blockDim.x + threadIdx.x) * kV;
  if (c0 >= a.channels) return;
  const int32_t b = SeqOfToken(a.cu, a.batch, t, a.tokens);
  const int32_t t0 = a.cu[b];
  if (t < t0 || t >= a.cu[b + 1]) return;  // a token outside every sequence (cu does not cover it): no output
  const int32_t slot = a.slots[b];
  const bool has_state = slot >= 0 && static_cast<uint64_t>(slot) < a.pool_slots;
  const int sl = static_cast<int>(a.width) - 1;
  const T* x = static_cast<const T*>(a.x);
  const T* w = static_cast<const T*>(a.w);
  float acc[kV];
#pragma unroll
  for (int e = 0; e < kV; ++e) acc[e] = a.bias != nullptr ? LoadF(a.bias, a.act_t, c0 + e) : 0.0f;
  const int32_t rel = t - t0;  // h index of this token's first tap is rel
  for (int j = 0; j < static_cast<int>(a.width); ++j) {
    const int32_t hi = rel + j;  // index into h = [state, inputs]
    float hv[kV];
    if (hi < sl) {
      const uint64_t so = (static_cast<uint64_t>(has_state ? slot : 0) * a.channels) * sl;
#pragma unroll
      for (int e = 0; e < kV; ++e) hv[e] = has_state ? LoadF(a.state, a.state_t, so + (c0 + e) * sl + hi) : 0.0f;
    } else {
      const uint64_t xo = static_cast<uint64_t>(t0 + hi - sl) * a.channels + c0;
      if constexpr (kVec) {
        const uint4 v = *reinterpret_cast<const uint4*>(x + xo);
        const uint32_t* vw = reinterpret_cast<const uint32_t*>(&v);
#pragma unroll
        for (int e = 0; e < kV; ++e) {
          hv[e] = sizeof(T) == 2 ? ((e & 1) ? Bf16HiToF32(vw[e >> 1]) : Bf16LoToF32(vw[e >> 1])) : __uint_as_float(vw[e]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < kV; ++e) hv[e] = LoadF(x, a.act_t, xo + e);
      }
    }
#pragma unroll
    for (int e = 0; e < kV; ++e) acc[e] = fmaf(LoadF(w, a.act_t, static_cast<uint64_t>(c0 + e) * a.width + j), hv[e], acc[e]);
  }
  const uint64_t yo = static_cast<uint64_t>(t) * a.channels + c0;
#pragma unroll
  for (int e = 0; e < kV; ++e) StoreF(a.y, a.act_t, yo + e, a.silu ? SiluF(acc[e]) : acc[e]);
}

// After ConvKernel (stream order): each (sequence, channel) slot keeps the last width - 1 entries of h. A thread reads
// them all (some may be old state entries) before writing any.
__global__ void __launch_bounds__(256) ConvStateKernel(ConvArgs a) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= static_cast<uint64_t>(a.batch) * a.channels) return;
  const uint32_t b = static_cast<uint32_t>(i / a.channels);
  const uint32_t c = static_cast<uint32_t>(i - static_cast<uint64_t>(b) * a.channels);
  const int32_t t0 = a.cu[b], t1 = a.cu[b + 1];
  const int32_t n = t1 - t0;
  const int32_t slot = a.slots[b];
  if (n <= 0 || slot < 0 || static_cast<uint64_t>(slot) >= a.pool_slots) return;  // untouched
  const int sl = static_cast<int>(a.width) - 1;
  const uint64_t so = (static_cast<uint64_t>(slot) * a.channels + c) * sl;
  float next[15];
#pragma unroll
  for (int j = 0; j < 15; ++j) {
    if (j < sl) {
      const int32_t hi = n + j;
      next[j] = hi < sl ? LoadF(a.state, a.state_t, so + hi)
                        : LoadF(a.x, a.act_t, static_cast<uint64_t>(t0 + hi - sl) * a.channels + c);
    }
  }
#pragma unroll
  for (int j = 0; j < 15; ++j) {
    if (j < sl) StoreF(a.state, a.state_t, so + j, next[j]);
  }
}

// The same update for bf16 inputs, widths 2-4 and 16-byte aligned buffers: one thread per (sequence, 8 channels), whose
// 8 x (width - 1) state entries are contiguous, so they are read and written as 16-byte vectors, and each input row it
// needs is one vector.
template <int kW>
__device__ __forceinline__ void ConvStateVecBlock(const ConvArgs& a, uint32_t b, uint32_t by) {
  constexpr int kV = 8, sl = kW - 1;
  const uint32_t c0 = (by * blockDim.x + threadIdx.x) * kV;
  if (c0 >= a.channels) return;
  const int32_t t0 = a.cu[b], t1 = a.cu[b + 1];
  const int32_t n = t1 - t0;
  const int32_t slot = a.slots[b];
  if (n <= 0 || slot < 0 || static_cast<uint64_t>(slot) >= a.pool_slots) return;  // untouched
  const uint64_t so = (static_cast<uint64_t>(slot) * a.channels + c0) * sl;
  const bool bf_state = a.state_t == ROOST_DTYPE_BF16;
  float old[kV * sl];  // [channel][entry], as stored
  if (n < sl) {        // some entries stay from the old state
    if (bf_state) {
#pragma unroll
      for (int q = 0; q < sl; ++q) {
        uint32_t qw[4];
        LoadWords<16>(static_cast<const uint16_t*>(a.state) + so + 8 * q, qw);
        UnpackWords<uint16_t, 4>(qw, old + 8 * q);
      }
    } else {
#pragma unroll
      for (int q = 0; q < 2 * sl; ++q) {
        uint32_t qw[4];
        LoadWords<16>(static_cast<const float*>(a.state) + so + 4 * q, qw);
        UnpackWords<float, 4>(qw, old + 4 * q);
      }
    }
  }
  float next[kV * sl];
#pragma unroll
  for (int j = 0; j < sl; ++j) {
    const int32_t hi = n + j;  // entry j of the new state is entry hi of [state, inputs]
    if (hi < sl) {
#pragma unroll
      for (int e = 0; e < kV; ++e) next[e * sl + j] = old[e * sl + (hi < sl ? hi : 0)];
    } else {
      uint32_t qw[4];
      float v[kV];
      LoadWords<16>(static_cast<const uint16_t*>(a.x) + static_cast<uint64_t>(t0 + hi - sl) * a.channels + c0, qw);
      UnpackWords<uint16_t, 4>(qw, v);
#pragma unroll
      for (int e = 0; e < kV; ++e) next[e * sl + j] = v[e];
    }
  }
  if (bf_state) {
#pragma unroll
    for (int q = 0; q < sl; ++q) {
      uint32_t qw[4];
      PackWords<uint16_t, 4>(next + 8 * q, qw);
      StoreWords<16>(static_cast<uint16_t*>(a.state) + so + 8 * q, qw);
    }
  } else {
#pragma unroll
    for (int q = 0; q < 2 * sl; ++q) {
      uint32_t qw[4];
      PackWords<float, 4>(next + 4 * q, qw);
      StoreWords<16>(static_cast<float*>(a.state) + so + 4 * q, qw);
    }
  }
}
template <int kW>
__global__ void __launch_bounds__(256) ConvStateVecKernel(ConvArgs a) {
  ConvStateVecBlock<kW>(a, blockIdx.x, blockIdx.y);
}

// ---- Recurrent-state copies ----------------------------------------------------------------------------------------
// A slot is cut into units (16 bytes when sizes and addresses allow, else single bytes). Each unit belongs to one
// thread, which applies the pairs to it in list order, so a pair that reads a slot an earlier pair wrote sees that
// write. The workgroup first resolves a batch of pairs into byte offsets in LDS (-1: a slot outside its pool, skipped)
// so that the pair list is read once per workgroup rather than once per unit.
constexpr uint32_t kPairBatch = 512;
constexpr uint32_t kUnitsPerThread = 4;

template <bool kVec>
__global__ void __launch_bounds__(256) SlotPairCopyKernel(const unsigned char* __restrict__ src, unsigned char* dst,
                                                          const int32_t* __restrict__ pairs, uint32_t count,
                                                          uint64_t slot_bytes, uint32_t from_col, uint64_t src_slots,
                                                          uint64_t dst_slots) {
  __shared__ int64_t offs[2][kPairBatch];
  const uint64_t units = kVec ? slot_bytes / 16 : slot_bytes;
  const uint64_t per_wg = static_cast<uint64_t>(blockDim.x) * kUnitsPerThread;
  const uint64_t first = static_cast<uint64_t>(blockIdx.x) * per_wg + threadIdx.x;
  for (uint32_t base = 0; base < count; base += kPairBatch) {
    const uint32_t n = min(kPairBatch, count - base);
    __syncthreads();  // the previous batch's offsets are no longer read
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
      const int32_t from = pairs[2 * (base + i) + from_col], to = pairs[2 * (base + i) + 1 - from_col];
      const bool ok = from >= 0 && to >= 0 && static_cast<uint64_t>(from) < src_slots &&
                      static_cast<uint64_t>(to) < dst_slots;
      offs[0][i] = ok ? static_cast<int64_t>(from) * static_cast<int64_t>(slot_bytes) : -1;
      offs[1][i] = ok ? static_cast<int64_t>(to) * static_cast<int64_t>(slot_bytes) : -1;
    }
    __syncthreads();
    for (uint32_t i = 0; i < n; ++i) {
      const int64_t f = offs[0][i], t = offs[1][i];
      if (f < 0) continue;
#pragma unroll
      for (uint32_t j = 0; j < kUnitsPerThread; ++j) {
        const uint64_t u = first + static_cast<uint64_t>(j) * blockDim.x;
        if (u >= units) break;
        if constexpr (kVec) {
          *reinterpret_cast<uint4*>(dst + t + 16 * u) = *reinterpret_cast<const uint4*>(src + f + 16 * u);
        } else {
          dst[t + u] = src[f + u];
        }
      }
    }
  }
}

bool FloatType(uint32_t dt) { return dt == ROOST_DTYPE_BF16 || dt == ROOST_DTYPE_F32; }
uint64_t ElemBytes(uint32_t dt) { return dt == ROOST_DTYPE_BF16 ? 2 : 4; }

// A span's byte range [first, end) when it is used for `elems` of its own elements.
struct ByteRange {
  uintptr_t first, end;
};
ByteRange Bytes(const RoostDeviceSpan& s, uint64_t elems) {
  const auto a = reinterpret_cast<uintptr_t>(s.address);
  return ByteRange{a, a + elems * ElemBytes(s.dtype)};
}
bool Intersect(ByteRange x, ByteRange y) { return x.first < y.end && y.first < x.end; }
// In-place use (the same first byte) is allowed; any other overlap is not.
bool Shifted(ByteRange x, ByteRange y) { return x.first != y.first && Intersect(x, y); }

// Rules every row op of this file shares: a float span of its own type (bf16 or f32), reserved word zero, an address
// when elements are needed, enough elements and natural alignment.
roost::Gate& FloatSpan(roost::Gate& gate, const char* name, const RoostDeviceSpan& s, uint64_t elems) {
  gate.Expect(FloatType(s.dtype), ROOST_STATUS_UNSUPPORTED, "%s is %s; built for bf16 and f32", name,
              roost::Describe(s.dtype).name);
  if (!gate.ok()) return gate;
  return gate.Tensor(name, s, s.dtype, elems).Aligned(name, s.address, static_cast<uint32_t>(ElemBytes(s.dtype)));
}

uint32_t Blocks(uint64_t items, uint32_t per_block) { return static_cast<uint32_t>(roost::CeilDiv(items, per_block)); }

// The entry-point preamble of this file's ops: a context, a params struct of a size and minor this library reads.
template <typename Params>
const Params* Preamble(roost::Gate& gate, RoostContext* ctx, const void* params) {
  gate.Expect(ctx != nullptr, ROOST_STATUS_INVALID_ARGUMENT, "no context was passed").Header(params, sizeof(Params));
  return gate.ok() ? static_cast<const Params*>(params) : nullptr;
}

// How GatedRmsNorm's run() serves a call: 16-byte vectors when the row and the buffers allow them, `lanes` lanes per
// row (a power of two up to 64, enough for one vector each), and the single-pass row kernel when one vector per lane
// covers the row.
struct NormShape {
  bool vec, single;
  uint32_t lanes;
};
NormShape NormForm(const RoostGatedRmsNormParams& p) {
  const uint32_t v = 16 / static_cast<uint32_t>(ElemBytes(p.input.dtype));
  NormShape f{};
  f.vec = p.dim % v == 0 && roost::IsAligned(p.input.address, 16) && roost::IsAligned(p.gate.address, 16) &&
          roost::IsAligned(p.output.address, 16);
  const uint32_t per_lane = f.vec ? v : 1;
  f.lanes = 1;
  while (f.lanes < 64 && f.lanes * per_lane < p.dim) f.lanes <<= 1;
  f.single = f.vec && f.lanes * per_lane == p.dim;
  return f;
}

}  // namespace

// ---- Entry points ---------------------------------------------------------------------------------------------------

extern "C" ROOST_API RoostStatus roost_gated_delta_rule_gates_run(RoostContext* ctx, const void* params,
                                                                   const RoostWorkspace*, void* stream) {
  constexpr char kOp[] = "gated_delta_rule_gates";
  roost::Gate gate(kOp);
  const auto* pp = Preamble<RoostGatedDeltaRuleGatesParams>(gate, ctx, params);
  ROOST_GATE_RETURN(gate);
  const auto& p = *pp;
  return roost::CatchAll(kOp, [&]() -> RoostStatus {
    gate.Expect(p.v_heads >= 1 && p.v_heads <= 0x7fffffffu, ROOST_STATUS_INVALID_ARGUMENT,
                "v_heads = %u outside 1..2^31-1", p.v_heads);
    ROOST_GATE_RETURN(gate);
    if (p.tokens == 0) return ROOST_STATUS_OK;
    const uint64_t vh = p.v_heads;
    const uint64_t as = p.a_stride == 0 ? vh : p.a_stride, bs = p.b_stride == 0 ? vh : p.b_stride;
    gate.Expect(as >= vh && bs >= vh, ROOST_STATUS_INVALID_ARGUMENT,
                "row strides a %llu, b %llu are narrower than the %llu value heads", static_cast<unsigned long long>(as),
                static_cast<unsigned long long>(bs), static_cast<unsigned long long>(vh));
    ROOST_GATE_RETURN(gate);
    const uint64_t total = uint64_t{p.tokens} * vh;
    const uint64_t a_reach = (p.tokens - 1ull) * as + vh, b_reach = (p.tokens - 1ull) * bs + vh;
    FloatSpan(gate, "a", p.a, a_reach);
    FloatSpan(gate, "b", p.b, b_reach);
    FloatSpan(gate, "a_log", p.a_log, vh);
    FloatSpan(gate, "dt_bias", p.dt_bias, vh);
    FloatSpan(gate, "g", p.g, total);
    FloatSpan(gate, "beta", p.beta, total);
    ROOST_GATE_RETURN(gate);
    // g and beta are written with no in-place form: they may share no byte with each other or with any input.
    const ByteRange g = Bytes(p.g, total), beta = Bytes(p.beta, total);
    const ByteRange inputs[] = {Bytes(p.a, a_reach), Bytes(p.b, b_reach), Bytes(p.a_log, vh), Bytes(p.dt_bias, vh)};
    bool clash = Intersect(g, beta);
    for (const ByteRange& in : inputs) clash = clash || Intersect(g, in) || Intersect(beta, in);
    gate.Expect(!clash, ROOST_STATUS_INVALID_ARGUMENT,
                "g or beta shares memory with the other or with an input; the gates are never computed in place")
        .Expect(total <= (uint64_t{1} << 40), ROOST_STATUS_INVALID_ARGUMENT, "%llu gate elements exceed one launch",
                static_cast<unsigned long long>(total));
    ROOST_GATE_RETURN(gate);
    hipLaunchKernelGGL(GatesKernel, dim3(Blocks(total, 256)), dim3(256), 0, roost::Stream(stream), p.a.address,
                       p.b.address, p.a_log.address, p.dt_bias.address, p.g.address, p.beta.address, p.a.dtype,
                       p.b.dtype, p.a_log.dtype, p.dt_bias.dtype, p.g.dtype, p.beta.dtype, total, p.v_heads, as, bs);
    return roost::HipStatus(hipGetLastError(), kOp, "kernel launch");
  });
}

RoostStatus roost_layer::AdmitNorm(const RoostGatedRmsNormParams& p, const char* op, bool* row_form) {
  roost::Gate gate(op);
  if (row_form != nullptr) *row_form = false;
  gate.Expect(p.reserved0 == 0, ROOST_STATUS_INVALID_ARGUMENT, "reserved0 = %u, must be 0", p.reserved0)
      .Expect(std::isfinite(p.eps) && p.eps >= 0.0f, ROOST_STATUS_INVALID_ARGUMENT,
              "eps = %g; a finite value >= 0 is required", p.eps)
      .Expect(p.dim >= 1 && p.dim <= 0x7fffffffu && p.rows <= 0x7fffffffu, ROOST_STATUS_INVALID_ARGUMENT,
              "dim = %u, rows = %u: dim must be 1..2^31-1 and rows at most 2^31-1", p.dim, p.rows);
  ROOST_GATE_RETURN(gate);
  if (p.rows == 0) return ROOST_STATUS_OK;
  const uint32_t act = p.input.dtype;
  const uint64_t n = uint64_t{p.rows} * p.dim;
  FloatSpan(gate, "input", p.input, n);
  FloatSpan(gate, "weight", p.weight, p.dim);
  ROOST_GATE_RETURN(gate);
  gate.Tensor("gate", p.gate, act, n)
      .Tensor("output", p.output, act, n)
      .Aligned("gate", p.gate.address, static_cast<uint32_t>(ElemBytes(act)))
      .Aligned("output", p.output.address, static_cast<uint32_t>(ElemBytes(act)))
      .Expect(!Shifted(Bytes(p.output, n), Bytes(p.input, n)) && !Shifted(Bytes(p.output, n), Bytes(p.gate, n)),
              ROOST_STATUS_INVALID_ARGUMENT,
              "output overlaps input or gate at another address; only an exact in-place alias is allowed");
  ROOST_GATE_RETURN(gate);
  if (row_form != nullptr) *row_form = NormForm(p).single;
  return ROOST_STATUS_OK;
}

namespace roost_layer {

RoostStatus RunNorm(const RoostGatedRmsNormParams& p, hipStream_t s, bool stream_input, const char* op) {
  if (p.rows == 0) return ROOST_STATUS_OK;
  const uint32_t act = p.input.dtype;
  const NormShape f = NormForm(p);
  const bool vec = f.vec, single = f.single;
  const uint32_t lanes = f.lanes;
  const uint64_t rows_per_block = 4ull * (64 / lanes);
  const dim3 grid(Blocks(p.rows, static_cast<uint32_t>(rows_per_block)));
  const dim3 row_grid(Blocks(p.rows, static_cast<uint32_t>(rows_per_block * kRmsRows)));
  if (act == ROOST_DTYPE_BF16) {
    const auto* x = static_cast<const uint16_t*>(p.input.address);
    const auto* g = static_cast<const uint16_t*>(p.gate.address);
    auto* o = static_cast<uint16_t*>(p.output.address);
    if (single) {
      auto* k = stream_input ? GatedRmsNormRowKernel<uint16_t, kRmsRows, true>
                             : GatedRmsNormRowKernel<uint16_t, kRmsRows, false>;
      hipLaunchKernelGGL(k, row_grid, dim3(256), 0, s, x, g, p.weight.address, p.weight.dtype, o, uint64_t{p.rows},
                         p.dim, lanes, p.eps);
    } else if (vec) {
      hipLaunchKernelGGL((GatedRmsNormKernel<uint16_t, true>), grid, dim3(256), 0, s, x, g, p.weight.address,
                         p.weight.dtype, o, uint64_t{p.rows}, p.dim, lanes, p.eps);
    } else {
      hipLaunchKernelGGL((GatedRmsNormKernel<uint16_t, false>), grid, dim3(256), 0, s, x, g, p.weight.address,
                         p.weight.dtype, o, uint64_t{p.rows}, p.dim, lanes, p.eps);
    }
  } else {
    const auto* x = static_cast<const float*>(p.input.address);
    const auto* g = static_cast<const float*>(p.gate.address);
    auto* o = static_cast<float*>(p.output.address);
    if (single) {
      auto* k = stream_input ? GatedRmsNormRowKernel<float, kRmsRows, true>
                             : GatedRmsNormRowKernel<float, kRmsRows, false>;
      hipLaunchKernelGGL(k, row_grid, dim3(256), 0, s, x, g, p.weight.address, p.weight.dtype, o, uint64_t{p.rows},
                         p.dim, lanes, p.eps);
    } else if (vec) {
      hipLaunchKernelGGL((GatedRmsNormKernel<float, true>), grid, dim3(256), 0, s, x, g, p.weight.address,
                         p.weight.dtype, o, uint64_t{p.rows}, p.dim, lanes, p.eps);
    } else {
      hipLaunchKernelGGL((GatedRmsNormKernel<float, false>), grid, dim3(256), 0, s, x, g, p.weight.address,
                         p.weight.dtype, o, uint64_t{p.rows}, p.dim, lanes, p.eps);
    }
  }
  return roost::HipStatus(hipGetLastError(), op, "kernel launch");
}

}  // namespace roost_layer

extern "C" ROOST_API RoostStatus roost_gated_rms_norm_run(RoostContext* ctx, const void* params, const RoostWorkspace*,
                                                           void* stream) {
  constexpr char kOp[] = "gated_rms_norm";
  roost::Gate gate(kOp);
  const auto* pp = Preamble<RoostGatedRmsNormParams>(gate, ctx, params);
  ROOST_GATE_RETURN(gate);
  const auto& p = *pp;
  return roost::CatchAll(kOp, [&]() -> RoostStatus {
    ROOST_RETURN_IF_FAILED(roost_layer::AdmitNorm(p, kOp, nullptr));
    return roost_layer::RunNorm(p, roost::Stream(stream), false, kOp);
  });
}

extern "C" ROOST_API RoostStatus roost_sigmoid_mul_run(RoostContext* ctx, const void* params, const RoostWorkspace*,
                                                        void* stream) {
  constexpr char kOp[] = "sigmoid_mul";
  roost::Gate gate(kOp);
  const auto* pp = Preamble<RoostSigmoidMulParams>(gate, ctx, params);
  ROOST_GATE_RETURN(gate);
  const auto& p = *pp;
  return roost::CatchAll(kOp, [&]() -> RoostStatus {
    const uint64_t n = uint64_t{p.rows} * p.dim;
    if (n == 0) return ROOST_STATUS_OK;
    const uint32_t act = p.input.dtype;
    FloatSpan(gate, "input", p.input, n);
    ROOST_GATE_RETURN(gate);
    gate.Tensor("gate", p.gate, act, n)
        .Tensor("output", p.output, act, n)
        .Aligned("gate", p.gate.address, static_cast<uint32_t>(ElemBytes(act)))
        .Aligned("output", p.output.address, static_cast<uint32_t>(ElemBytes(act)))
        .Expect(!Shifted(Bytes(p.output, n), Bytes(p.input, n)) && !Shifted(Bytes(p.output, n), Bytes(p.gate, n)),
                ROOST_STATUS_INVALID_ARGUMENT,
                "output overlaps input or gate at another address; only an exact in-place alias is allowed");
    ROOST_GATE_RETURN(gate);
    const uint64_t v = 16 / ElemBytes(act);
    const bool vec = n % v == 0 && roost::IsAligned(p.input.address, 16) && roost::IsAligned(p.gate.address, 16) &&
                     roost::IsAligned(p.output.address, 16);
    const uint64_t steps = vec ? n / v : n;
    const dim3 grid(static_cast<uint32_t>(std::min<uint64_t>(roost::CeilDiv(steps, 256), 65536)));
    hipStream_t s = roost::Stream(stream);
    if (act == ROOST_DTYPE_BF16) {
      const auto* x = static_cast<const uint16_t*>(p.input.address);
      const auto* g = static_cast<const uint16_t*>(p.gate.address);
      auto* o = static_cast<uint16_t*>(p.output.address);
      if (vec) hipLaunchKernelGGL((SigmoidMulKernel<uint16_t, true>), grid, dim3(256), 0, s, x, g, o, n);
      else hipLaunchKernelGGL((SigmoidMulKernel<uint16_t, false>), grid, dim3(256), 0, s, x, g, o, n);
    } else {
      const auto* x = static_cast<const float*>(p.input.address);
      const auto* g = static_cast<const float*>(p.gate.address);
      auto* o = static_cast<float*>(p.output.address);
      if (vec) hipLaunchKernelGGL((SigmoidMulKernel<float, true>), grid, dim3(256), 0, s, x, g, o, n);
      else hipLaunchKernelGGL((SigmoidMulKernel<float, false>), grid, dim3(256), 0, s, x, g, o, n);
    }
    return roost::HipStatus(hipGetLastError(), kOp, "kernel launch");
  });
}

RoostStatus roost_layer::AdmitConv(const RoostCausalConv1dParams& p, const char* op) {
  roost::Gate gate(op);
  gate.Expect(p.reserved0 == 0, ROOST_STATUS_INVALID_ARGUMENT, "reserved0 = %u, must be 0", p.reserved0)
      .Expect(p.width >= 1 && p.width <= 16 && p.channels > 0, ROOST_STATUS_INVALID_ARGUMENT,
              "width = %u, channels = %u: the filter spans 1..16 taps over at least one channel", p.width, p.channels)
      .Expect(p.channels <= 65535u * 128u && p.tokens <= 0x7fffffffu && p.batch <= 0x7fffffffu,
              ROOST_STATUS_INVALID_ARGUMENT, "%u channels, %u tokens, %u sequences exceed one launch", p.channels,
              p.tokens, p.batch);
  ROOST_GATE_RETURN(gate);
  if (p.batch == 0 || p.tokens == 0) return ROOST_STATUS_OK;
  const uint32_t act = p.input.dtype;
  const uint32_t st = p.conv_state.dtype == ROOST_DTYPE_UNDEFINED ? act : p.conv_state.dtype;
  gate.Expect(FloatType(act), ROOST_STATUS_UNSUPPORTED, "input is %s; built for bf16 and f32", roost::Describe(act).name)
      .Expect(FloatType(st), ROOST_STATUS_UNSUPPORTED, "conv_state is %s; built for bf16 and f32",
              roost::Describe(st).name);
  ROOST_GATE_RETURN(gate);
  const uint64_t sl = p.width - 1ull;
  const uint64_t n = uint64_t{p.tokens} * p.channels;
  const bool has_bias = p.bias.address != nullptr;
  const auto eb = static_cast<uint32_t>(ElemBytes(act));
  gate.Tensor("input", p.input, act, n)
      .Tensor("output", p.output, act, n)
      .Tensor("weight", p.weight, act, uint64_t{p.channels} * p.width)
      .OptionalTensor("bias", p.bias, act, p.channels)
      .Tensor("state_slots", p.state_slots, ROOST_DTYPE_I32, p.batch)
      .Tensor("cu_seqlens", p.cu_seqlens, ROOST_DTYPE_I32, p.batch + 1ull)
      .Expect(sl == 0 || (p.conv_state.reserved0 == 0 && p.conv_state.address != nullptr),
              ROOST_STATUS_INVALID_ARGUMENT, "a %u-tap filter keeps %llu tokens of state; conv_state is missing",
              p.width, static_cast<unsigned long long>(sl))
      .Expect(!Intersect(Bytes(p.input, n), Bytes(p.output, n)), ROOST_STATUS_INVALID_ARGUMENT,
              "input and output share memory; the convolution is never computed in place")
      .Aligned("input", p.input.address, eb)
      .Aligned("output", p.output.address, eb)
      .Aligned("weight", p.weight.address, eb)
      .Aligned("bias", has_bias ? p.bias.address : nullptr, eb)
      .Aligned("conv_state", sl > 0 ? p.conv_state.address : nullptr, static_cast<uint32_t>(ElemBytes(st)))
      .Aligned("state_slots", p.state_slots.address, 4)
      .Aligned("cu_seqlens", p.cu_seqlens.address, 4);
  return gate.status();
}

namespace {

// The kernels' view of an admitted CausalConv1d call.
ConvArgs MakeConvArgs(const RoostCausalConv1dParams& p) {
  const uint32_t act = p.input.dtype;
  const uint64_t sl = p.width - 1ull;
  ConvArgs a{};
  a.x = p.input.address;
  a.w = p.weight.address;
  a.bias = p.bias.address;
  a.y = p.output.address;
  a.state = p.conv_state.address;
  a.slots = static_cast<const int32_t*>(p.state_slots.address);
  a.cu = static_cast<const int32_t*>(p.cu_seqlens.address);
  a.act_t = act;
  a.state_t = p.conv_state.dtype == ROOST_DTYPE_UNDEFINED ? act : p.conv_state.dtype;
  a.batch = p.batch;
  a.tokens = p.tokens;
  a.channels = p.channels;
  a.width = p.width;
  a.silu = p.silu != 0;
  // Slots the pool holds; the state span's length is in its own elements (a zero length means no slot is valid).
  a.pool_slots = sl == 0 ? 0 : p.conv_state.length / (uint64_t{p.channels} * sl);
  return a;
}

// A layer call's last two steps in one launch: workgroups [0, norm_blocks) run GatedRmsNormRowKernel's rows (bf16,
// the input read as cached), the rest ConvStateVecKernel's (sequence, channel block) pairs, state_by blocks per
// sequence. The two touch disjoint memory, so their order within the launch does not matter.
template <int kW>
__global__ void __launch_bounds__(256) LayerTailKernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ gate,
                                                       const void* __restrict__ weight, uint32_t w_t,
                                                       uint16_t* __restrict__ out, uint64_t rows, uint32_t lanes,
                                                       float eps, uint32_t norm_blocks, ConvArgs a, uint32_t state_by) {
  const uint32_t bx = blockIdx.x;
  if (bx < norm_blocks) {
    GatedRmsNormRows<uint16_t, kRmsRows, false>(x, gate, weight, w_t, out, rows, 128, lanes, eps, bx);
  } else {
    ConvStateVecBlock<kW>(a, (bx - norm_blocks) / state_by, (bx - norm_blocks) % state_by);
  }
}

}  // namespace

RoostStatus roost_layer::ConvStateUpdate(const RoostCausalConv1dParams& p, hipStream_t s, const char* op) {
  if (p.batch == 0 || p.tokens == 0 || p.width == 1) return ROOST_STATUS_OK;
  const ConvArgs a = MakeConvArgs(p);
  const bool vec = p.input.dtype == ROOST_DTYPE_BF16 && p.width <= 4 && p.channels % 8 == 0 &&
                   roost::IsAligned(p.input.address, 16) && roost::IsAligned(p.conv_state.address, 16) &&
                   p.channels / 8 <= 65535u * 256u;
  if (vec) {
    const dim3 grid(p.batch, Blocks(p.channels / 8, 256));
    switch (p.width) {
      case 2: hipLaunchKernelGGL(ConvStateVecKernel<2>, grid, dim3(256), 0, s, a); break;
      case 3: hipLaunchKernelGGL(ConvStateVecKernel<3>, grid, dim3(256), 0, s, a); break;
      default: hipLaunchKernelGGL(ConvStateVecKernel<4>, grid, dim3(256), 0, s, a); break;
    }
  } else {
    hipLaunchKernelGGL(ConvStateKernel, dim3(Blocks(uint64_t{p.batch} * p.channels, 256)), dim3(256), 0, s, a);
  }
  return roost::HipStatus(hipGetLastError(), op, "state update launch");
}

RoostStatus roost_layer::RunNormAndConvState(const RoostGatedRmsNormParams& np, const RoostCausalConv1dParams& cp,
                                             hipStream_t s, const char* op) {
  const NormShape f = NormForm(np);
  const bool state_vec = cp.batch != 0 && cp.tokens != 0 && cp.width >= 2 && cp.width <= 4 &&
                         cp.input.dtype == ROOST_DTYPE_BF16 && cp.channels % 8 == 0 &&
                         roost::IsAligned(cp.input.address, 16) && roost::IsAligned(cp.conv_state.address, 16) &&
                         cp.channels / 8 <= 65535u * 256u;
  const bool norm_rows = np.rows != 0 && np.input.dtype == ROOST_DTYPE_BF16 && f.single && np.dim == 128;
  if (!state_vec || !norm_rows) {
    ROOST_RETURN_IF_FAILED(RunNorm(np, s, false, op));
    return ConvStateUpdate(cp, s, op);
  }
  const uint64_t rows_per_block = 4ull * (64 / f.lanes) * kRmsRows;
  const uint64_t norm_blocks = (uint64_t{np.rows} + rows_per_block - 1) / rows_per_block;
  const uint32_t state_by = Blocks(cp.channels / 8, 256);
  const uint64_t total = norm_blocks + uint64_t{cp.batch} * state_by;
  if (total > 0xFFFFFFFFull) {
    ROOST_RETURN_IF_FAILED(RunNorm(np, s, false, op));
    return ConvStateUpdate(cp, s, op);
  }
  const ConvArgs a = MakeConvArgs(cp);
  const auto* x = static_cast<const uint16_t*>(np.input.address);
  const auto* g = static_cast<const uint16_t*>(np.gate.address);
  auto* o = static_cast<uint16_t*>(np.output.address);
  const dim3 grid(static_cast<uint32_t>(total));
  const uint32_t nb = static_cast<uint32_t>(norm_blocks);
  switch (cp.width) {
    case 2: hipLaunchKernelGGL(LayerTailKernel<2>, grid, dim3(256), 0, s, x, g, np.weight.address, np.weight.dtype, o,
                               uint64_t{np.rows}, f.lanes, np.eps, nb, a, state_by); break;
    case 3: hipLaunchKernelGGL(LayerTailKernel<3>, grid, dim3(256), 0, s, x, g, np.weight.address, np.weight.dtype, o,
                               uint64_t{np.rows}, f.lanes, np.eps, nb, a, state_by); break;
    default: hipLaunchKernelGGL(LayerTailKernel<4>, grid, dim3(256), 0, s, x, g, np.weight.address, np.weight.dtype, o,
                                uint64_t{np.rows}, f.lanes, np.eps, nb, a, state_by); break;
  }
  return roost::HipStatus(hipGetLastError(), op, "norm and state launch");
}

extern "C" ROOST_API RoostStatus roost_causal_conv1d_run(RoostContext* ctx, const void* params, const RoostWorkspace*,
                                                          void* stream) {
  constexpr char kOp[] = "causal_conv1d";
  roost::Gate gate(kOp);
  const auto* pp = Preamble<RoostCausalConv1dParams>(gate, ctx, params);
  ROOST_GATE_RETURN(gate);
  const auto& p = *pp;
  return roost::CatchAll(kOp, [&]() -> RoostStatus {
    ROOST_RETURN_IF_FAILED(roost_layer::AdmitConv(p, kOp));
    if (p.batch == 0 || p.tokens == 0) return ROOST_STATUS_OK;
    const uint32_t act = p.input.dtype;
    const ConvArgs a = MakeConvArgs(p);
    const uint64_t v = 16 / ElemBytes(act);
    const bool vec = p.channels % v == 0 && roost::IsAligned(p.input.address, 16) && roost::IsAligned(p.output.address, 16);
    const uint32_t per_thread = vec ? static_cast<uint32_t>(v) : 1u;
    hipStream_t s = roost::Stream(stream);
    const bool bf = act == ROOST_DTYPE_BF16;
    // The tiled kernel takes 8-byte channel vectors (4 bf16 or 2 f32 channels) when the channel count and the
    // buffers allow them.
    const bool vec8 = p.channels % (8 / ElemBytes(act)) == 0 && roost::IsAligned(p.input.address, 8) &&
                      roost::IsAligned(p.output.address, 8) && roost::IsAligned(p.weight.address, 8) &&
                      roost::IsAligned(p.bias.address, 8);
    const uint32_t cblocks = Blocks(p.channels / (8 / ElemBytes(act)), 256);
    const uint64_t tiled_blocks = uint64_t{cblocks} * Blocks(p.tokens, kConvTile);
    // Tiles of kConvTile tokens pay off when sequences are long; a batch of short ones (a decode step: every tile
    // would cross sequences and take the per-token path) runs on the one-thread-per-token form.
    const bool long_seqs = uint64_t{p.tokens} >= uint64_t{p.batch} * kConvTile;
    const bool short_form = !long_seqs && bf && p.width >= 2 && p.width <= 4 && p.channels % 8 == 0 &&
                            roost::IsAligned(p.input.address, 16) && roost::IsAligned(p.output.address, 16) &&
                            roost::IsAligned(p.weight.address, 16) && roost::IsAligned(a.bias, 16) &&
                            roost::IsAligned(p.conv_state.address, 16) && p.channels / 8 <= 65535u * 256u;
    if (short_form) {
      const dim3 grid(p.tokens, Blocks(p.channels / 8, 256));
      switch (p.width) {
        case 2: hipLaunchKernelGGL(ConvShortKernel<2>, grid, dim3(256), 0, s, a); break;
        case 3: hipLaunchKernelGGL(ConvShortKernel<3>, grid, dim3(256), 0, s, a); break;
        default: hipLaunchKernelGGL(ConvShortKernel<4>, grid, dim3(256), 0, s, a); break;
      }
    } else if (vec8 && long_seqs && p.width >= 2 && p.width <= 4 && tiled_blocks <= 0xFFFFFFFFull) {
      const dim3 tiled(static_cast<uint32_t>(tiled_blocks));
      switch (p.width * 2 + (bf ? 1 : 0)) {
        case 5: hipLaunchKernelGGL((ConvTileKernel<uint16_t, 2, 8>), tiled, dim3(256), 0, s, a, cblocks); break;
        case 7: hipLaunchKernelGGL((ConvTileKernel<uint16_t, 3, 8>), tiled, dim3(256), 0, s, a, cblocks); break;
        case 9: hipLaunchKernelGGL((ConvTileKernel<uint16_t, 4, 8>), tiled, dim3(256), 0, s, a, cblocks); break;
        case 4: hipLaunchKernelGGL((ConvTileKernel<float, 2, 8>), tiled, dim3(256), 0, s, a, cblocks); break;
        case 6: hipLaunchKernelGGL((ConvTileKernel<float, 3, 8>), tiled, dim3(256), 0, s, a, cblocks); break;
        default: hipLaunchKernelGGL((ConvTileKernel<float, 4, 8>), tiled, dim3(256), 0, s, a, cblocks); break;
      }
    } else {
      const dim3 grid(p.tokens, Blocks(roost::CeilDiv(p.channels, per_thread), 256));
      if (bf) {
        if (vec) hipLaunchKernelGGL((ConvKernel<uint16_t, true>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((ConvKernel<uint16_t, false>), grid, dim3(256), 0, s, a);
      } else {
        if (vec) hipLaunchKernelGGL((ConvKernel<float, true>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((ConvKernel<float, false>), grid, dim3(256), 0, s, a);
      }
    }
    ROOST_RETURN_IF_FAILED(roost::HipStatus(hipGetLastError(), kOp, "convolution launch"));
    return roost_layer::ConvStateUpdate(p, s, kOp);
  });
}

namespace {

RoostStatus LaunchCopyPairs(const char* op, const void* src, uint64_t src_bytes, void* dst, uint64_t dst_bytes,
                            const RoostDeviceSpan& pairs, uint64_t slot_bytes, uint32_t count, uint32_t from_col,
                            hipStream_t stream) {
  // Pool sizes in slots; a pool of unknown size (length 0) leaves its slots unchecked, as the reference does.
  const uint64_t src_slots = src_bytes == 0 ? UINT64_MAX : src_bytes / slot_bytes;
  const uint64_t dst_slots = dst_bytes == 0 ? UINT64_MAX : dst_bytes / slot_bytes;
  const bool vec = slot_bytes % 16 == 0 && roost::IsAligned(src, 16) && roost::IsAligned(dst, 16);
  const uint64_t units = vec ? slot_bytes / 16 : slot_bytes;
  const uint64_t grid = roost::CeilDiv(units, uint64_t{256} * kUnitsPerThread);
  if (grid > 0x7fffffff) return roost::Report(ROOST_STATUS_INVALID_ARGUMENT, op, "slot_bytes %llu is too large", static_cast<unsigned long long>(slot_bytes));
  auto* kernel = vec ? SlotPairCopyKernel<true> : SlotPairCopyKernel<false>;
  hipLaunchKernelGGL(kernel, dim3(static_cast<uint32_t>(grid)), dim3(256), 0, stream,
                     static_cast<const unsigned char*>(src), static_cast<unsigned char*>(dst),
                     static_cast<const int32_t*>(pairs.address), count, slot_bytes, from_col, src_slots, dst_slots);
  return roost::HipStatus(hipGetLastError(), op, "slot copy launch");
}

// A pool is raw bytes: its span's length counts elements of its dtype, or bytes when the dtype is undefined.
uint64_t PoolBytes(const RoostDeviceSpan& s) {
  return s.length * (s.dtype == ROOST_DTYPE_UNDEFINED ? 1 : roost::ElementBytes(s.dtype));
}

// The slot-copy ops' shared rules: pools present, `count` (from, to) int32 pairs.
void AdmitPairs(roost::Gate& gate, const RoostDeviceSpan* const* pools, const char* const* names, int n_pools,
                const RoostDeviceSpan& pairs, uint32_t count) {
  for (int i = 0; i < n_pools; ++i) {
    gate.Expect(pools[i]->reserved0 == 0 && pools[i]->address != nullptr, ROOST_STATUS_INVALID_ARGUMENT,
                "%s: the pool span is missing or has a non-zero reserved word", names[i]);
  }
  gate.Tensor("pairs", pairs, ROOST_DTYPE_I32, uint64_t{count} * 2).Aligned("pairs", pairs.address, 4);
}

}  // namespace

extern "C" ROOST_API RoostStatus roost_recurrent_state_copy_run(RoostContext* ctx, const void* params,
                                                                 const RoostWorkspace*, void* stream) {
  constexpr char kOp[] = "recurrent_state_copy";
  roost::Gate gate(kOp);
  const auto* pp = Preamble<RoostRecurrentStateCopyParams>(gate, ctx, params);
  ROOST_GATE_RETURN(gate);
  const auto& p = *pp;
  return roost::CatchAll(kOp, [&]() -> RoostStatus {
    gate.Expect(p.reserved0 == 0, ROOST_STATUS_INVALID_ARGUMENT, "reserved0 = %u, must be 0", p.reserved0);
    ROOST_GATE_RETURN(gate);
    if (p.count == 0 || p.slot_bytes == 0) return ROOST_STATUS_OK;
    const RoostDeviceSpan* pools[] = {&p.pool};
    const char* names[] = {"pool"};
    AdmitPairs(gate, pools, names, 1, p.pairs, p.count);
    ROOST_GATE_RETURN(gate);
    const uint64_t bytes = PoolBytes(p.pool);
    return LaunchCopyPairs(kOp, p.pool.address, bytes, p.pool.address, bytes, p.pairs, p.slot_bytes, p.count, 0,
                           roost::Stream(stream));
  });
}

extern "C" ROOST_API RoostStatus roost_recurrent_state_snapshot_run(RoostContext* ctx, const void* params,
                                                                     const RoostWorkspace*, void* stream) {
  constexpr char kOp[] = "recurrent_state_snapshot";
  roost::Gate gate(kOp);
  const auto* pp = Preamble<RoostRecurrentStateSnapshotParams>(gate, ctx, params);
  ROOST_GATE_RETURN(gate);
  const auto& p = *pp;
  return roost::CatchAll(kOp, [&]() -> RoostStatus {
    if (p.count == 0 || p.slot_bytes == 0) return ROOST_STATUS_OK;
    const RoostDeviceSpan* pools[] = {&p.pool, &p.snapshots};
    const char* names[] = {"pool", "snapshots"};
    AdmitPairs(gate, pools, names, 2, p.pairs, p.count);
    ROOST_GATE_RETURN(gate);
    const bool restore = p.restore != 0;
    const RoostDeviceSpan& src = restore ? p.snapshots : p.pool;
    const RoostDeviceSpan& dst = restore ? p.pool : p.snapshots;
    return LaunchCopyPairs(kOp, src.address, PoolBytes(src), dst.address, PoolBytes(dst), p.pairs, p.slot_bytes,
                           p.count, restore ? 1u : 0u, roost::Stream(stream));
  });
}
