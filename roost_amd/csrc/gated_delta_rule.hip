// GatedDeltaRule (ROOST_OP_GATED_DELTA_RULE) for gfx950: the gated delta rule of Qwen3.5's linear-attention layers,
// read through row-strided q/k/v views, with the fp32 recurrent state read from and written back to its pool slot.
//
// Semantics are CpuOps.GatedDeltaRule (reference: src/Starlings.Roost.Ops/CpuOps.Hybrid.cs:30-157): per sequence b and
// value head h (key head h / (v_heads / k_heads)), state S [k_dim, v_dim] from slot state_slots[b] (zero when
// use_initial_state is 0), q and k l2-normalised with eps 1e-6, q scaled (scale 0 -> 1/sqrt(k_dim)), then per token
//   S = S * exp(g_t);  d = beta_t * (v_t - S^T k_t);  S = S + k_t d^T;  o_t = S^T q_t,
// and S is written back once as fp32. The library contract around it is the reference's
// (kernels/src/ops/gated_delta_rule.cu:231-278 validation; :400-576 chunk variant; :580-649 recurrent variant): an
// empty sequence leaves its slot untouched; a sequence whose slot is negative runs from a zero state and is not written
// back (slots are device data and are never range-checked on the host).
//
// Recurrent variant -- HBM bound (the state is read once and written once per call; the views are read in place, with
// no gather or state copy): one 128-thread workgroup per (sequence, value head). Thread t owns the 4 value columns
// 4*(t/4)..+3 over 32 key rows 32*(t%4)..+31 of S in registers (128 floats), so the column sums S^T k and S^T q need
// only a reduction over the 4 lanes of a quad, and consecutive lanes read consecutive 16-byte pieces of a state row.

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>

#include "common.h"

namespace {

using namespace roost_dev;

constexpr uint32_t kHeads = 16;
constexpr uint32_t kDim = 128;
constexpr uint32_t kRow = kHeads * kDim;
constexpr uint64_t kStateElems = uint64_t{kHeads} * kDim * kDim;
constexpr uint64_t kMaxTokens = uint64_t{1} << 24;
constexpr uint32_t kMaxBatch = 1u << 20;
constexpr uint32_t kChunk = 64;
// The recurrent variant hands a sequence of at least this many tokens to the chunk (WY) kernels: one token of the
// token-serial recurrence costs about as much latency as a chunk step covering 64 tokens.
constexpr uint32_t kRouteMinTokens = 16;
constexpr uint32_t kPlanMagic = 0x50444752;  // "RGDP"

uint32_t Stride(uint32_t s) { return s == 0 ? kRow : s; }

constexpr char kOp[] = "gated_delta_rule";

// The call's rules, shared by both variants. The statuses are the contract's (the reference refuses the same shapes:
// kernels/src/ops/gated_delta_rule.cu:231-278); `planning` adds plan()'s need for the host cu_seqlens copy.
RoostStatus Admit(const RoostGatedDeltaRuleParams& p, bool planning) {
  roost::Gate gate(kOp);
  gate.Header(&p, sizeof(RoostGatedDeltaRuleParams))
      .Expect(p.k_heads == kHeads && p.v_heads == kHeads && p.k_dim == kDim && p.v_dim == kDim,
              ROOST_STATUS_UNSUPPORTED, "heads %u/%u of dims %u/%u (key/value): the kernels are built for the "
              "Qwen3.5-0.8B shape, 16/16 heads of 128", p.k_heads, p.v_heads, p.k_dim, p.v_dim)
      .Expect(p.l2_norm_qk != 0, ROOST_STATUS_UNSUPPORTED, "l2_norm_qk = 0: the kernels always normalise q and k")
      .Expect(p.tokens <= kMaxTokens && p.batch <= kMaxBatch, ROOST_STATUS_INVALID_ARGUMENT,
              "%u tokens in %u sequences exceeds one call's limits (%llu tokens, %u sequences)", p.tokens, p.batch,
              static_cast<unsigned long long>(kMaxTokens), kMaxBatch);
  ROOST_GATE_RETURN(gate);
  const uint64_t qs = Stride(p.q_stride), ks = Stride(p.k_stride), vs = Stride(p.v_stride);
  gate.Expect(qs >= kRow && ks >= kRow && vs >= kRow, ROOST_STATUS_INVALID_ARGUMENT,
              "row strides q %llu, k %llu, v %llu: each view row holds %u elements", static_cast<unsigned long long>(qs),
              static_cast<unsigned long long>(ks), static_cast<unsigned long long>(vs), kRow);
  ROOST_GATE_RETURN(gate);
  // A strided view reaches (tokens - 1) * stride + one row.
  const uint64_t t = p.tokens;
  auto reach = [t](uint64_t stride) { return t == 0 ? 0 : (t - 1) * stride + kRow; };
  gate.Tensor("q", p.q, ROOST_DTYPE_BF16, reach(qs))
      .Tensor("k", p.k, ROOST_DTYPE_BF16, reach(ks))
      .Tensor("v", p.v, ROOST_DTYPE_BF16, reach(vs));
  ROOST_GATE_RETURN(gate);
  // g, beta and output of another type are shapes the kernels do not cover (UNSUPPORTED, as the contract has it).
  gate.Expect(p.g.dtype == ROOST_DTYPE_F32 && p.beta.dtype == ROOST_DTYPE_BF16 && p.output.dtype == ROOST_DTYPE_BF16,
              ROOST_STATUS_UNSUPPORTED, "g %s, beta %s, output %s: built for f32 g with bf16 beta and output",
              roost::Describe(p.g.dtype).name, roost::Describe(p.beta.dtype).name, roost::Describe(p.output.dtype).name);
  ROOST_GATE_RETURN(gate);
  gate.Tensor("g", p.g, ROOST_DTYPE_F32, t * kHeads)
      .Tensor("beta", p.beta, ROOST_DTYPE_BF16, t * kHeads)
      .Tensor("output", p.output, ROOST_DTYPE_BF16, t * kRow)
      .Tensor("state", p.state, ROOST_DTYPE_F32, kStateElems)
      .Expect(p.state.length % kStateElems == 0, ROOST_STATUS_INVALID_ARGUMENT,
              "state pool of %llu floats is not a whole number of [16, 128, 128] slots",
              static_cast<unsigned long long>(p.state.length))
      .Tensor("state_slots", p.state_slots, ROOST_DTYPE_I32, p.batch)
      .Tensor("cu_seqlens", p.cu_seqlens, ROOST_DTYPE_I32, uint64_t{p.batch} + 1)
      .Aligned("g", p.g.address, 16)
      .Aligned("beta", p.beta.address, 16)
      .Aligned("output", p.output.address, 16)
      .Aligned("state", p.state.address, 16)
      .Aligned("q", p.q.address, 2)
      .Aligned("k", p.k.address, 2)
      .Aligned("v", p.v.address, 2)
      .Expect(!planning || p.cu_seqlens_host != nullptr || p.batch == 0 || p.tokens == 0,
              ROOST_STATUS_INVALID_ARGUMENT, "plan() reads cu_seqlens_host, which is NULL");
  return gate.status();
}

// workspace() only sizes the call: the header and the token / sequence limits.
RoostStatus AdmitForSizing(const void* params, const RoostWorkspaceSizes* sizes) {
  roost::Gate gate(kOp);
  gate.Expect(sizes != nullptr, ROOST_STATUS_INVALID_ARGUMENT, "the sizes out-pointer is NULL")
      .Header(params, sizeof(RoostGatedDeltaRuleParams));
  ROOST_GATE_RETURN(gate);
  const auto& p = *static_cast<const RoostGatedDeltaRuleParams*>(params);
  gate.Expect(p.tokens <= kMaxTokens && p.batch <= kMaxBatch, ROOST_STATUS_INVALID_ARGUMENT,
              "%u tokens in %u sequences exceeds one call's limits", p.tokens, p.batch);
  return gate.status();
}

float Scale(const RoostGatedDeltaRuleParams& p) {
  return p.scale != 0.0f ? p.scale : 1.0f / std::sqrt(static_cast<float>(kDim));
}

struct GdnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const float* g;
  const uint16_t* beta;
  uint16_t* out;
  float* state;
  const int32_t* slots;
  const int32_t* cu;
  int32_t route_min;   // > 0: sequences of this many tokens or more belong to the chunk kernels
  uint64_t q_stride, k_stride, v_stride;
  uint64_t pool_slots;
  uint32_t use_initial_state;
  float scale;
};

// Loads 32 consecutive bf16 of a row as floats: 16-byte loads when the view is 16-byte aligned, else 2-byte loads.
template <bool kVec>
__device__ __forceinline__ void Load32(const uint16_t* src, float* dst) {
  if constexpr (kVec) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 w = reinterpret_cast<const uint4*>(src)[i];
      dst[8 * i + 0] = Bf16LoToF32(w.x); dst[8 * i + 1] = Bf16HiToF32(w.x);
      dst[8 * i + 2] = Bf16LoToF32(w.y); dst[8 * i + 3] = Bf16HiToF32(w.y);
      dst[8 * i + 4] = Bf16LoToF32(w.z); dst[8 * i + 5] = Bf16HiToF32(w.z);
      dst[8 * i + 6] = Bf16LoToF32(w.w); dst[8 * i + 7] = Bf16HiToF32(w.w);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 32; ++i) dst[i] = Bf16ToF32(src[i]);
  }
}

typedef float f32x4v_t __attribute__((ext_vector_type(4)));

// The recurrent step reads each state row once and writes it once, in whole 512-byte runs per wavefront: non-temporal
// accesses keep that stream out of the caches.
__device__ __forceinline__ float4 LoadStreamF4(const float* p) {
  const f32x4v_t v = __builtin_nontemporal_load(reinterpret_cast<const f32x4v_t*>(p));
  return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void StoreStreamF4(float* p, const float4& x) {
  __builtin_nontemporal_store(f32x4v_t{x.x, x.y, x.z, x.w}, reinterpret_cast<f32x4v_t*>(p));
}

__device__ __forceinline__ float QuadSum(float x) {
  x += __shfl_xor(x, 1, 64);
  x += __shfl_xor(x, 2, 64);
  return x;
}

// One workgroup per (sequence, value head): the token-serial recurrence with S held in registers.
template <bool kVec>
__global__ void __launch_bounds__(128) RecurrentKernel(GdnArgs a) {
  const uint32_t b = blockIdx.x;
  const uint32_t h = blockIdx.y;
  const int32_t t0 = a.cu[b];
  const int32_t t1 = a.cu[b + 1];
  if (t1 <= t0) return;  // an empty sequence leaves its slot untouched
  if (a.route_min > 0 && t1 - t0 >= a.route_min) return;  // run by the chunk kernels
  const int32_t slot = a.slots[b];
  const bool has_slot = slot >= 0 && static_cast<uint64_t>(slot) < a.pool_slots;
  const int t = threadIdx.x;
  const int rq = t & 3;   // key rows 32*rq .. +31
  const int cg = t >> 2;  // value columns 4*cg .. +3
  const uint32_t kh = h;  // one value head per key head
  float4 s[32];
  float* sp = has_slot ? a.state + (static_cast<uint64_t>(slot) * kHeads + h) * kDim * kDim : nullptr;
  if (has_slot && a.use_initial_state) {
#pragma unroll
    for (int i = 0; i < 32; ++i) s[i] = LoadStreamF4(sp + (rq * 32 + i) * kDim + cg * 4);
  } else {
#pragma unroll
    for (int i = 0; i < 32; ++i) s[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  for (int32_t tok = t0; tok < t1; ++tok) {
    float qv[32], kv[32];
    Load32<kVec>(a.q + static_cast<uint64_t>(tok) * a.q_stride + kh * kDim + rq * 32, qv);
    Load32<kVec>(a.k + static_cast<uint64_t>(tok) * a.k_stride + kh * kDim + rq * 32, kv);
    float qq = 0.f, kk = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      qq = fmaf(qv[i], qv[i], qq);
      kk = fmaf(kv[i], kv[i], kk);
    }
    qq = QuadSum(qq);
    kk = QuadSum(kk);
    const float qn = a.scale / sqrtf(qq + 1e-6f);
    const float kn = 1.0f / sqrtf(kk + 1e-6f);
    const uint64_t gi = static_cast<uint64_t>(tok) * kHeads + h;
    const float decay = expf(a.g[gi]);
    const float beta = Bf16ToF32(a.beta[gi]);
    const uint16_t* vrow = a.v + static_cast<uint64_t>(tok) * a.v_stride + h * kDim + cg * 4;
    float vv[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) vv[c] = Bf16ToF32(vrow[c]);
    // S^T k over this thread's rows, then across the quad.
    float sk[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const float ki = kv[i] * kn;
      kv[i] = ki;
      sk[0] = fmaf(s[i].x, ki, sk[0]);
      sk[1] = fmaf(s[i].y, ki, sk[1]);
      sk[2] = fmaf(s[i].z, ki, sk[2]);
      sk[3] = fmaf(s[i].w, ki, sk[3]);
    }
    float d[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) d[c] = beta * (vv[c] - decay * QuadSum(sk[c]));
    float o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const float ki = kv[i];
      const float qi = qv[i] * qn;
      s[i].x = fmaf(s[i].x, decay, ki * d[0]);
      s[i].y = fmaf(s[i].y, decay, ki * d[1]);
      s[i].z = fmaf(s[i].z, decay, ki * d[2]);
      s[i].w = fmaf(s[i].w, decay, ki * d[3]);
      o[0] = fmaf(s[i].x, qi, o[0]);
      o[1] = fmaf(s[i].y, qi, o[1]);
      o[2] = fmaf(s[i].z, qi, o[2]);
      o[3] = fmaf(s[i].w, qi, o[3]);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = QuadSum(o[c]);
    if (rq == 0) {
      uint2 w;
      w.x = PackBf16(o[0], o[1]);
      w.y = PackBf16(o[2], o[3]);
      *reinterpret_cast<uint2*>(a.out + (static_cast<uint64_t>(tok) * kHeads + h) * kDim + cg * 4) = w;
    }
  }
  if (has_slot) {
#pragma unroll
    for (int i = 0; i < 32; ++i) StoreStreamF4(sp + (rq * 32 + i) * kDim + cg * 4, s[i]);
  }
}

GdnArgs MakeArgs(const RoostGatedDeltaRuleParams& p) {
  GdnArgs a{};
  a.q = static_cast<const uint16_t*>(p.q.address);
  a.k = static_cast<const uint16_t*>(p.k.address);
  a.v = static_cast<const uint16_t*>(p.v.address);
  a.g = static_cast<const float*>(p.g.address);
  a.beta = static_cast<const uint16_t*>(p.beta.address);
  a.out = static_cast<uint16_t*>(p.output.address);
  a.state = static_cast<float*>(p.state.address);
  a.slots = static_cast<const int32_t*>(p.state_slots.address);
  a.cu = static_cast<const int32_t*>(p.cu_seqlens.address);
  a.q_stride = Stride(p.q_stride);
  a.k_stride = Stride(p.k_stride);
  a.v_stride = Stride(p.v_stride);
  a.pool_slots = p.state.length / kStateElems;
  a.use_initial_state = p.use_initial_state;
  a.scale = Scale(p);
  return a;
}

bool Vec16(const RoostGatedDeltaRuleParams& p) {
  auto Aligned = [](const void* a, uint64_t n) { return roost::IsAligned(a, n); };
  const uint64_t qs = Stride(p.q_stride), ks = Stride(p.k_stride), vs = Stride(p.v_stride);
  return Aligned(p.q.address, 16) && Aligned(p.k.address, 16) && Aligned(p.v.address, 8) && qs % 8 == 0 &&
         ks % 8 == 0 && vs % 4 == 0;
}

RoostStatus LaunchRecurrent(const RoostGatedDeltaRuleParams& p, hipStream_t stream, int32_t route_min = 0) {
  GdnArgs a = MakeArgs(p);
  a.route_min = route_min;
  const dim3 grid(p.batch, kHeads);
  if (Vec16(p)) {
    hipLaunchKernelGGL(RecurrentKernel<true>, grid, dim3(128), 0, stream, a);
  } else {
    hipLaunchKernelGGL(RecurrentKernel<false>, grid, dim3(128), 0, stream, a);
  }
  return roost::HipStatus(hipGetLastError(), kOp, "recurrent launch");
}

// ---- Chunk variant: WY form on MFMA ---------------------------------------------------------------------------------
//
// A sequence is cut into chunks of 64 tokens from its first token (the last one may be shorter). Within a chunk with
// start state S0, cumulative log-decay G_t = g_1 + .. + g_t, normalised k^_t = k_t * rk_t and q^_t = q_t * rq_t, the
// token recurrence above is exactly
//   A_tj = beta_t e^(G_t - G_j) k^_t . k^_j  (j < t),   T = (I + A)^-1,
//   Y_t  = beta_t (v_t - e^G_t S0^T k^_t),              V = T Y              (the delta of every token),
//   o_t  = e^G_t S0^T q^_t + sum_{j <= t} e^(G_t - G_j) (q^_t . k^_j) V_j,
//   S    = e^G_n S0 + sum_j e^(G_n - G_j) k^_j V_j^T.
// The prep kernel (one workgroup per chunk and head, all chunks in parallel) computes k.k and q.k on MFMA from the raw
// bf16 rows (exact products, fp32 sums; the norms are applied afterwards in fp32), T by blocked forward substitution in
// fp32, and stores T, P_tj = e^(G_t - G_j) q^_t . k^_j and the per-token factors in a per-(chunk, head) record. The scan
// kernel walks the chunks of one (sequence, head, 32-column value block) in order with S in registers. Every product that
// feeds the state runs with its fp32 operand split into bf16 hi + lo parts (raw k and q are exact in bf16 already):
// K.S0 as 2 MFMAs, T.Y as 3, k^T.V as 2, which keeps the state within about 1e-5 of the double-precision recurrence
// where single bf16 operands drift by a few 1e-3. The output terms, rounded to bf16 at the end, use single bf16 operands.

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kTilePitch = 136;  // bf16 per LDS row of a [64 tokens][128 dims] q/k tile (272 B: 16-byte aligned)
constexpr int kTokPitch = 72;    // bf16 per LDS row of a [dim or column][64 tokens] tile (144 B)
constexpr int kVBlock = 32;      // value columns per scan workgroup
constexpr uint32_t kVBlocks = kDim / kVBlock;

// Per-(chunk, head) record written by the prep kernel, row-major bf16 matrices: T (hi and lo parts) and P as
// [token t][token j], raw k transposed as [dim][token], then the per-token factors. The scan reads 16-byte pieces of
// their rows as MFMA operands. Entries above the diagonal of T and P are written as zero.
constexpr uint32_t kRecT = 0;          // T hi [64][64], then T lo [64][64]
constexpr uint32_t kRecP = 16384;      // P [64][64]
constexpr uint32_t kRecKT = 24576;     // k^T [128][64]
constexpr uint32_t kRecScal = 40960;   // float [5][64]: e^G rk, beta, rq e^G, e^(Gn - G) rk, e^Gn (at [4][0])
constexpr uint32_t kRecBytes = 42240;  // a multiple of 256

struct ChunkArgs {
  GdnArgs a;
  const int4* chunks;  // [chunks] (sequence, first token, tokens, 0)
  const int4* seqs;    // [batch] (first chunk, chunk count, first token, end token)
  uint8_t* recs;       // [chunks][heads] records
  const int32_t* seq_list;  // when set: chain c runs sequence seq_list[c / heads] (-1: none)
  uint32_t chains;     // batch * heads, or (length of seq_list) * heads
};

__device__ __forceinline__ f32x4_t Mfma(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                 0, 0, 0);
}

// Round-to-nearest-even pack of two floats (v_cvt_pk_bf16_f32); used for operands only, never for stored outputs.
__device__ __forceinline__ uint32_t PackRne(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// x = hi + lo + O(2^-16 |x|): hi is x truncated to bf16, lo the remainder rounded to bf16. Two floats per word.
__device__ __forceinline__ void Split2(float x0, float x1, uint32_t& hi, uint32_t& lo) {
  const uint32_t u0 = __float_as_uint(x0) & 0xFFFF0000u;
  const uint32_t u1 = __float_as_uint(x1) & 0xFFFF0000u;
  hi = (u0 >> 16) | u1;
  lo = PackRne(x0 - __uint_as_float(u0), x1 - __uint_as_float(u1));
}

template <bool kVec>
__device__ __forceinline__ uint4 Load8(const uint16_t* p) {
  if constexpr (kVec) {
    return *reinterpret_cast<const uint4*>(p);
  } else {
    uint4 r;
    r.x = p[0] | (static_cast<uint32_t>(p[1]) << 16);
    r.y = p[2] | (static_cast<uint32_t>(p[3]) << 16);
    r.z = p[4] | (static_cast<uint32_t>(p[5]) << 16);
    r.w = p[6] | (static_cast<uint32_t>(p[7]) << 16);
    return r;
  }
}

__device__ __forceinline__ float SumSq8(uint4 v) {
  float s = 0.0f;
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = Bf16LoToF32(w[i]), b = Bf16HiToF32(w[i]);
    s = fmaf(a, a, s);
    s = fmaf(b, b, s);
  }
  return s;
}

// fp32 16 x 16 x 4 MFMA: lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16]; the result layout is that of the
// bf16 16 x 16 products (lane l: rows 4 (l / 16) + i, column l % 16).
__device__ __forceinline__ f32x4_t MfmaF32(float a, float b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// One workgroup per (chunk, head); wave w owns row tile w (tokens 16w..16w+15) of the 64 x 64 products.
template <bool kVec>
__global__ void __launch_bounds__(256, 4) ChunkPrepKernel(ChunkArgs ca) {
  const GdnArgs& a = ca.a;
  const int4 ch = ca.chunks[blockIdx.x];
  const uint32_t h = blockIdx.y;
  const int t0 = ch.y, n = ch.z;
  if (n <= 0) return;  // an unused entry of a table sized for the worst case
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, kq = lane >> 4;
  uint8_t* rec = ca.recs + (static_cast<uint64_t>(blockIdx.x) * kHeads + h) * kRecBytes;

  // region0 holds the raw q (tile 0) and k (tile 1) rows; once the products are formed it holds A and T (fp32).
  __shared__ __align__(16) uint8_t region0[2 * 64 * kTilePitch * 2];
  __shared__ float g_lds[64], rk_lds[64], rq_lds[64], b_lds[64];
  auto qk = reinterpret_cast<uint16_t(*)[64][kTilePitch]>(region0);
  auto a_lds = reinterpret_cast<float(*)[65]>(region0);
  auto t_lds = reinterpret_cast<float(*)[65]>(region0 + 64 * 65 * 4);

  {  // Raw rows into LDS (zero past the chunk's end) and their sums of squares. Every load is issued unconditionally
     // from a clamped row and masked afterwards, so that all of them are in flight together.
    const int row = tid >> 2, part = tid & 3;
    const uint32_t keep = row < n ? ~0u : 0u;
    const uint64_t tok = static_cast<uint64_t>(t0 + min(row, n - 1));
    const uint16_t* kp = a.k + tok * a.k_stride + h * kDim + part * 32;
    const uint16_t* qp = a.q + tok * a.q_stride + h * kDim + part * 32;
    uint4 kv[4], qv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kv[i] = Load8<kVec>(kp + 8 * i);
      qv[i] = Load8<kVec>(qp + 8 * i);
    }
    const uint64_t gi = static_cast<uint64_t>(t0 + min(lane, n - 1)) * kHeads + h;
    const float graw = a.g[gi];
    const uint16_t braw = a.beta[gi];
    float kk = 0.0f, qq = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kv[i] = make_uint4(kv[i].x & keep, kv[i].y & keep, kv[i].z & keep, kv[i].w & keep);
      qv[i] = make_uint4(qv[i].x & keep, qv[i].y & keep, qv[i].z & keep, qv[i].w & keep);
      kk += SumSq8(kv[i]);
      qq += SumSq8(qv[i]);
      *reinterpret_cast<uint4*>(&qk[1][row][part * 32 + 8 * i]) = kv[i];
      *reinterpret_cast<uint4*>(&qk[0][row][part * 32 + 8 * i]) = qv[i];
    }
    kk = QuadSum(kk);
    qq = QuadSum(qq);
    if (part == 0) {
      rk_lds[row] = 1.0f / sqrtf(kk + 1e-6f);
      rq_lds[row] = a.scale / sqrtf(qq + 1e-6f);
    }
    if (w == 0) {  // cumulative log-decay (zero increments past the end) and beta
      float gv = lane < n ? graw : 0.0f;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const float y = __shfl_up(gv, d, 64);
        if (lane >= d) gv += y;
      }
      g_lds[lane] = gv;
      b_lds[lane] = lane < n ? Bf16ToF32(braw) : 0.0f;
    }
  }
  __syncthreads();

  // kk4[c] = k.k^T at rows 16w.., columns 16c..; pt4[c] = k.q^T at rows 16c.. (key tokens j), columns 16w.. (query
  // tokens t), i.e. P^T, whose result lanes hold four consecutive j of one t: one 8-byte piece of a row of P. A row-major
  // 16 x 32 tile supplies the A and the B operand in the same lane layout, so the k rows of tile c serve as both.
  f32x4_t kk4[4], pt4[4];
  {
    uint4 ak[4], bq[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      ak[s] = *reinterpret_cast<const uint4*>(&qk[1][16 * w + r16][32 * s + 8 * kq]);
      bq[s] = *reinterpret_cast<const uint4*>(&qk[0][16 * w + r16][32 * s + 8 * kq]);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      kk4[c] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      pt4[c] = kk4[c];
      if (c <= w) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const uint4 kc = *reinterpret_cast<const uint4*>(&qk[1][16 * c + r16][32 * s + 8 * kq]);
          kk4[c] = Mfma(ak[s], kc, kk4[c]);
          pt4[c] = Mfma(kc, bq[s], pt4[c]);
        }
      }
    }
  }
  // Raw k transposed: 16-byte pieces k^T[d][8g .. 8g + 7]; consecutive lanes read consecutive dims of a row.
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int piece = tid + 256 * m, d = piece & 127, g8 = piece >> 7;
    uint32_t wd[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      wd[e] = static_cast<uint32_t>(qk[1][8 * g8 + 2 * e][d]) | (static_cast<uint32_t>(qk[1][8 * g8 + 2 * e + 1][d]) << 16);
    }
    *reinterpret_cast<uint4*>(rec + kRecKT + (d * 64 + 8 * g8) * 2) = make_uint4(wd[0], wd[1], wd[2], wd[3]);
  }
  __syncthreads();  // the q/k tiles are dead: region0 becomes A and T

#pragma unroll
  for (int c = 0; c < 4; ++c) {
    uint2 pw = make_uint2(0, 0);
    float pv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      {  // A[r][j], r = 16w + 4kq + i, j = 16c + r16 (strictly lower); zero above the diagonal of A and T
        const int r = 16 * w + 4 * kq + i, j = 16 * c + r16;
        float av = 0.0f;
        if (j < r) av = b_lds[r] * expf(g_lds[r] - g_lds[j]) * kk4[c][i] * rk_lds[r] * rk_lds[j];
        a_lds[r][j] = av;
        if (c > w) t_lds[r][j] = 0.0f;
      }
      {  // P[t][j], t = 16w + r16, j = 16c + 4kq + i (on and below the diagonal)
        const int t = 16 * w + r16, j = 16 * c + 4 * kq + i;
        pv[i] = j <= t ? pt4[c][i] * rq_lds[t] * rk_lds[j] * expf(g_lds[t] - g_lds[j]) : 0.0f;
      }
    }
    if (c <= w) {
      pw.x = PackRne(pv[0], pv[1]);
      pw.y = PackRne(pv[2], pv[3]);
    }
    *reinterpret_cast<uint2*>(rec + kRecP + ((16 * w + r16) * 64 + 16 * c + 4 * kq) * 2) = pw;
  }
  __syncthreads();

  // T = (I + A)^-1. Diagonal 16 x 16 blocks by forward substitution (wave w, one column per lane) ...
  if (lane < 16) {
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float acc = i == lane ? 1.0f : 0.0f;
#pragma unroll
      for (int j = 0; j < i; ++j) acc = fmaf(-a_lds[16 * w + i][16 * w + j], x[j], acc);
      x[i] = acc;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) t_lds[16 * w + i][16 * w + lane] = x[i];
  }
  __syncthreads();
  // ... then the blocks below it, T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj, in order of distance d = i - j from the
  // diagonal, one block per wave, on fp32 MFMA. The partial sum goes through the (unused) mirror block A[j][i].
#pragma unroll
  for (int d = 1; d < 4; ++d) {
    if (w < 4 - d) {
      const int j = w, i = w + d;
      f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int k = j; k < i; ++k) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          acc = MfmaF32(a_lds[16 * i + r16][16 * k + 4 * kk + kq], t_lds[16 * k + 4 * kk + kq][16 * j + r16], acc);
        }
      }
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) a_lds[16 * j + 4 * kq + ii][16 * i + r16] = acc[ii];
      f32x4_t tij = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        tij = MfmaF32(t_lds[16 * i + r16][16 * i + 4 * kk + kq], a_lds[16 * j + 4 * kk + kq][16 * i + r16], tij);
      }
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) t_lds[16 * i + 4 * kq + ii][16 * j + r16] = -tij[ii];
    }
    __syncthreads();
  }
  // T rows as bf16 hi + lo, 8 columns per piece.
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const int piece = tid + 256 * m, row = piece >> 3, c8 = piece & 7;
    const float* src = &t_lds[row][8 * c8];
    uint4 hi, lo;
    Split2(src[0], src[1], hi.x, lo.x);
    Split2(src[2], src[3], hi.y, lo.y);
    Split2(src[4], src[5], hi.z, lo.z);
    Split2(src[6], src[7], hi.w, lo.w);
    *reinterpret_cast<uint4*>(rec + kRecT + (row * 64 + 8 * c8) * 2) = hi;
    *reinterpret_cast<uint4*>(rec + kRecT + 8192 + (row * 64 + 8 * c8) * 2) = lo;
  }
  if (tid < 64) {
    float* sc = reinterpret_cast<float*>(rec + kRecScal);
    const float gt = g_lds[tid], gn = g_lds[63];
    const float e = expf(gt);
    sc[tid] = e * rk_lds[tid];
    sc[64 + tid] = b_lds[tid];
    sc[128 + tid] = rq_lds[tid] * e;
    sc[192 + tid] = expf(gn - gt) * rk_lds[tid];
    if (tid == 0) sc[256] = expf(gn);
  }
}

// Per wave and chunk, the record's rows that wave uses are copied into LDS by global_load_lds (no registers on the
// way), double-buffered across chunks. 16-byte pieces are stored at swizzled positions so that the MFMA operand reads
// (16 lanes reading the same piece index of 16 different rows) hit distinct banks.
constexpr int kStageT = 0;         // T hi rows 16w..16w+15: [16][8 pieces of 16 B]
constexpr int kStageTLo = 2048;    // T lo rows
constexpr int kStageP = 4096;      // P rows
constexpr int kStageKT = 6144;     // k^T rows 32w..32w+31: [32][8 pieces]
constexpr int kStageScal = 10240;  // float [4][16]: e^G rk, beta, rq e^G, e^(Gn - G) rk of tokens 16w..16w+15
constexpr int kStageBytes = 10496;

// Position of 16-byte piece c8 of row r in a [rows][8 pieces] staging block.
__device__ __forceinline__ int Swz(int r, int c8) { return r * 128 + 16 * (c8 ^ ((r >> 1) & 7)); }

__device__ __forceinline__ uint32_t LdsAddr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p));
}

// global -> LDS copies (global_load_lds): lane l's bytes land at lds + size * l; lds must be wave-uniform. Issued from
// inline assembly so that the compiler does not treat every later LDS access as waiting on them (it cannot tell which
// LDS bytes they write); the scan waits for them itself, one chunk later. M0 carries the LDS address and is restored.
__device__ __forceinline__ void Dma16(const void* g, uint32_t lds) {
  uint32_t save;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
               : "=&s"(save) : "v"(g), "s"(lds));
}
__device__ __forceinline__ void Dma4(const void* g, uint32_t lds) {
  uint32_t save;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
               : "=&s"(save) : "v"(g), "s"(lds));
}

// s_waitcnt vmcnt(0) alone (expcnt and lgkmcnt fields at their maxima).
__device__ __forceinline__ void WaitVmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// The registers one wave needs for one chunk: its 16 raw k and q rows (MFMA A operands), its v values in the MFMA
// result layout and the chunk's total decay.
struct ChunkRegs {
  uint4 kr[4], qr[4];
  float vv[2][4];
  float decay;
  int t0, n;
};

// Chunk c of a sequence starts at token sq.z + 64c; its record is number sq.x + c. Loads the wave's registers and
// starts the copy of its record rows into `stage` (this wave's block of one buffer).
template <bool kVec>
__device__ __forceinline__ void LoadChunk(const ChunkArgs& ca, const int4& sq, int c, uint32_t h, uint32_t vb, int w,
                                          int lane, ChunkRegs& r, uint8_t* stage) {
  const GdnArgs& a = ca.a;
  const uint32_t chunk = static_cast<uint32_t>(sq.x + c);
  r.t0 = sq.z + static_cast<int>(kChunk) * c;
  r.n = min(static_cast<int>(kChunk), sq.w - r.t0);
  const int r16 = lane & 15, kq = lane >> 4;
  const int row = 16 * w + r16;
  const bool ok = row < r.n;
  const uint64_t tok = static_cast<uint64_t>(r.t0 + (ok ? row : r.n - 1));
  const uint16_t* kp = a.k + tok * a.k_stride + h * kDim + 8 * kq;
  const uint16_t* qp = a.q + tok * a.q_stride + h * kDim + 8 * kq;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const uint4 kv = Load8<kVec>(kp + 32 * s), qv = Load8<kVec>(qp + 32 * s);
    r.kr[s] = ok ? kv : make_uint4(0, 0, 0, 0);
    r.qr[s] = ok ? qv : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int rv = 16 * w + 4 * kq + i;
    const bool okv = rv < r.n;
    const uint16_t* vp = a.v + static_cast<uint64_t>(r.t0 + (okv ? rv : r.n - 1)) * a.v_stride + h * kDim +
                         vb * kVBlock + r16;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const float x = Bf16ToF32(vp[16 * nt]);
      r.vv[nt][i] = okv ? x : 0.0f;
    }
  }
  const uint8_t* rec = ca.recs + (static_cast<uint64_t>(chunk) * kHeads + h) * kRecBytes;
  r.decay = reinterpret_cast<const float*>(rec + kRecScal)[256];
  // Record rows into LDS: lane l fills byte 16 l of each 1 KB instruction block.
  const uint32_t base = LdsAddr(stage);
  const int rr = lane >> 3, pos = lane & 7;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int rw = 8 * i + rr, c8 = pos ^ ((rw >> 1) & 7);
    const uint8_t* src = rec + ((16 * w + rw) * 64 + 8 * c8) * 2;
    Dma16(src + kRecT, base + kStageT + 1024 * i);
    Dma16(src + kRecT + 8192, base + kStageTLo + 1024 * i);
    Dma16(src + kRecP, base + kStageP + 1024 * i);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int rw = 8 * i + rr, c8 = pos ^ ((rw >> 1) & 7);
    Dma16(rec + kRecKT + ((32 * w + rw) * 64 + 8 * c8) * 2, base + kStageKT + 1024 * i);
  }
  Dma4(rec + kRecScal + ((lane >> 4) * 64 + 16 * w + r16) * 4, base + kStageScal);
}

// A chunk's output values of one lane, stored one chunk later (so that the wait at the top of a chunk never waits on
// stores issued just before it).
struct ChunkOut {
  uint16_t o[2][4];
  int t0, n;
};

__device__ __forceinline__ void StoreOut(const GdnArgs& a, const ChunkOut& r, uint32_t h, uint32_t vb, int w, int r16,
                                         int kq) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = 16 * w + 4 * kq + i;
    if (t < r.n) {
      uint16_t* op = a.out + (static_cast<uint64_t>(r.t0 + t) * kHeads + h) * kDim + vb * kVBlock + r16;
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) op[16 * nt] = r.o[nt][i];
    }
  }
}

__device__ __forceinline__ float F4(const float4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

template <typename T>
__device__ __forceinline__ T LdsRead(const uint8_t* p) {
  return *reinterpret_cast<const T*>(p);
}

// One chunk of the scan (see ChunkScanKernel); `stage` is this wave's staged record block for the chunk.
__device__ __forceinline__ void ScanStep(const GdnArgs& a, const ChunkRegs& cur, const uint8_t* stage,
                                         f32x4_t (&st)[2][2], uint32_t h, uint32_t vb, int w, int r16, int kq,
                                         uint16_t (&s_lds)[2][kVBlock][kTilePitch],
                                         uint16_t (&y_lds)[2][kVBlock][kTokPitch],
                                         uint16_t (&vn_lds)[3][kVBlock][kTokPitch], ChunkOut& out) {
  // (1) S as bf16 hi/lo B operands.
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      uint2 hi, lo;
      Split2(st[mt][nt][0], st[mt][nt][1], hi.x, lo.x);
      Split2(st[mt][nt][2], st[mt][nt][3], hi.y, lo.y);
      const int d0 = 32 * w + 16 * mt + 4 * kq, col = 16 * nt + r16;
      *reinterpret_cast<uint2*>(&s_lds[0][col][d0]) = hi;
      *reinterpret_cast<uint2*>(&s_lds[1][col][d0]) = lo;
    }
  }
  __syncthreads();
  // (2) X = k S0 (hi + lo) and q S0 (hi) for tokens 16w..16w+15; Y = beta (v - e^G rk X).
  uint4 bh[4][2], bl[4][2];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      bh[s][nt] = *reinterpret_cast<const uint4*>(&s_lds[0][16 * nt + r16][32 * s + 8 * kq]);
      bl[s][nt] = *reinterpret_cast<const uint4*>(&s_lds[1][16 * nt + r16][32 * s + 8 * kq]);
    }
  }
  f32x4_t xs4[2], oq4[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) xs4[nt] = oq4[nt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      xs4[nt] = Mfma(cur.kr[s], bh[s][nt], xs4[nt]);
      oq4[nt] = Mfma(cur.qr[s], bh[s][nt], oq4[nt]);
    }
  }
#pragma unroll
  for (int s = 0; s < 4; ++s) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) xs4[nt] = Mfma(cur.kr[s], bl[s][nt], xs4[nt]);
  }
  const float4 xs = LdsRead<float4>(stage + kStageScal + 16 * kq);
  const float4 beta = LdsRead<float4>(stage + kStageScal + 64 + 16 * kq);
  const float4 os = LdsRead<float4>(stage + kStageScal + 128 + 16 * kq);
  const float4 ws = LdsRead<float4>(stage + kStageScal + 192 + 16 * kq);
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    float y[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) y[i] = F4(beta, i) * (cur.vv[nt][i] - F4(xs, i) * xs4[nt][i]);
    uint2 hi, lo;
    Split2(y[0], y[1], hi.x, lo.x);
    Split2(y[2], y[3], hi.y, lo.y);
    const int col = 16 * nt + r16, t = 16 * w + 4 * kq;
    *reinterpret_cast<uint2*>(&y_lds[0][col][t]) = hi;
    *reinterpret_cast<uint2*>(&y_lds[1][col][t]) = lo;
  }
  __syncthreads();
  // (3) V = T Y over the pieces on or below the diagonal (hi.hi + hi.lo + lo.hi).
  f32x4_t vn4[2] = {f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    if (s <= (w >> 1)) {
      const uint4 th = LdsRead<uint4>(stage + kStageT + Swz(r16, 4 * s + kq));
      const uint4 tl = LdsRead<uint4>(stage + kStageTLo + Swz(r16, 4 * s + kq));
      uint4 yh[2], yl[2];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        yh[nt] = *reinterpret_cast<const uint4*>(&y_lds[0][16 * nt + r16][32 * s + 8 * kq]);
        yl[nt] = *reinterpret_cast<const uint4*>(&y_lds[1][16 * nt + r16][32 * s + 8 * kq]);
      }
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        vn4[nt] = Mfma(th, yh[nt], vn4[nt]);
        vn4[nt] = Mfma(th, yl[nt], vn4[nt]);
        vn4[nt] = Mfma(tl, yh[nt], vn4[nt]);
      }
    }
  }
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int col = 16 * nt + r16, t = 16 * w + 4 * kq;
    uint2 v, hi, lo;
    v.x = PackRne(vn4[nt][0], vn4[nt][1]);
    v.y = PackRne(vn4[nt][2], vn4[nt][3]);
    Split2(vn4[nt][0] * ws.x, vn4[nt][1] * ws.y, hi.x, lo.x);
    Split2(vn4[nt][2] * ws.z, vn4[nt][3] * ws.w, hi.y, lo.y);
    *reinterpret_cast<uint2*>(&vn_lds[0][col][t]) = v;
    *reinterpret_cast<uint2*>(&vn_lds[1][col][t]) = hi;
    *reinterpret_cast<uint2*>(&vn_lds[2][col][t]) = lo;
  }
  __syncthreads();
  // (4) o = rq e^G q S0 + P V for tokens 16w..16w+15.
  f32x4_t pv4[2] = {f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    if (s <= (w >> 1)) {
      const uint4 pr = LdsRead<uint4>(stage + kStageP + Swz(r16, 4 * s + kq));
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const uint4 b = *reinterpret_cast<const uint4*>(&vn_lds[0][16 * nt + r16][32 * s + 8 * kq]);
        pv4[nt] = Mfma(pr, b, pv4[nt]);
      }
    }
  }
  out.t0 = cur.t0;
  out.n = cur.n;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) out.o[nt][i] = F32ToBf16(fmaf(F4(os, i), oq4[nt][i], pv4[nt][i]));
  }
  // (5) S = e^Gn S0 + k^T (ws V) (hi + lo) for state rows 32w..32w+31.
  uint4 vh[2][2], vl[2][2], ak[2][2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      vh[s][nt] = *reinterpret_cast<const uint4*>(&vn_lds[1][16 * nt + r16][32 * s + 8 * kq]);
      vl[s][nt] = *reinterpret_cast<const uint4*>(&vn_lds[2][16 * nt + r16][32 * s + 8 * kq]);
    }
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) ak[mt][s] = LdsRead<uint4>(stage + kStageKT + Swz(16 * mt + r16, 4 * s + kq));
  }
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      f32x4_t acc = st[mt][nt] * cur.decay;
#pragma unroll
      for (int s = 0; s < 2; ++s) acc = Mfma(ak[mt][s], vh[s][nt], acc);
#pragma unroll
      for (int s = 0; s < 2; ++s) acc = Mfma(ak[mt][s], vl[s][nt], acc);
      st[mt][nt] = acc;
    }
  }
}

// One workgroup per (sequence, head, value block of 32 columns); wave w owns state rows 32w..32w+31 and, for the
// token-side products, tokens 16w..16w+15 of each chunk. blockIdx -> (chain, block) keeps the four value blocks of a
// chain on one XCD (workgroups are dealt to the 8 XCDs round-robin), so they share the chain's k, q and records in L2.
template <bool kVec>
__global__ void __launch_bounds__(256, 1) ChunkScanKernel(ChunkArgs ca) {
  const GdnArgs& a = ca.a;
  const uint32_t x = blockIdx.x;
  const uint32_t chain = (x & 7) + 8 * (x >> 5);
  const uint32_t vb = (x >> 3) & 3;
  if (chain >= ca.chains) return;
  const int32_t listed = ca.seq_list != nullptr ? ca.seq_list[chain / kHeads] : static_cast<int32_t>(chain / kHeads);
  if (listed < 0) return;
  const uint32_t seq = static_cast<uint32_t>(listed), h = chain % kHeads;
  const int4 sq = ca.seqs[seq];
  if (sq.y == 0) return;  // an empty sequence leaves its slot untouched
  const int32_t slot = a.slots[seq];
  const bool has_slot = slot >= 0 && static_cast<uint64_t>(slot) < a.pool_slots;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, kq = lane >> 4;

  __shared__ __align__(16) uint16_t s_lds[2][kVBlock][kTilePitch];  // S hi, lo as [column][dim]
  __shared__ __align__(16) uint16_t y_lds[2][kVBlock][kTokPitch];   // Y hi, lo as [column][token]
  __shared__ __align__(16) uint16_t vn_lds[3][kVBlock][kTokPitch];  // V (bf16), V * ws hi, lo as [column][token]
  __shared__ __align__(16) uint8_t stage_lds[2][4][kStageBytes];    // [buffer][wave] staged record rows
  uint8_t* stage0 = stage_lds[0][w];
  uint8_t* stage1 = stage_lds[1][w];

  // st[mt][nt][i] = S[32w + 16mt + 4kq + i][32vb + 16nt + r16]
  f32x4_t st[2][2];
  float* sp = has_slot ? a.state + (static_cast<uint64_t>(slot) * kHeads + h) * kDim * kDim : nullptr;
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 32 * w + 16 * mt + 4 * kq + i, c = vb * kVBlock + 16 * nt + r16;
        st[mt][nt][i] = (has_slot && a.use_initial_state) ? sp[d * kDim + c] : 0.0f;
      }
    }
  }

  // Two register sets and two staging buffers in turn: the loads of chunk c + 1 are in flight while chunk c is
  // computed (the last chunk is loaded again past the end rather than branching around the load).
  // Each step first waits for every vector memory operation issued one step earlier (the chunk's registers, its
  // staged record rows, the previous chunk's outputs), then starts the loads of the next chunk.
  ChunkRegs ra, rb;
  ChunkOut out;
  out.n = 0;
  const int last = sq.y - 1;
  LoadChunk<kVec>(ca, sq, 0, h, vb, w, lane, ra, stage0);
  for (int c = 0;;) {
    WaitVmem();
    LoadChunk<kVec>(ca, sq, min(c + 1, last), h, vb, w, lane, rb, stage1);
    StoreOut(a, out, h, vb, w, r16, kq);
    ScanStep(a, ra, stage0, st, h, vb, w, r16, kq, s_lds, y_lds, vn_lds, out);
    if (++c > last) break;
    WaitVmem();
    LoadChunk<kVec>(ca, sq, min(c + 1, last), h, vb, w, lane, ra, stage0);
    StoreOut(a, out, h, vb, w, r16, kq);
    ScanStep(a, rb, stage1, st, h, vb, w, r16, kq, s_lds, y_lds, vn_lds, out);
    if (++c > last) break;
  }
  StoreOut(a, out, h, vb, w, r16, kq);
  WaitVmem();  // the copies of the re-loaded last chunk land before the workgroup's LDS is released
  if (has_slot) {
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = 32 * w + 16 * mt + 4 * kq + i, c = vb * kVBlock + 16 * nt + r16;
          sp[d * kDim + c] = st[mt][nt][i];
        }
      }
    }
  }
}

// ---- Chunk variant: plan tables ---------------------------------------------------------------------------------------

struct ChunkStamp {  // what plan() leaves in ws->plan for run()
  uint32_t magic;
  uint32_t batch;
  uint32_t tokens;
  uint32_t chunks;
};

struct ChunkArena {
  uint64_t chunk_table;  // [max_chunks] int4 (sequence, first token, tokens, 0)
  uint64_t seq_table;    // [batch] int4 (first chunk, chunk count, first token, end token)
  uint64_t seq_list;     // [max_long] int32: the chunked sequences in order (recurrent variant only)
  uint32_t max_long;
  uint64_t tables_bytes;
  uint64_t records;      // [max_chunks][heads] records of kRecBytes
  uint64_t total;
  uint32_t max_chunks;
};

ChunkArena MakeArena(uint64_t max_chunks, uint64_t batch, uint64_t max_long = 0) {
  ChunkArena l{};
  l.max_chunks = static_cast<uint32_t>(max_chunks);
  l.max_long = static_cast<uint32_t>(max_long);
  l.chunk_table = 0;
  l.seq_table = roost::RoundUp(16ull * l.max_chunks, 256);
  l.seq_list = l.seq_table + 16ull * batch;
  l.tables_bytes = roost::RoundUp(l.seq_list + 4ull * max_long, 256);
  l.records = l.tables_bytes;
  l.total = l.records + uint64_t{l.max_chunks} * kHeads * kRecBytes;
  return l;
}

// Every sequence may be chunked (chunk variant): at most tokens / 64 + batch chunks.
ChunkArena MakeChunkArena(uint64_t tokens, uint64_t batch) { return MakeArena(tokens / kChunk + batch, batch); }

// Only sequences of kRouteMinTokens or more are chunked (recurrent variant): sum ceil(len / 64) over them is at most
// tokens / 64 plus their number, which is at most min(batch, tokens / kRouteMinTokens).
ChunkArena MakeRouteArena(uint64_t tokens, uint64_t batch) {
  const uint64_t max_long = std::min<uint64_t>(batch, tokens / kRouteMinTokens);
  return MakeArena(tokens / kChunk + max_long, batch, max_long);
}


// Builds the chunk and sequence tables of the recurrent variant on the device from cu_seqlens, so that run() needs no
// plan and no host copy: a sequence of kRouteMinTokens or more tokens gets ceil(len / 64) chunk entries and a non-zero
// count in its sequence entry; every other sequence gets count 0 (the recurrent kernel runs it). Entries of the chunk
// table past the last one written have 0 tokens, which the prep kernel skips. The table holds every chunk whenever
// cu_seqlens ends at the call's token count; otherwise the sequences whose chunks do not fit get count 0 and no
// output (device tables are not range-checked, as everywhere in this ABI), and nothing is written out of bounds. One
// workgroup walks the batch 1024 sequences at a time with a workgroup-wide prefix sum of the chunk counts.
__global__ void __launch_bounds__(1024) RouteKernel(const int32_t* cu, uint32_t batch, uint32_t max_chunks,
                                                    int4* chunks, int4* seqs, int32_t* seq_list, uint32_t max_long) {
  __shared__ uint32_t wave_sum[16], wave_long[16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (uint32_t i = tid; i < max_chunks; i += 1024) chunks[i] = make_int4(0, 0, 0, 0);
  for (uint32_t i = tid; i < max_long; i += 1024) seq_list[i] = -1;
  __syncthreads();  // the fills land before any entry below is written over them
  uint32_t base = 0, long_base = 0;
  for (uint32_t start = 0; start < batch; start += 1024) {
    const uint32_t b = start + tid;
    int32_t t0 = 0, t1 = 0;
    uint32_t cnt = 0;
    if (b < batch) {
      t0 = cu[b];
      t1 = cu[b + 1];
      const int32_t len = t1 - t0;
      cnt = len >= static_cast<int32_t>(kRouteMinTokens) ? (static_cast<uint32_t>(len) + kChunk - 1) / kChunk : 0;
    }
    uint32_t incl = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t y = __shfl_up(incl, o);
      if (lane >= o) incl += y;
    }
    if (lane == 63) wave_sum[w] = incl;
    __syncthreads();
    uint32_t before = 0, total = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t x = wave_sum[i];
      before += i < w ? x : 0;
      total += x;
    }
    const uint64_t first = uint64_t{base} + before + incl - cnt;
    const bool routed = b < batch && cnt != 0 && first + cnt <= max_chunks;
    // Second prefix sum: the position of each routed sequence in seq_list.
    const uint32_t is_long = routed ? 1u : 0u;
    uint32_t lincl = is_long;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t y = __shfl_up(lincl, o);
      if (lane >= o) lincl += y;
    }
    if (lane == 63) wave_long[w] = lincl;
    __syncthreads();
    uint32_t lbefore = 0, ltotal = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t x = wave_long[i];
      lbefore += i < w ? x : 0;
      ltotal += x;
    }
    if (b < batch) {
      if (routed) {
        seqs[b] = make_int4(static_cast<int32_t>(first), static_cast<int32_t>(cnt), t0, t1);
        for (uint32_t c = 0; c < cnt; ++c) {
          const int32_t tc = t0 + static_cast<int32_t>(c * kChunk);
          chunks[first + c] = make_int4(static_cast<int32_t>(b), tc, min(static_cast<int32_t>(kChunk), t1 - tc), 0);
        }
        const uint32_t li = long_base + lbefore + lincl - 1;
        if (li < max_long) seq_list[li] = static_cast<int32_t>(b);
      } else {
        seqs[b] = make_int4(0, 0, t0, t1);
      }
    }
    base = static_cast<uint32_t>(min<uint64_t>(uint64_t{base} + total, 0xFFFFFFFFull));
    long_base += ltotal;
    __syncthreads();  // wave_sum and wave_long are rewritten by the next pass
  }
}

RoostStatus LaunchChunk(const RoostGatedDeltaRuleParams& p, const RoostWorkspace* ws, const ChunkArena& l,
                        uint32_t chunks, hipStream_t stream) {
  ChunkArgs ca{};
  ca.a = MakeArgs(p);
  auto* base = static_cast<uint8_t*>(ws->device);
  ca.chunks = reinterpret_cast<const int4*>(base + l.chunk_table);
  ca.seqs = reinterpret_cast<const int4*>(base + l.seq_table);
  ca.recs = base + l.records;
  // The recurrent variant's calls list their chunked sequences; the chunk variant's chains are every sequence.
  ca.seq_list = l.max_long > 0 ? reinterpret_cast<const int32_t*>(base + l.seq_list) : nullptr;
  ca.chains = (l.max_long > 0 ? l.max_long : p.batch) * kHeads;
  const dim3 prep(chunks, kHeads);
  const dim3 scan((ca.chains + 7) / 8 * 8 * kVBlocks);
  if (Vec16(p)) {
    hipLaunchKernelGGL(ChunkPrepKernel<true>, prep, dim3(256), 0, stream, ca);
    hipLaunchKernelGGL(ChunkScanKernel<true>, scan, dim3(256), 0, stream, ca);
  } else {
    hipLaunchKernelGGL(ChunkPrepKernel<false>, prep, dim3(256), 0, stream, ca);
    hipLaunchKernelGGL(ChunkScanKernel<false>, scan, dim3(256), 0, stream, ca);
  }
  return roost::HipStatus(hipGetLastError(), kOp, "chunk launch");
}

// The recurrent variant's routed path over a device region laid out as `l`: RouteKernel writes the chunk tables of the
// sequences of kRouteMinTokens or more tokens from the device cu_seqlens, the chunk kernels run those sequences and the
// recurrent kernel the rest, in that order on one stream. (Two streams were slower: the short kernels lose more to
// sharing the chip than the overlap saves.) Two sequences of one call sharing a state slot leave the recurrent one's
// state.
RoostStatus LaunchRouted(const RoostGatedDeltaRuleParams& p, uint8_t* base, const ChunkArena& l, hipStream_t s) {
  hipLaunchKernelGGL(RouteKernel, dim3(1), dim3(1024), 0, s, static_cast<const int32_t*>(p.cu_seqlens.address),
                     p.batch, l.max_chunks, reinterpret_cast<int4*>(base + l.chunk_table),
                     reinterpret_cast<int4*>(base + l.seq_table), reinterpret_cast<int32_t*>(base + l.seq_list),
                     l.max_long);
  ROOST_RETURN_IF_FAILED(roost::HipStatus(hipGetLastError(), kOp, "route launch"));
  RoostWorkspace ws{};
  ws.device = base;
  ws.device_bytes = l.total;
  ROOST_RETURN_IF_FAILED(LaunchChunk(p, &ws, l, l.max_chunks, s));
  return LaunchRecurrent(p, s, static_cast<int32_t>(kRouteMinTokens));
}

}  // namespace

// ---- Recurrent entry points ---------------------------------------------------------------------------------------

extern "C" ROOST_API RoostStatus roost_gdn_recurrent_workspace(RoostContext*, const void* params,
                                                               RoostWorkspaceSizes* sizes) {
  ROOST_RETURN_IF_FAILED(AdmitForSizing(params, sizes));
  const auto& p = *static_cast<const RoostGatedDeltaRuleParams*>(params);
  // The views and the pool slots are read in place; a call that may hold a sequence of kRouteMinTokens or more
  // tokens also gets the chunk tables and records for the sequences it hands to the chunk kernels.
  *sizes = RoostWorkspaceSizes{};
  sizes->device_bytes = p.tokens >= kRouteMinTokens ? MakeRouteArena(p.tokens, p.batch).total : 0;
  sizes->device_alignment = 256;
  return ROOST_STATUS_OK;
}

extern "C" ROOST_API RoostStatus roost_gdn_recurrent_run(RoostContext* ctx, const void* params, const RoostWorkspace* ws,
                                                         void* stream) {
  roost::Gate gate(kOp);
  gate.Expect(ctx != nullptr && params != nullptr, ROOST_STATUS_INVALID_ARGUMENT, "a context and params are required");
  ROOST_GATE_RETURN(gate);
  const auto& p = *static_cast<const RoostGatedDeltaRuleParams*>(params);
  return roost::CatchAll(kOp, [&]() -> RoostStatus {
    ROOST_RETURN_IF_FAILED(Admit(p, false));
    if (p.batch == 0 || p.tokens == 0) return ROOST_STATUS_OK;
    hipStream_t s = roost::Stream(stream);
    if (p.tokens < kRouteMinTokens) return LaunchRecurrent(p, s);
    if (p.cu_seqlens_host != nullptr) {
      // The host copy says whether any sequence reaches kRouteMinTokens; if none does, the recurrent kernel runs every
      // sequence (so a graph captured from this call stays correct whatever lengths it is replayed with).
      bool any_long = false;
      for (uint32_t b = 0; b < p.batch && !any_long; ++b) {
        any_long = p.cu_seqlens_host[b + 1] - p.cu_seqlens_host[b] >= static_cast<int32_t>(kRouteMinTokens);
      }
      if (!any_long) return LaunchRecurrent(p, s);
    }
    // Every launch size below follows from tokens and batch alone, so the call can be captured into a graph.
    const ChunkArena l = MakeRouteArena(p.tokens, p.batch);
    gate.Expect(roost::HasDeviceRegion(ws, l.total), ROOST_STATUS_WORKSPACE_TOO_SMALL,
                "%u tokens may route sequences to the chunk kernels, which need %llu device workspace bytes",
                p.tokens, static_cast<unsigned long long>(l.total));
    ROOST_GATE_RETURN(gate);
    return LaunchRouted(p, static_cast<uint8_t*>(ws->device), l, s);
  });
}

// ---- Chunk entry points ---------------------------------------------------------------------------------------------

extern "C" ROOST_API RoostStatus roost_gdn_chunk_workspace(RoostContext*, const void* params, RoostWorkspaceSizes* sizes) {
  ROOST_RETURN_IF_FAILED(AdmitForSizing(params, sizes));
  const auto& p = *static_cast<const RoostGatedDeltaRuleParams*>(params);
  const ChunkArena l = MakeChunkArena(p.tokens, p.batch);
  *sizes = RoostWorkspaceSizes{};
  sizes->device_bytes = l.total;
  sizes->pinned_host_bytes = l.tables_bytes;
  sizes->plan_bytes = sizeof(ChunkStamp);
  sizes->device_alignment = 256;
  return ROOST_STATUS_OK;
}

// Writes the chunk table (sequence, first token, tokens) of every 64-token chunk and the per-sequence table (first
// chunk, count, token range) into `host`; returns the chunk count, or -1 when cu_seqlens goes backwards at `*bad`.
static int64_t FillChunkTables(const int32_t* cu, uint32_t batch, const ChunkArena& l, uint8_t* host, uint32_t* bad) {
  auto* chunks = reinterpret_cast<int4*>(host + l.chunk_table);
  auto* seqs = reinterpret_cast<int4*>(host + l.seq_table);
  int32_t n = 0;
  for (uint32_t b = 0; b < batch; ++b) {
    const int32_t lo = cu[b], hi = cu[b + 1];
    if (hi < lo) {
      *bad = b;
      return -1;
    }
    const int32_t first = n;
    for (int32_t t = lo; t < hi; t += kChunk) chunks[n++] = int4{static_cast<int32_t>(b), t, std::min<int32_t>(kChunk, hi - t), 0};
    seqs[b] = int4{first, n - first, lo, hi};
  }
  return n;
}

extern "C" ROOST_API RoostStatus roost_gdn_chunk_plan(RoostContext* ctx, const void* params, const RoostWorkspace* ws,
                                                      void* stream) {
  roost::Gate gate(kOp);
  gate.Expect(ctx != nullptr && params != nullptr && ws != nullptr, ROOST_STATUS_INVALID_ARGUMENT,
              "plan() needs a context, params and a workspace");
  ROOST_GATE_RETURN(gate);
  const auto& p = *static_cast<const RoostGatedDeltaRuleParams*>(params);
  return roost::CatchAll(kOp, [&]() -> RoostStatus {
    ROOST_RETURN_IF_FAILED(Admit(p, true));
    const ChunkArena l = MakeChunkArena(p.tokens, p.batch);
    gate.Expect(roost::HasDeviceRegion(ws, l.total) && ws->pinned_host != nullptr &&
                    ws->pinned_host_bytes >= l.tables_bytes && ws->plan != nullptr &&
                    ws->plan_bytes >= sizeof(ChunkStamp),
                ROOST_STATUS_WORKSPACE_TOO_SMALL,
                "the call needs %llu device bytes, %llu pinned bytes and a %zu-byte plan record",
                static_cast<unsigned long long>(l.total), static_cast<unsigned long long>(l.tables_bytes),
                sizeof(ChunkStamp));
    ROOST_GATE_RETURN(gate);
    ChunkStamp stamp{kPlanMagic, p.batch, p.tokens, 0};
    if (p.batch > 0 && p.tokens > 0) {
      const int32_t* cu = p.cu_seqlens_host;
      gate.Expect(cu[0] == 0 && static_cast<uint32_t>(cu[p.batch]) == p.tokens, ROOST_STATUS_INVALID_ARGUMENT,
                  "cu_seqlens_host runs from %d to %d; it must run from 0 to tokens = %u", cu[0], cu[p.batch], p.tokens);
      ROOST_GATE_RETURN(gate);
      uint32_t bad = 0;
      const int64_t n = FillChunkTables(cu, p.batch, l, static_cast<uint8_t*>(ws->pinned_host), &bad);
      gate.Expect(n >= 0, ROOST_STATUS_INVALID_ARGUMENT, "cu_seqlens_host goes backwards at sequence %u", bad);
      ROOST_GATE_RETURN(gate);
      stamp.chunks = static_cast<uint32_t>(n);
      ROOST_RETURN_IF_FAILED(roost::HipStatus(hipMemcpyAsync(ws->device, ws->pinned_host, l.seq_table + 16ull * p.batch,
                                                             hipMemcpyHostToDevice, roost::Stream(stream)),
                                              kOp, "copy of the chunk tables to the device"));
    }
    std::memcpy(ws->plan, &stamp, sizeof(stamp));
    return ROOST_STATUS_OK;
  });
}

extern "C" ROOST_API RoostStatus roost_gdn_chunk_run(RoostContext* ctx, const void* params, const RoostWorkspace* ws,
                                                     void* stream) {
  roost::Gate gate(kOp);
  gate.Expect(ctx != nullptr && params != nullptr, ROOST_STATUS_INVALID_ARGUMENT, "a context and params are required");
  ROOST_GATE_RETURN(gate);
  const auto& p = *static_cast<const RoostGatedDeltaRuleParams*>(params);
  return roost::CatchAll(kOp, [&]() -> RoostStatus {
    ROOST_RETURN_IF_FAILED(Admit(p, false));
    if (p.batch == 0 || p.tokens == 0) return ROOST_STATUS_OK;
    const ChunkArena l = MakeChunkArena(p.tokens, p.batch);
    gate.Expect(roost::HasDeviceRegion(ws, l.total) && ws->plan != nullptr && ws->plan_bytes >= sizeof(ChunkStamp),
                ROOST_STATUS_WORKSPACE_TOO_SMALL, "the call needs %llu device bytes and its plan record",
                static_cast<unsigned long long>(l.total));
    ROOST_GATE_RETURN(gate);
    ChunkStamp stamp;
    std::memcpy(&stamp, ws->plan, sizeof(stamp));
    if (stamp.magic != kPlanMagic || stamp.batch != p.batch || stamp.tokens != p.tokens || stamp.chunks > l.max_chunks) {
      return roost::Report(ROOST_STATUS_NOT_PLANNED, kOp, "no plan() for %u tokens in %u sequences in this workspace",
                           p.tokens, p.batch);
    }
    if (stamp.chunks == 0) return ROOST_STATUS_OK;
    return LaunchChunk(p, ws, l, stamp.chunks, roost::Stream(stream));
  });
}

// ---- Allocation-free recurrent entry point -------------------------------------------------------------------------
//
// The recurrent variant with its routing scratch (chunk tables and per-(chunk, head) records of the sequences it hands
// to the chunk kernels) in a file-scope device array instead of a caller workspace, for callers that cannot allocate.
// Every call on a device shares that device's array, which keeps the last call's contents; RouteKernel rewrites every
// table entry the chunk kernels read, and the prep kernel writes every record before the scan reads it, so nothing
// has to start at zero. Calls that overlap on one device (two streams, two threads) race on the array.

namespace {

constexpr uint64_t kStaticScratchBytes = 48ull << 20;  // 48 MiB per device, held until the process ends
constexpr int kMaxDevices = 64;

__device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

std::mutex g_scratch_mutex;
uint8_t* g_scratch_ptr[kMaxDevices] = {};  // device address of `scratch` on each device, once looked up

// The device address of this device's `scratch`, looked up once per device with that device current. The array's
// name is a host-side stand-in in host code; only this address may be handed to kernels.
RoostStatus ScratchFor(int device, uint8_t** out) {
  if (device < 0 || device >= kMaxDevices) {
    return roost::Report(ROOST_STATUS_INVALID_ARGUMENT, kOp, "device %d is outside the %d devices this path tracks",
                         device, kMaxDevices);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[device] == nullptr) {
    void* ptr = nullptr;
    ROOST_RETURN_IF_FAILED(
        roost::HipStatus(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), kOp, "lookup of the static scratch array"));
    g_scratch_ptr[device] = static_cast<uint8_t*>(ptr);
  }
  *out = g_scratch_ptr[device];
  return ROOST_STATUS_OK;
}

}  // namespace

extern "C" ROOST_API RoostStatus roost_amd_gdn_recurrent_run_noalloc(RoostContext* ctx, const void* params,
                                                                     void* stream) {
  roost::Gate gate(kOp);
  gate.Expect(ctx != nullptr && params != nullptr, ROOST_STATUS_INVALID_ARGUMENT, "a context and params are required");
  ROOST_GATE_RETURN(gate);
  const auto& p = *static_cast<const RoostGatedDeltaRuleParams*>(params);
  return roost::CatchAll(kOp, [&]() -> RoostStatus {
    ROOST_RETURN_IF_FAILED(Admit(p, false));
    if (p.batch == 0 || p.tokens == 0) return ROOST_STATUS_OK;
    hipStream_t s = roost::Stream(stream);
    if (p.tokens < kRouteMinTokens) return LaunchRecurrent(p, s);
    const ChunkArena l = MakeRouteArena(p.tokens, p.batch);
    gate.Expect(l.total <= kStaticScratchBytes, ROOST_STATUS_INVALID_ARGUMENT,
                "%u tokens in %u sequences need %llu bytes of routing scratch; the allocation-free path holds %llu",
                p.tokens, p.batch, static_cast<unsigned long long>(l.total),
                static_cast<unsigned long long>(kStaticScratchBytes));
    ROOST_GATE_RETURN(gate);
    int current = -1;
    ROOST_RETURN_IF_FAILED(roost::HipStatus(hipGetDevice(&current), kOp, "query of the current device"));
    gate.Expect(current == ctx->device, ROOST_STATUS_INVALID_ARGUMENT,
                "the context is for device %d but device %d is current", ctx->device, current);
    ROOST_GATE_RETURN(gate);
    uint8_t* base = nullptr;
    ROOST_RETURN_IF_FAILED(ScratchFor(current, &base));
    return LaunchRouted(p, base, l, s);
  });
}
