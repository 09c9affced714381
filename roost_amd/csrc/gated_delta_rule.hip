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
// no gather or state copy): four 256-thread workgroups per (sequence, value head), one per quarter of the value columns,
// each lane holding 16 floats of S in registers (RecurrentUnit). Sequences of 16 or more tokens go to the chunk (WY)
// kernels instead; their prep workgroups share one launch with the recurrent ones (WyPrepRecurrentKernel). The gates
// may be folded in (roost_amd_gdn_recurrent_gated_run): g and beta are then computed where they are read. A decode
// step of the whole layer -- CausalConv1d, the gates, the recurrence and GatedRmsNorm -- runs as two launches
// (ConvRecurrentKernel, then the norm with the convolution's state update; roost_amd_gdn_decode_layer_run).

#include <algorithm>
#include <cmath>
#include <cstring>
#include <cstddef>
#include <mutex>

#include "common.h"
#include "gdn_layer.h"

namespace {

using namespace roost_dev;

constexpr uint32_t kDim = 128;          // key and value head size (Qwen3.5)
constexpr uint32_t kMaxHeads = 128;     // value heads of one call
constexpr uint32_t kMaxGroup = 8;       // value heads per key head
constexpr uint64_t kMaxTokens = uint64_t{1} << 24;
constexpr uint32_t kMaxBatch = 1u << 20;
constexpr uint32_t kChunk = 64;
// The recurrent variant hands a sequence of at least this many tokens to the chunk (WY) kernels: one token of the
// token-serial recurrence costs about as much latency as a chunk step covering 64 tokens.
constexpr uint32_t kRouteMinTokens = 16;
constexpr uint32_t kPlanMagic = 0x50444752;  // "RGDP"

// Row widths of the views (elements): q and k rows hold k_heads heads, v and output rows v_heads heads; a stride of 0
// means rows packed at their width. A state slot is [v_heads, 128, 128] fp32.
uint64_t KRow(const RoostGatedDeltaRuleParams& p) { return uint64_t{p.k_heads} * kDim; }
uint64_t VRow(const RoostGatedDeltaRuleParams& p) { return uint64_t{p.v_heads} * kDim; }
uint64_t StateElems(const RoostGatedDeltaRuleParams& p) { return uint64_t{p.v_heads} * kDim * kDim; }
uint64_t Stride(uint32_t s, uint64_t row) { return s == 0 ? row : s; }

constexpr char kOp[] = "gated_delta_rule";

// The call's rules, shared by both variants. The statuses are the contract's (the reference refuses the same shapes:
// kernels/src/ops/gated_delta_rule.cu:231-278); `planning` adds plan()'s need for the host cu_seqlens copy.
// fused_gates: g and beta come from the call's GatedDeltaRuleGates inputs, so their spans are not read.
RoostStatus Admit(const RoostGatedDeltaRuleParams& p, bool planning, bool fused_gates = false) {
  roost::Gate gate(kOp);
  gate.Header(&p, sizeof(RoostGatedDeltaRuleParams))
      .Expect(p.k_dim == kDim && p.v_dim == kDim, ROOST_STATUS_UNSUPPORTED,
              "head sizes %u / %u (key / value): the kernels are built for 128 (Qwen3.5)", p.k_dim, p.v_dim)
      .Expect(p.k_heads >= 1 && p.v_heads % std::max(p.k_heads, 1u) == 0 && p.v_heads / std::max(p.k_heads, 1u) >= 1 &&
                  p.v_heads / std::max(p.k_heads, 1u) <= kMaxGroup && p.v_heads <= kMaxHeads,
              ROOST_STATUS_UNSUPPORTED, "%u value heads over %u key heads: built for 1 to %u value heads per key head, "
              "at most %u value heads", p.v_heads, p.k_heads, kMaxGroup, kMaxHeads)
      .Expect(p.l2_norm_qk != 0, ROOST_STATUS_UNSUPPORTED, "l2_norm_qk = 0: the kernels always normalise q and k")
      .Expect(p.tokens <= kMaxTokens && p.batch <= kMaxBatch, ROOST_STATUS_INVALID_ARGUMENT,
              "%u tokens in %u sequences exceeds one call's limits (%llu tokens, %u sequences)", p.tokens, p.batch,
              static_cast<unsigned long long>(kMaxTokens), kMaxBatch);
  ROOST_GATE_RETURN(gate);
  const uint64_t krow = KRow(p), vrow = VRow(p);
  const uint64_t qs = Stride(p.q_stride, krow), ks = Stride(p.k_stride, krow), vs = Stride(p.v_stride, vrow);
  gate.Expect(qs >= krow && ks >= krow && vs >= vrow, ROOST_STATUS_INVALID_ARGUMENT,
              "row strides q %llu, k %llu, v %llu: q and k rows hold %llu elements, v rows %llu",
              static_cast<unsigned long long>(qs), static_cast<unsigned long long>(ks),
              static_cast<unsigned long long>(vs), static_cast<unsigned long long>(krow),
              static_cast<unsigned long long>(vrow));
  ROOST_GATE_RETURN(gate);
  // A strided view reaches (tokens - 1) * stride + one row.
  const uint64_t t = p.tokens;
  auto reach = [t](uint64_t stride, uint64_t row) { return t == 0 ? 0 : (t - 1) * stride + row; };
  gate.Tensor("q", p.q, ROOST_DTYPE_BF16, reach(qs, krow))
      .Tensor("k", p.k, ROOST_DTYPE_BF16, reach(ks, krow))
      .Tensor("v", p.v, ROOST_DTYPE_BF16, reach(vs, vrow));
  ROOST_GATE_RETURN(gate);
  // g, beta and output of another type are shapes the kernels do not cover (UNSUPPORTED, as the contract has it).
  gate.Expect(fused_gates || (p.g.dtype == ROOST_DTYPE_F32 && p.beta.dtype == ROOST_DTYPE_BF16),
              ROOST_STATUS_UNSUPPORTED, "g %s, beta %s: built for f32 g with bf16 beta", roost::Describe(p.g.dtype).name,
              roost::Describe(p.beta.dtype).name)
      .Expect(p.output.dtype == ROOST_DTYPE_BF16, ROOST_STATUS_UNSUPPORTED, "output %s: built for bf16 output",
              roost::Describe(p.output.dtype).name);
  ROOST_GATE_RETURN(gate);
  if (!fused_gates) {
    gate.Tensor("g", p.g, ROOST_DTYPE_F32, t * p.v_heads)
        .Tensor("beta", p.beta, ROOST_DTYPE_BF16, t * p.v_heads)
        .Aligned("g", p.g.address, 16)
        .Aligned("beta", p.beta.address, 16);
  }
  gate.Tensor("output", p.output, ROOST_DTYPE_BF16, t * vrow)
      .Tensor("state", p.state, ROOST_DTYPE_F32, StateElems(p))
      .Expect(p.state.length % StateElems(p) == 0, ROOST_STATUS_INVALID_ARGUMENT,
              "state pool of %llu floats is not a whole number of [%u, 128, 128] slots",
              static_cast<unsigned long long>(p.state.length), p.v_heads)
      .Tensor("state_slots", p.state_slots, ROOST_DTYPE_I32, p.batch)
      .Tensor("cu_seqlens", p.cu_seqlens, ROOST_DTYPE_I32, uint64_t{p.batch} + 1)
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
              "%u tokens in %u sequences exceeds one call's limits", p.tokens, p.batch)
      .Expect(p.v_heads >= 1 && p.v_heads <= kMaxHeads, ROOST_STATUS_UNSUPPORTED,
              "%u value heads: built for 1 to %u", p.v_heads, kMaxHeads);
  return gate.status();
}

float Scale(const RoostGatedDeltaRuleParams& p) {
  return p.scale != 0.0f ? p.scale : 1.0f / std::sqrt(static_cast<float>(kDim));
}

// The GatedDeltaRuleGates inputs of a call that folds the gates in (roost_amd_gdn_recurrent_gated_run).
struct GateSource {
  const void* a = nullptr;  // [tokens, v_heads] at a_stride
  const void* b = nullptr;  // [tokens, v_heads] at b_stride
  const void* a_log = nullptr;
  const void* dt_bias = nullptr;
  uint32_t a_t = 0, b_t = 0, alog_t = 0, dtb_t = 0;  // dtypes (bf16 or f32)
  uint64_t a_stride = 0, b_stride = 0;
};

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
  uint32_t vh;     // value heads (the rows of v, output, g and beta, the heads of a state slot)
  uint32_t group;  // value heads per key head: value head h reads q / k head h / group
  uint32_t batch;  // sequences of the call (the length of slots)
  GateSource gs;   // when gs.a is set, g and beta are computed from these instead of read from g and beta
};

// g and beta of (token, value head): read from the call's g and beta, or computed from the gates' inputs exactly as
// the GatedDeltaRuleGates op computes and stores them (beta rounded to bf16, as its bf16 output holds it).
// In two steps, so that a kernel can request a token's gate inputs early and compute from them later: GateLoad reads
// (a, dt_bias, a_log, b), or (g, beta) when the gates are not folded in; GateFrom computes.
struct GateIn {
  float x0, x1, x2, x3;
};
__device__ __forceinline__ GateIn GateLoad(const GdnArgs& a, uint64_t tok, uint32_t h) {
  if (a.gs.a != nullptr) {
    return GateIn{LoadF(a.gs.a, a.gs.a_t, static_cast<int64_t>(tok * a.gs.a_stride + h)),
                  LoadF(a.gs.dt_bias, a.gs.dtb_t, h), LoadF(a.gs.a_log, a.gs.alog_t, h),
                  LoadF(a.gs.b, a.gs.b_t, static_cast<int64_t>(tok * a.gs.b_stride + h))};
  }
  const uint64_t gi = tok * a.vh + h;
  return GateIn{a.g[gi], Bf16ToF32(a.beta[gi]), 0.0f, 0.0f};
}
__device__ __forceinline__ void GateFrom(const GdnArgs& a, const GateIn& in, float& g, float& beta) {
  if (a.gs.a != nullptr) {
    float bv;
    GateValues(in.x0, in.x1, in.x2, in.x3, g, bv);
    beta = Bf16ToF32(F32ToBf16(bv));
  } else {
    g = in.x0;
    beta = in.x1;
  }
}
__device__ __forceinline__ void GateAt(const GdnArgs& a, uint64_t tok, uint32_t h, float& g, float& beta) {
  GateFrom(a, GateLoad(a, tok, h), g, beta);
}

// Zeros in device memory: the stand-in a kernel reads for an absent operand, so that its request needs no branch.
__device__ __align__(16) uint32_t kZeroTaps[4] = {0u, 0u, 0u, 0u};

// GateLoad / GateFrom in the same two steps, without a branch around any request: every input is requested both as
// bf16 and as f32, the form its dtype does not use (and every input of the source not in use) from kZeroTaps, so the
// two requests' bits combine into the value's f32 bits with one shift and one or. (Requests inside a dtype branch made
// each wait for everything in flight before it.)
struct GateRaw {
  uint32_t h[4], w[4];  // bf16 and f32 requests of a, dt_bias, a_log, b (folded) or of g and beta (read)
};
__device__ __forceinline__ GateRaw GateRequest(const GdnArgs& a, uint64_t tok, uint32_t h) {
  const bool fold = a.gs.a != nullptr;
  const auto* z16 = reinterpret_cast<const uint16_t*>(kZeroTaps);
  GateRaw r;
  auto both = [&](int q, bool use, const void* p, uint32_t dt, uint64_t i) {
    const bool bf = use && dt == ROOST_DTYPE_BF16, f32 = use && dt != ROOST_DTYPE_BF16;
    r.h[q] = *(bf ? static_cast<const uint16_t*>(p) + i : z16);
    r.w[q] = *(f32 ? static_cast<const uint32_t*>(p) + i : kZeroTaps);
  };
  const uint64_t gi = tok * a.vh + h;
  both(0, true, fold ? a.gs.a : a.g, fold ? a.gs.a_t : ROOST_DTYPE_F32, fold ? tok * a.gs.a_stride + h : gi);
  both(1, true, fold ? a.gs.dt_bias : static_cast<const void*>(a.beta), fold ? a.gs.dtb_t : ROOST_DTYPE_BF16,
       fold ? h : gi);
  both(2, fold, a.gs.a_log, a.gs.alog_t, h);
  both(3, fold, a.gs.b, a.gs.b_t, tok * a.gs.b_stride + h);
  return r;
}
__device__ __forceinline__ GateIn GateWiden(const GdnArgs& a, const GateRaw& r) {
  float x[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) x[q] = __uint_as_float((r.h[q] << 16) | r.w[q]);
  return a.gs.a != nullptr ? GateIn{x[0], x[1], x[2], x[3]} : GateIn{x[0], x[1], 0.0f, 0.0f};
}

// The same two steps with one branch per input on its dtype and a single request each (the bits kept as loaded, no
// use of them inside the branch). ConvRecurrentKernel runs faster on this form (the decode layer 0.0626 against
// 0.0631 ms), the recurrent kernels on GateRequest's.
__device__ __forceinline__ uint32_t RequestBits(const void* p, uint32_t dt, int64_t i) {
  return dt == ROOST_DTYPE_BF16 ? static_cast<uint32_t>(static_cast<const uint16_t*>(p)[i])
                                : static_cast<const uint32_t*>(p)[i];
}
__device__ __forceinline__ GateRaw GateRequestByType(const GdnArgs& a, uint64_t tok, uint32_t h) {
  GateRaw r{};
  if (a.gs.a != nullptr) {
    r.h[0] = RequestBits(a.gs.a, a.gs.a_t, static_cast<int64_t>(tok * a.gs.a_stride + h));
    r.h[1] = RequestBits(a.gs.dt_bias, a.gs.dtb_t, h);
    r.h[2] = RequestBits(a.gs.a_log, a.gs.alog_t, h);
    r.h[3] = RequestBits(a.gs.b, a.gs.b_t, static_cast<int64_t>(tok * a.gs.b_stride + h));
  } else {
    const uint64_t gi = tok * a.vh + h;
    r.w[0] = __float_as_uint(a.g[gi]);
    r.w[1] = a.beta[gi];
  }
  return r;
}
__device__ __forceinline__ GateIn GateWidenByType(const GdnArgs& a, const GateRaw& r) {
  auto f = [](uint32_t v, uint32_t dt) { return __uint_as_float(dt == ROOST_DTYPE_BF16 ? v << 16 : v); };
  if (a.gs.a != nullptr) {
    return GateIn{f(r.h[0], a.gs.a_t), f(r.h[1], a.gs.dtb_t), f(r.h[2], a.gs.alog_t), f(r.h[3], a.gs.b_t)};
  }
  return GateIn{__uint_as_float(r.w[0]), __uint_as_float(r.w[1] << 16), 0.0f, 0.0f};
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

// Sum over the 8 lanes of a row group (lanes 8m .. 8m + 7).
__device__ __forceinline__ float OctSum(float x) {
  x += __shfl_xor(x, 1, 64);
  x += __shfl_xor(x, 2, 64);
  x += __shfl_xor(x, 4, 64);
  return x;
}

__device__ __forceinline__ float QuadSum(float x) {
  x += __shfl_xor(x, 1, 64);
  x += __shfl_xor(x, 2, 64);
  return x;
}

// The value columns of a state are independent in the recurrence (column c reads only S[:, c], k, q and v[c]), so each
// (sequence, value head) is split over kRecQuarters workgroups of 32 columns. Within one, wavefront w holds rows
// 32 w .. + 31 and lane l rows 32 w + 4 (l % 8) .. + 3 of columns 4 (l / 8) .. + 3 (16 floats): a state-row access by a
// wavefront is eight whole 128-byte lines, and the dot products over rows reduce over the 8 lanes of a row group and
// then over the 4 wavefronts through LDS. At 16 floats of state per lane the workgroups of a whole decode step are
// resident at once, beside the prep workgroups when both share a launch.
constexpr uint32_t kRecQuarters = 4;
constexpr uint32_t kRecThreads = 256;

// One token of the recurrence for one thread's share of a (sequence, value head): rows row0 .. + 3 and kC value
// columns of S, in groups of 4: group m of lane cg is columns 32 m + 4 cg .. + 3 (so the 8 lanes of a row group cover
// whole 128-byte rows of S per access), from the token's q and k elements
// 2 lane, 2 lane + 1 (the norms), rows row0 .. + 3 of q and k, the kC columns of v and the token's gates; red_sk and
// red_o are the [4 wavefronts][8 kC] LDS reduction arrays of the columns' workgroup (two workgroup barriers). Lanes with
// w == 0 and rg == 0 receive their kC output columns. Every column sees the operations RecurrentUnit applies to it, in
// the same order (RecurrentUnit keeps its own copy, for its register allocation), so the decode layer's
// ConvRecurrentKernel (kC = 4) and the recurrent kernels agree bit for bit.
template <int kC>
__device__ __forceinline__ void RecurrentStep(float (&s)[4][kC], const float (&q2)[2], const float (&k2)[2],
                                              const float (&q4)[4], float (&k4)[4], const float (&vv)[kC], float graw,
                                              float beta, float scale, int w, int rg, int cg, float (*red_sk)[8 * kC],
                                              float (*red_o)[8 * kC], float (&ot)[kC]) {
  static_assert(kC % 4 == 0, "columns go through LDS as float4");
  const float decay = expf(graw);
  float qq = fmaf(q2[0], q2[0], q2[1] * q2[1]), kk = fmaf(k2[0], k2[0], k2[1] * k2[1]);
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    qq += __shfl_xor(qq, o, 64);
    kk += __shfl_xor(kk, o, 64);
  }
  const float qn = scale / sqrtf(qq + 1e-6f);
  const float kn = 1.0f / sqrtf(kk + 1e-6f);
  // S^T k: this lane's 4 rows, the row group's 32, then the workgroup's 128 through LDS.
  float sk[kC];
#pragma unroll
  for (int c = 0; c < kC; ++c) sk[c] = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    k4[i] *= kn;
#pragma unroll
    for (int c = 0; c < kC; ++c) sk[c] = fmaf(s[i][c], k4[i], sk[c]);
  }
#pragma unroll
  for (int c = 0; c < kC; ++c) sk[c] = OctSum(sk[c]);
  if (rg == 0) {
#pragma unroll
    for (int c = 0; c < kC; c += 4)
      *reinterpret_cast<float4*>(&red_sk[w][8 * c + 4 * cg]) = make_float4(sk[c], sk[c + 1], sk[c + 2], sk[c + 3]);
  }
  __syncthreads();
  float d[kC];
#pragma unroll
  for (int c = 0; c < kC; c += 4) {
    float4 tot = *reinterpret_cast<const float4*>(&red_sk[0][8 * c + 4 * cg]);
#pragma unroll
    for (int ww = 1; ww < 4; ++ww) {
      const float4 x = *reinterpret_cast<const float4*>(&red_sk[ww][8 * c + 4 * cg]);
      tot = make_float4(tot.x + x.x, tot.y + x.y, tot.z + x.z, tot.w + x.w);
    }
    d[c] = beta * (vv[c] - decay * tot.x);
    d[c + 1] = beta * (vv[c + 1] - decay * tot.y);
    d[c + 2] = beta * (vv[c + 2] - decay * tot.z);
    d[c + 3] = beta * (vv[c + 3] - decay * tot.w);
  }
  float o[kC];
#pragma unroll
  for (int c = 0; c < kC; ++c) o[c] = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float ki = k4[i], qi = q4[i] * qn;
#pragma unroll
    for (int c = 0; c < kC; ++c) s[i][c] = fmaf(s[i][c], decay, ki * d[c]);
#pragma unroll
    for (int c = 0; c < kC; ++c) o[c] = fmaf(s[i][c], qi, o[c]);
  }
#pragma unroll
  for (int c = 0; c < kC; ++c) o[c] = OctSum(o[c]);
  if (rg == 0) {
#pragma unroll
    for (int c = 0; c < kC; c += 4)
      *reinterpret_cast<float4*>(&red_o[w][8 * c + 4 * cg]) = make_float4(o[c], o[c + 1], o[c + 2], o[c + 3]);
  }
  __syncthreads();
  if (w == 0 && rg == 0) {
#pragma unroll
    for (int c = 0; c < kC; c += 4) {
      float4 t = *reinterpret_cast<const float4*>(&red_o[0][8 * c + 4 * cg]);
#pragma unroll
      for (int ww = 1; ww < 4; ++ww) {
        const float4 x = *reinterpret_cast<const float4*>(&red_o[ww][8 * c + 4 * cg]);
        t = make_float4(t.x + x.x, t.y + x.y, t.z + x.z, t.w + x.w);
      }
      ot[c] = t.x;
      ot[c + 1] = t.y;
      ot[c + 2] = t.z;
      ot[c + 3] = t.w;
    }
  }
}

// The state rows row0 .. + 3 of a lane's kC columns (groups of 4 at sp + 32 m, row stride kDim), as fp32 streams that
// skip the caches; zeros (read from kZeroTaps, without a branch) when `valid` is false.
template <int kC>
__device__ __forceinline__ void LoadStateRows(bool valid, const float* sp, int row0, float (&s)[4][kC]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int c = 0; c < kC; c += 4) {
      const float4 v =
          LoadStreamF4(valid ? sp + (row0 + i) * kDim + 8 * c : reinterpret_cast<const float*>(kZeroTaps));
      s[i][c] = v.x;
      s[i][c + 1] = v.y;
      s[i][c + 2] = v.z;
      s[i][c + 3] = v.w;
    }
}
template <int kC>
__device__ __forceinline__ void StoreStateRows(float* sp, int row0, const float (&s)[4][kC]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int c = 0; c < kC; c += 4)
      StoreStreamF4(sp + (row0 + i) * kDim + 8 * c, make_float4(s[i][c], s[i][c + 1], s[i][c + 2], s[i][c + 3]));
}

// Whether sequence j runs on the recurrent kernel with state slot `slot`: non-empty, not routed to the chunk kernels.
__device__ __forceinline__ bool ChainMember(const GdnArgs& a, uint32_t j, int32_t slot) {
  if (a.slots[j] != slot) return false;
  const int32_t u0 = a.cu[j], u1 = a.cu[j + 1];
  return u1 > u0 && (a.route_min <= 0 || u1 - u0 < a.route_min);
}

// Workgroup (sequence b, value head h, column quarter): the token-serial recurrence with its share of S in registers.
template <bool kVec, bool kPreload = false, bool kPreGate = kPreload>
__device__ __forceinline__ void RecurrentUnit(const GdnArgs& a, uint32_t b, uint32_t h, uint32_t quarter) {
  __shared__ float red_sk[4][32], red_o[4][32];
  int32_t t0 = a.cu[b];
  int32_t t1 = a.cu[b + 1];
  if (t1 <= t0) return;  // an empty sequence leaves its slot untouched
  if (a.route_min > 0 && t1 - t0 >= a.route_min) return;  // run by the chunk kernels
  const int32_t slot = a.slots[b];
  const bool has_slot = slot >= 0 && static_cast<uint64_t>(slot) < a.pool_slots;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int rg = lane & 7;  // key rows 32 w + 4 rg .. + 3
  const int cg = lane >> 3;  // value columns 32 quarter + 4 cg .. + 3
  const int row0 = 32 * w + 4 * rg;
  const uint32_t col = 32 * quarter + 4 * cg;
  const uint32_t kh = h / a.group;
  // Wavefront 0 scans the slot table for sequences sharing this one's slot (below). Its first kScanNow entries per
  // lane are requested first of all: the memory counter retires in order, so waiting for them later does not wait
  // for the state loads issued after them.
  constexpr int kScanNow = 2;  // slot entries per lane requested up front (128 sequences)
  int32_t sj[kScanNow] = {};
  if (has_slot && w == 0) {
#pragma unroll
    for (int i = 0; i < kScanNow; ++i) sj[i] = a.slots[min(static_cast<uint32_t>(lane + 64 * i), a.batch - 1)];
  }
  // With kPreload the first token's q, k and v words and gate inputs are requested before the state too: its norms
  // and gates then wait only for themselves and are computed while the state is in flight (RecurrentKernel: 48.4
  // against 49.5 us at 128 states; inside the prep launch's 80-register bound the extra live registers spill, and it
  // keeps the loads in the step). kPreGate requests only the gate inputs early: the prep launch does so when it
  // computes the gates itself (four inputs and the gate arithmetic per token: config 5's GDN layer 0.0446 against
  // 0.0460 ms), not when it reads g and beta (0.0415 against 0.0412 ms).
  uint32_t qw = 0, kw = 0;
  uint2 qr = make_uint2(0, 0), kr = qr, vw = qr;
  auto load_rows = [&](int32_t tok) {
    if constexpr (kVec) {
      const uint16_t* qrow = a.q + static_cast<uint64_t>(tok) * a.q_stride + kh * kDim;
      const uint16_t* krow = a.k + static_cast<uint64_t>(tok) * a.k_stride + kh * kDim;
      const uint16_t* vrow = a.v + static_cast<uint64_t>(tok) * a.v_stride + h * kDim + col;
      qw = *reinterpret_cast<const uint32_t*>(qrow + 2 * lane);
      kw = *reinterpret_cast<const uint32_t*>(krow + 2 * lane);
      qr = *reinterpret_cast<const uint2*>(qrow + row0);
      kr = *reinterpret_cast<const uint2*>(krow + row0);
      vw = *reinterpret_cast<const uint2*>(vrow);
    }
  };
  GateIn gin{};
  GateRaw graw0{};
  if constexpr (kPreload) load_rows(t0);
  if constexpr (kPreGate) graw0 = GateRequest(a, static_cast<uint64_t>(t0), h);
  bool first_step = kPreload, first_gate = kPreGate;
  float4 s[4];
  float* sp = has_slot ? a.state + (static_cast<uint64_t>(slot) * a.vh + h) * kDim * kDim + col : nullptr;
  // Requested without a branch (zeros from kZeroTaps without a slot or an initial state): behind a branch, every wait
  // after it for a request made before it would also wait for the state, as on the path that skips it.
  const bool load_state = has_slot && a.use_initial_state;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    s[i] = LoadStreamF4(load_state ? sp + (row0 + i) * kDim : reinterpret_cast<const float*>(kZeroTaps));
  // Sequences of one call that share a slot run in batch order, as CpuOps runs them: each starts from the state the
  // one before it left (or from zero without use_initial_state). The workgroup of the first such sequence carries
  // the state through all of them in registers and writes it once; the others' workgroups leave.
  // The scan runs in the first token step, after that step's loads are issued; its verdict reaches the other
  // wavefronts through LDS at the step's first barrier.
  __shared__ uint32_t chain_flags;  // bit 0: an earlier sequence shares the slot; bit 1: a later one does
  bool scan_pending = has_slot, chained = false;
  uint32_t cur = b;  // the sequence whose tokens run now (later members of a chain follow in turn)
  for (int32_t tok = t0;;) {
    const uint16_t* qrow = a.q + static_cast<uint64_t>(tok) * a.q_stride + kh * kDim;
    const uint16_t* krow = a.k + static_cast<uint64_t>(tok) * a.k_stride + kh * kDim;
    // The norms: lane l squares elements 2l, 2l + 1 and the wavefront reduces, so that every wavefront has them whole.
    float q2[2], k2[2], q4[4], k4[4], vv[4];
    const uint16_t* vrow = a.v + static_cast<uint64_t>(tok) * a.v_stride + h * kDim + col;
    if constexpr (kVec) {
      if (!first_step) load_rows(tok);
      q2[0] = Bf16LoToF32(qw); q2[1] = Bf16HiToF32(qw);
      k2[0] = Bf16LoToF32(kw); k2[1] = Bf16HiToF32(kw);
      q4[0] = Bf16LoToF32(qr.x); q4[1] = Bf16HiToF32(qr.x); q4[2] = Bf16LoToF32(qr.y); q4[3] = Bf16HiToF32(qr.y);
      k4[0] = Bf16LoToF32(kr.x); k4[1] = Bf16HiToF32(kr.x); k4[2] = Bf16LoToF32(kr.y); k4[3] = Bf16HiToF32(kr.y);
      vv[0] = Bf16LoToF32(vw.x); vv[1] = Bf16HiToF32(vw.x); vv[2] = Bf16LoToF32(vw.y); vv[3] = Bf16HiToF32(vw.y);
    } else {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        q2[i] = Bf16ToF32(qrow[2 * lane + i]);
        k2[i] = Bf16ToF32(krow[2 * lane + i]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        q4[i] = Bf16ToF32(qrow[row0 + i]);
        k4[i] = Bf16ToF32(krow[row0 + i]);
        vv[i] = Bf16ToF32(vrow[i]);
      }
    }
    gin = first_gate ? GateWiden(a, graw0) : GateLoad(a, static_cast<uint64_t>(tok), h);
    first_step = false;
    first_gate = false;
    float graw, beta;
    GateFrom(a, gin, graw, beta);
    const float decay = expf(graw);
    float qq = fmaf(q2[0], q2[0], q2[1] * q2[1]), kk = fmaf(k2[0], k2[0], k2[1] * k2[1]);
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      qq += __shfl_xor(qq, o, 64);
      kk += __shfl_xor(kk, o, 64);
    }
    if (scan_pending && w == 0) {  // (the loads above have landed: the slot entries, requested earlier, have too)
      // Tied to the norms, so that the compiler cannot move the scan above this step's loads.
#pragma unroll
      for (int i = 0; i < kScanNow; ++i) asm volatile("" : "+v"(sj[i]) : "v"(qq), "v"(kk));
      bool earlier = false, later = false;
#pragma unroll
      for (int i = 0; i < kScanNow; ++i) {
        const uint32_t jj = static_cast<uint32_t>(lane + 64 * i);
        if (jj < a.batch && jj != b && sj[i] == slot && ChainMember(a, jj, slot)) {
          earlier |= jj < b;
          later |= jj > b;
        }
      }
      for (uint32_t jj = static_cast<uint32_t>(lane + 64 * kScanNow); jj < a.batch; jj += 64) {
        if (jj != b && ChainMember(a, jj, slot)) {
          earlier |= jj < b;
          later |= jj > b;
        }
      }
      const uint32_t f = (__any(earlier) ? 1u : 0u) | (__any(later) ? 2u : 0u);  // whole-wavefront ballots
      if (lane == 0) chain_flags = f;
    }
    const float qn = a.scale / sqrtf(qq + 1e-6f);
    const float kn = 1.0f / sqrtf(kk + 1e-6f);
    // S^T k: this lane's 4 rows, the row group's 32, then the workgroup's 128 through LDS.
    float sk[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      k4[i] *= kn;
      sk[0] = fmaf(s[i].x, k4[i], sk[0]);
      sk[1] = fmaf(s[i].y, k4[i], sk[1]);
      sk[2] = fmaf(s[i].z, k4[i], sk[2]);
      sk[3] = fmaf(s[i].w, k4[i], sk[3]);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) sk[c] = OctSum(sk[c]);
    if (rg == 0) *reinterpret_cast<float4*>(&red_sk[w][4 * cg]) = make_float4(sk[0], sk[1], sk[2], sk[3]);
    __syncthreads();
    if (scan_pending) {
      scan_pending = false;
      const uint32_t f = chain_flags;
      if (f & 1u) return;  // nothing written yet; every wavefront of the workgroup leaves here
      chained = (f & 2u) != 0;
    }
    float4 tot = *reinterpret_cast<const float4*>(&red_sk[0][4 * cg]);
#pragma unroll
    for (int ww = 1; ww < 4; ++ww) {
      const float4 x = *reinterpret_cast<const float4*>(&red_sk[ww][4 * cg]);
      tot = make_float4(tot.x + x.x, tot.y + x.y, tot.z + x.z, tot.w + x.w);
    }
    const float d[4] = {beta * (vv[0] - decay * tot.x), beta * (vv[1] - decay * tot.y),
                        beta * (vv[2] - decay * tot.z), beta * (vv[3] - decay * tot.w)};
    float o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float ki = k4[i], qi = q4[i] * qn;
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
    for (int c = 0; c < 4; ++c) o[c] = OctSum(o[c]);
    if (rg == 0) *reinterpret_cast<float4*>(&red_o[w][4 * cg]) = make_float4(o[0], o[1], o[2], o[3]);
    __syncthreads();
    if (w == 0 && rg == 0) {
      float4 ot = *reinterpret_cast<const float4*>(&red_o[0][4 * cg]);
#pragma unroll
      for (int ww = 1; ww < 4; ++ww) {
        const float4 x = *reinterpret_cast<const float4*>(&red_o[ww][4 * cg]);
        ot = make_float4(ot.x + x.x, ot.y + x.y, ot.z + x.z, ot.w + x.w);
      }
      uint2 pw;
      pw.x = PackBf16(ot.x, ot.y);
      pw.y = PackBf16(ot.z, ot.w);
      *reinterpret_cast<uint2*>(a.out + (static_cast<uint64_t>(tok) * a.vh + h) * kDim + col) = pw;
    }
    if (++tok < t1) continue;
    if (!chained) break;
    // The next sequence of the chain, if any (a uniform walk: every lane reads the same entries; rare).
    uint32_t next = cur + 1;
    while (next < a.batch && !ChainMember(a, next, slot)) ++next;
    if (next >= a.batch) break;
    cur = next;
    tok = a.cu[cur];
    t1 = a.cu[cur + 1];
    if (!a.use_initial_state) {
#pragma unroll
      for (int i = 0; i < 4; ++i) s[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  if (has_slot) {
#pragma unroll
    for (int i = 0; i < 4; ++i) StoreStreamF4(sp + (row0 + i) * kDim, s[i]);
  }
}

template <bool kVec>
__global__ void __launch_bounds__(kRecThreads) RecurrentKernel(GdnArgs a) {
  RecurrentUnit<kVec, true>(a, blockIdx.x, blockIdx.y / kRecQuarters, blockIdx.y % kRecQuarters);
}

GdnArgs MakeArgs(const RoostGatedDeltaRuleParams& p, const GateSource& gs = GateSource{}) {
  GdnArgs a{};
  a.gs = gs;
  a.q = static_cast<const uint16_t*>(p.q.address);
  a.k = static_cast<const uint16_t*>(p.k.address);
  a.v = static_cast<const uint16_t*>(p.v.address);
  a.g = static_cast<const float*>(p.g.address);
  a.beta = static_cast<const uint16_t*>(p.beta.address);
  a.out = static_cast<uint16_t*>(p.output.address);
  a.state = static_cast<float*>(p.state.address);
  a.slots = static_cast<const int32_t*>(p.state_slots.address);
  a.cu = static_cast<const int32_t*>(p.cu_seqlens.address);
  a.q_stride = Stride(p.q_stride, KRow(p));
  a.k_stride = Stride(p.k_stride, KRow(p));
  a.v_stride = Stride(p.v_stride, VRow(p));
  a.pool_slots = p.state.length / StateElems(p);
  a.vh = p.v_heads;
  a.group = p.v_heads / p.k_heads;
  a.batch = p.batch;
  a.use_initial_state = p.use_initial_state;
  a.scale = Scale(p);
  return a;
}

bool Vec16(const RoostGatedDeltaRuleParams& p) {
  auto Aligned = [](const void* a, uint64_t n) { return roost::IsAligned(a, n); };
  const uint64_t qs = Stride(p.q_stride, KRow(p)), ks = Stride(p.k_stride, KRow(p)), vs = Stride(p.v_stride, VRow(p));
  return Aligned(p.q.address, 16) && Aligned(p.k.address, 16) && Aligned(p.v.address, 16) && qs % 8 == 0 &&
         ks % 8 == 0 && vs % 8 == 0;
}

RoostStatus LaunchRecurrent(const RoostGatedDeltaRuleParams& p, hipStream_t stream, int32_t route_min = 0,
                            const GateSource& gs = GateSource{}) {
  GdnArgs a = MakeArgs(p, gs);
  a.route_min = route_min;
  const dim3 grid(p.batch, p.v_heads * kRecQuarters);
  if (Vec16(p)) {
    hipLaunchKernelGGL(RecurrentKernel<true>, grid, dim3(kRecThreads), 0, stream, a);
  } else {
    hipLaunchKernelGGL(RecurrentKernel<false>, grid, dim3(kRecThreads), 0, stream, a);
  }
  return roost::HipStatus(hipGetLastError(), kOp, "recurrent launch");
}

// ---- Decode layer: CausalConv1d + gates + recurrence in one kernel, then GatedRmsNorm + the convolution's state ---
//
// ConvRecurrentKernel (below) runs the recurrent kernel's quarter workgroups with the convolution and the gates
// computed where the recurrence reads them; one more launch (RunNormAndConvState) normalises the GDN output rows and
// writes the convolution states. The convolution's output, g and beta never reach memory.
struct LayerArgs {
  GdnArgs a;                  // the recurrence; its q, k and v are not used (the workgroups convolve them)
  const uint16_t* x;          // the convolution's input [tokens, channels] (bf16)
  const uint16_t* conv_w;     // [channels, width]
  const uint16_t* conv_b;     // [channels], or NULL
  const void* conv_state;     // [slots, channels, width - 1]
  const int32_t* conv_slots;  // [batch]
  uint64_t conv_pool_slots;
  uint32_t conv_state_t, channels, width, silu;
  uint32_t cq, ck, cv;        // the channels of element 0 of q, k and v head 0
};

constexpr uint32_t kLayerMaxWidth = 4;

// The decode layer's recurrence on the recurrent kernel's quarter workgroups (sequence b, value head h, 32 value
// columns), with the convolution folded in: per token the workgroup convolves the 288 channels it reads (the key head's
// 128 q and 128 k channels and its 32 v channels; CausalConv1d's arithmetic: bias, then the taps oldest first with
// fmaf, SiLU, rounded to bf16) into LDS, then runs RecurrentStep<4> (the recurrent kernel's arithmetic) and writes its
// 32 output columns as the GDN op rounds them. Sequences sharing a state slot run in batch order, carried by the first one's workgroup, as in RecurrentUnit.
// Every workgroup reads the old convolution state (the four ops' convolution reads it before its state kernel runs), so
// the state update and the gated norm run afterwards as their own launches. kW is the convolution's width and CS its
// state's element type (uint16_t: bf16, or float).
//
// A workgroup lives for a few memory round trips, so the first token's operands (taps, weights, bias, gate inputs,
// the slot-table entries of the sharing scan) are all requested before the state, without a use of any of them in
// between: the memory counter retires in order, so waiting for one of them then leaves the state's loads in flight.
template <int kW, typename CS>
__global__ void __launch_bounds__(kRecThreads) ConvRecurrentKernel(LayerArgs L) {
  const GdnArgs& a = L.a;
  constexpr int kSl = kW - 1;                 // state taps
  constexpr int kSt = kSl > 0 ? kSl : 1;
  constexpr int kChans = 2 * kDim + 32;       // channels a workgroup convolves
  constexpr bool kBf16State = sizeof(CS) == 2;
  __shared__ float red_sk[4][32], red_o[4][32];
  __shared__ __align__(16) uint16_t xin[kChans];  // this token's q, k and v columns, as the convolution rounds them
  __shared__ uint32_t chain_flags;  // bit 0: an earlier sequence shares the slot; bit 1: a later one does
  const uint32_t b = blockIdx.x, h = blockIdx.y / kRecQuarters, quarter = blockIdx.y % kRecQuarters;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int rg = lane & 7, cg = lane >> 3;
  const int row0 = 32 * w + 4 * rg;
  const uint32_t col = 32 * quarter + 4 * cg;
  const uint32_t kh = h / a.group;
  int32_t t0 = a.cu[b];
  int32_t t1 = a.cu[b + 1];
  if (t1 <= t0) return;  // an empty sequence leaves its slots untouched
  const int32_t slot = a.slots[b];
  const bool has_slot = slot >= 0 && static_cast<uint64_t>(slot) < a.pool_slots;
  const int32_t cslot0 = L.conv_slots[b];
  const GateRaw graw0 = GateRequestByType(a, static_cast<uint64_t>(t0), h);
  // Channel j of the token: q element j (j < 128), k element j - 128 (j < 256), v column 32 quarter + j - 256; thread
  // tid convolves channel tid and, for tid < 32, channel 256 + tid (the other threads' second channel repeats their
  // first, so that every request is in bounds; its result is not stored).
  uint32_t cc[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int j = tid < 32 ? tid + 256 * u : tid;
    cc[u] = j < static_cast<int>(kDim)      ? L.cq + kh * kDim + j
            : j < 2 * static_cast<int>(kDim) ? L.ck + kh * kDim + (j - kDim)
                                             : L.cv + h * kDim + 32 * quarter + (j - 2 * kDim);
  }
  // The first token's taps (entry k of [state, sequence] for k < kW: the state's kSl entries, then the token itself).
  const bool cslot0_ok = cslot0 >= 0 && static_cast<uint64_t>(cslot0) < L.conv_pool_slots;
  // Absent operands (no bias, a slot outside the pool) are read from kZeroTaps, so that no request sits in a branch.
  uint16_t rw[2][kW], rb[2], rx[2];
  CS rs[2][kSt];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
#pragma unroll
    for (int k = 0; k < kW; ++k) rw[u][k] = L.conv_w[static_cast<uint64_t>(cc[u]) * kW + k];
    rb[u] = *(L.conv_b != nullptr ? L.conv_b + cc[u] : reinterpret_cast<const uint16_t*>(kZeroTaps));
    const CS* st = cslot0_ok ? static_cast<const CS*>(L.conv_state) +
                                   (static_cast<uint64_t>(cslot0) * L.channels + cc[u]) * kSl
                             : reinterpret_cast<const CS*>(kZeroTaps);
#pragma unroll
    for (int k = 0; k < kSl; ++k) rs[u][k] = st[k];
    rx[u] = L.x[static_cast<uint64_t>(t0) * L.channels + cc[u]];
  }
  constexpr int kScanNow = 2;  // slot entries per lane requested up front (128 sequences)
  int32_t sj[kScanNow];
#pragma unroll
  for (int i = 0; i < kScanNow; ++i) sj[i] = a.slots[min(static_cast<uint32_t>(lane + 64 * i), a.batch - 1)];
  float s[4][4];
  float* sp = has_slot ? a.state + (static_cast<uint64_t>(slot) * a.vh + h) * kDim * kDim + col : nullptr;
  // Behind a branch here (zeros on the other path): 0.0611 against 0.0631 ms for the request from kZeroTaps that
  // RecurrentUnit makes.
  if (has_slot && a.use_initial_state) {
    LoadStateRows<4>(true, sp, row0, s);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int c = 0; c < 4; ++c) s[i][c] = 0.0f;
  }
  auto state_tap = [&](CS v) { return kBf16State ? Bf16ToF32(static_cast<uint16_t>(v)) : static_cast<float>(v); };
  bool scan_pending = has_slot, chained = false, first = true;
  uint32_t cur = b;  // the sequence whose tokens run now (later members of a chain follow in turn)
  int32_t cur_t0 = t0;
  for (int32_t tok = t0;;) {
    if (first) {  // from the requests above
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        float acc = Bf16ToF32(rb[u]);
#pragma unroll
        for (int k = 0; k < kSl; ++k) acc = fmaf(Bf16ToF32(rw[u][k]), state_tap(rs[u][k]), acc);
        acc = fmaf(Bf16ToF32(rw[u][kSl]), Bf16ToF32(rx[u]), acc);
        if (u == 0 || tid < 32) xin[tid + 256 * u] = F32ToBf16(L.silu ? SiluF(acc) : acc);
      }
    } else {  // a later token, or a later sequence of a chain: entry rel + k of [state, sequence] is tap k (the
              // weights and bias read again rather than held in registers through the step)
      const int32_t rel = tok - cur_t0;
      const int32_t cslot = L.conv_slots[cur];
      const bool cslot_ok = cslot >= 0 && static_cast<uint64_t>(cslot) < L.conv_pool_slots;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        float acc = L.conv_b != nullptr ? Bf16ToF32(L.conv_b[cc[u]]) : 0.0f;
#pragma unroll
        for (int k = 0; k < kW; ++k) {
          const int32_t hi = rel + k;
          float tap;
          if (hi < kSl) {
            tap = cslot_ok ? state_tap(static_cast<const CS*>(L.conv_state)[(static_cast<uint64_t>(cslot) * L.channels +
                                                                              cc[u]) * kSl + hi])
                           : 0.0f;
          } else {
            tap = Bf16ToF32(L.x[static_cast<uint64_t>(cur_t0 + hi - kSl) * L.channels + cc[u]]);
          }
          acc = fmaf(Bf16ToF32(L.conv_w[static_cast<uint64_t>(cc[u]) * kW + k]), tap, acc);
        }
        if (u == 0 || tid < 32) xin[tid + 256 * u] = F32ToBf16(L.silu ? SiluF(acc) : acc);
      }
    }
    if (scan_pending && w == 0) {  // sequences sharing this one's slot (RecurrentUnit's rule), once
      bool earlier = false, later = false;
#pragma unroll
      for (int i = 0; i < kScanNow; ++i) {
        const uint32_t jj = static_cast<uint32_t>(lane + 64 * i);
        if (jj < a.batch && jj != b && sj[i] == slot && ChainMember(a, jj, slot)) {
          earlier |= jj < b;
          later |= jj > b;
        }
      }
      for (uint32_t jj = static_cast<uint32_t>(lane + 64 * kScanNow); jj < a.batch; jj += 64) {
        if (jj != b && ChainMember(a, jj, slot)) {
          earlier |= jj < b;
          later |= jj > b;
        }
      }
      const uint32_t f = (__any(earlier) ? 1u : 0u) | (__any(later) ? 2u : 0u);
      if (lane == 0) chain_flags = f;
    }
    __syncthreads();
    if (scan_pending) {
      scan_pending = false;
      const uint32_t f = chain_flags;
      if (f & 1u) return;  // nothing written yet; every wavefront of the workgroup leaves here
      chained = (f & 2u) != 0;
    }
    const uint16_t* qv = xin;
    const uint16_t* kv = xin + kDim;
    float q2[2], k2[2], q4[4], k4[4], vv[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      q2[i] = Bf16ToF32(qv[2 * lane + i]);
      k2[i] = Bf16ToF32(kv[2 * lane + i]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      q4[i] = Bf16ToF32(qv[row0 + i]);
      k4[i] = Bf16ToF32(kv[row0 + i]);
      vv[i] = Bf16ToF32(xin[2 * kDim + 4 * cg + i]);
    }
    const GateIn gin = first ? GateWidenByType(a, graw0) : GateLoad(a, static_cast<uint64_t>(tok), h);
    first = false;
    float graw, beta;
    GateFrom(a, gin, graw, beta);
    float ot[4];
    RecurrentStep<4>(s, q2, k2, q4, k4, vv, graw, beta, a.scale, w, rg, cg, red_sk, red_o, ot);
    if (w == 0 && rg == 0) {
      uint2 pw;
      pw.x = PackBf16(ot[0], ot[1]);
      pw.y = PackBf16(ot[2], ot[3]);
      *reinterpret_cast<uint2*>(a.out + (static_cast<uint64_t>(tok) * a.vh + h) * kDim + col) = pw;
    }
    if (++tok < t1) continue;
    if (!chained) break;
    uint32_t next = cur + 1;
    while (next < a.batch && !ChainMember(a, next, slot)) ++next;
    if (next >= a.batch) break;
    cur = next;
    cur_t0 = tok = a.cu[cur];
    t1 = a.cu[cur + 1];
    if (!a.use_initial_state) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) s[i][c] = 0.f;
    }
  }
  if (has_slot) StoreStateRows<4>(sp, row0, s);
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
constexpr int kVBlock = 32;      // value columns per scan workgroup
constexpr uint32_t kVBlocks = kDim / kVBlock;

struct ChunkArgs {
  GdnArgs a;
  const int4* chunks;  // [chunks] (sequence, first token, tokens, 0)
  const int4* seqs;    // [batch] (first chunk, chunk count, first token, end token)
  uint8_t* recs;       // [chunks][heads] records
  const int32_t* seq_list;  // when set: chain c runs sequence seq_list[c / heads] (-1: none)
  uint32_t chains;     // batch * heads, or (length of seq_list) * heads
  // When set (the recurrent variant's routed calls of at most kFoldBatch sequences), the prep launch routes itself:
  // each workgroup finds its chunk from cu_seqlens, and workgroup (0, 0) writes the sequence table and the list of
  // routed sequences (fold_seqs, fold_list) that the scan reads; no chunk table is used.
  const int32_t* fold_cu;
  int4* fold_seqs;
  int32_t* fold_list;
  uint32_t fold_batch, fold_max_chunks, fold_max_long;
  uint32_t prep_x;  // WyPrepRecurrentKernel: workgroup columns that prep chunks (the rest run recurrent sequences)
};

constexpr uint32_t kFoldBatch = 1024;  // sequences one prep workgroup routes (4 per thread)

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

constexpr float kLog2e = 1.4426950408889634f;
// 2^x on the hardware's v_exp_f32 (about 1 ulp; results below 2^-126 flush to zero, which only ever multiplies
// factors that are already negligible).
__device__ __forceinline__ float Exp2(float x) { return __builtin_amdgcn_exp2f(x); }

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
// s_waitcnt vmcnt(0) alone (expcnt and lgkmcnt fields at their maxima).
__device__ __forceinline__ void WaitVmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

__device__ __forceinline__ float F4(const float4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// ---- Chunk variant: operand records and the WY scan ----------------------------------------------------------------
//
// WyPrepKernel (one workgroup per chunk and head, all in parallel) turns a chunk's raw rows into one 20 KB record of
// ready-made MFMA operands: T = (I + A)^-1 split into bf16 hi and lo parts, P, and the per-token factors. WyScanKernel
// (one workgroup per sequence, head and 32-column value block: two compute and two copier wavefronts) walks the chunks
// in order with the state in registers: per chunk the copiers bring the record and the raw k, q and v rows into LDS
// (global_load_lds, one chunk ahead), and each compute wavefront advances its 16 state columns with no exchange between
// wavefronts.
//
// Operand layouts (v_mfma_f32_16x16x32_bf16: A lane l = row l%16, k-slots 8(l/16)..+7; B lane l = column l%16, same
// k-slots; C lane l = column l%16, rows 4(l/16)+i). A product's C tiles feed the next product's B operand without any
// exchange by ordering its k-slots to match: slot 8g + 4h + i of k-step s stands for row 32s + 16h + 4g + i of the C
// tiles 2s (h = 0) and 2s + 1 (h = 1). The state S [128 x 16] lives in eight C tiles m = 2s + h whose row 4g + i is
// state row 32s + 8g + 4h + i, so that the k-slots of S's B operand are 8 consecutive state rows and the k rows of
// X = k S are plain 16-byte LDS reads; the transposed k operand of the state update is read with ds_read_b64_tr_b16 in
// the same row order.

namespace wy {

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kPairs = 6;                 // (token tile r, k-step s') on and below the diagonal: s' <= r / 2
constexpr int kRecTHi = 0;                // [pair][64 lanes] uint4: T hi operands
constexpr int kRecTLo = kPairs * 1024;    // T lo operands
constexpr int kRecP = 2 * kPairs * 1024;  // P operands
constexpr int kRecScal = 3 * kPairs * 1024;  // float [4][64] xs, beta, os, ws; then the chunk's decay
constexpr int kRecBytes = 20 * 1024;      // 19.25 KB used, copied as 20 1 KB blocks
__host__ __device__ constexpr int Pair(int r, int sp) { return r < 2 ? r : 2 * r - 2 + sp; }

// 16-byte piece c (0..15) of row r of a 256-byte-row tile sits at piece c ^ Hsw(r): the 16 rows of a row tile then
// spread a same-piece read over all banks, and so do the transposed reads (4 rows x 4 pieces).
__device__ __forceinline__ int Hsw(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }
__device__ __forceinline__ int T16(int r, int c) { return r * 256 + 16 * (c ^ Hsw(r)); }

// 16-byte piece c (0..3) of row r of a 64-byte-row tile (the v block and the output block) sits at piece c ^ ((r / 4) %
// 4): rows r, r + 4, r + 8 and r + 12, which start on the same bank, then spread the transposed v reads and the 8-byte
// output writes over all banks.
__host__ __device__ __forceinline__ uint32_t VSw(uint32_t r, uint32_t c) { return c ^ ((r >> 2) & 3); }

template <typename T>
__device__ __forceinline__ T Lds(const uint8_t* base, int off) {
  return *reinterpret_cast<const T*>(base + off);
}

__device__ __forceinline__ u32x2_t TrRead(const uint8_t* p) {
  typedef short i16x4_t __attribute__((ext_vector_type(4)));
  auto* ptr = reinterpret_cast<__attribute__((address_space(3))) i16x4_t*>(
      const_cast<__attribute__((address_space(3))) char*>((const __attribute__((address_space(3))) char*)p));
  return __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(ptr));
}

}  // namespace wy

// One workgroup per (chunk, head); wave w owns token tile w (tokens 16w .. 16w + 15) of the 64 x 64 products. The
// arithmetic is the prep of the WY form: k.k^T and k.q^T on bf16 MFMA from the raw rows (exact products; the norms are
// applied afterwards in fp32), T by blocked substitution in fp32 (16 x 16 diagonal blocks by forward substitution, the
// blocks below on v_mfma_f32_16x16x4f32).
// RouteKernel's rule for one chunk, computed by the prep workgroup that preps it: sequences of kRouteMinTokens or more
// tokens get ceil(len / 64) chunks, numbered in sequence order, as long as they fit max_chunks. Returns chunk x's
// (sequence, first token, tokens), or tokens 0 past the routed chunks. The writer (workgroup (0, 0)) also writes the
// per-sequence table (first chunk, count, first token, end token) and the routed sequences' list, -1 past its end.
__device__ int4 FoldRoute(const ChunkArgs& ca, uint32_t x, bool writer) {
  __shared__ uint32_t wave_cnt[4], wave_long[4];
  __shared__ int4 found;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const uint32_t batch = ca.fold_batch;
  int32_t t0[4], t1[4];
  uint32_t cnt[4], mine = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t b = 4 * tid + i;
    t0[i] = b < batch ? ca.fold_cu[b] : 0;
    t1[i] = b < batch ? ca.fold_cu[b + 1] : 0;
    const int32_t len = t1[i] - t0[i];
    cnt[i] = len >= static_cast<int32_t>(kRouteMinTokens) ? (static_cast<uint32_t>(len) + kChunk - 1) / kChunk : 0;
    mine += cnt[i];
  }
  // Exclusive prefix of the chunk counts over the threads (sequence order is thread order, then i).
  uint32_t incl = mine;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  if (lane == 63) wave_cnt[w] = incl;
  if (tid == 0) found = make_int4(0, 0, 0, 0);
  __syncthreads();
  uint64_t first = incl - mine;
  for (int i = 0; i < w; ++i) first += wave_cnt[i];
  bool routed[4];
  uint32_t mine_long = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    routed[i] = cnt[i] != 0 && first + cnt[i] <= ca.fold_max_chunks;
    if (routed[i] && x >= first && x < first + cnt[i]) {
      const int32_t c0 = t0[i] + static_cast<int32_t>(kChunk * (x - first));
      found = make_int4(static_cast<int32_t>(4 * tid + i), c0, min(static_cast<int32_t>(kChunk), t1[i] - c0), 0);
    }
    mine_long += routed[i] ? 1u : 0u;
    first += cnt[i];
  }
  if (writer) {  // the scan's tables: a second prefix over the routed sequences gives each its place in the list
    uint32_t lincl = mine_long;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t y = __shfl_up(lincl, o);
      if (lane >= o) lincl += y;
    }
    if (lane == 63) wave_long[w] = lincl;
    __syncthreads();
    uint32_t li = lincl - mine_long, total_long = 0;
    for (int i = 0; i < 4; ++i) {
      li += i < w ? wave_long[i] : 0;
      total_long += wave_long[i];
    }
    uint64_t f = first;
#pragma unroll
    for (int i = 3; i >= 0; --i) f -= cnt[i];  // back to this thread's first chunk
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t b = 4 * tid + i;
      if (b < batch) {
        ca.fold_seqs[b] = routed[i] ? make_int4(static_cast<int32_t>(f), static_cast<int32_t>(cnt[i]), t0[i], t1[i])
                                    : make_int4(0, 0, t0[i], t1[i]);
        if (routed[i] && li < ca.fold_max_long) ca.fold_list[li] = static_cast<int32_t>(b);
      }
      li += routed[i] ? 1u : 0u;
      f += cnt[i];
    }
    for (uint32_t i = total_long + tid; i < ca.fold_max_long; i += 256) ca.fold_list[i] = -1;
  }
  __syncthreads();
  return found;
}

template <bool kVec>
__device__ __forceinline__ void WyPrepChunk(const ChunkArgs& ca, uint32_t x, uint32_t h) {
  using namespace wy;
  const GdnArgs& a = ca.a;
  const int4 ch = ca.fold_cu != nullptr ? FoldRoute(ca, x, x == 0 && h == 0) : ca.chunks[x];
  const int t0 = ch.y, n = ch.z;
  if (n <= 0) return;  // an unused entry of a table sized for the worst case
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, kq = lane >> 4;
  const uint32_t kh = h / a.group;
  uint8_t* rec = ca.recs + (static_cast<uint64_t>(x) * a.vh + h) * kRecBytes;

  // region0 holds the raw k rows (a [64][kTilePitch] bf16 tile; each wavefront keeps its own 16 q rows in registers).
  // Once the products are formed it holds A and T (fp32) as their 10 lower-triangular 16 x 16 blocks each, and one
  // 16 x 16 block of partial sums per wavefront: 24 KB in all, so that 6 workgroups share a CU.
  constexpr int kBlk = 256;  // floats per 16 x 16 block
  __shared__ __align__(16) uint8_t region0[(2 * 10 + 4) * kBlk * 4];
  static_assert(sizeof(region0) >= 64 * kTilePitch * 2, "the k tile fits the region");
  __shared__ float g_lds[64], rk_lds[64], rq_lds[64], b_lds[64];
  auto kt = reinterpret_cast<uint16_t(*)[kTilePitch]>(region0);
  float* const a_mem = reinterpret_cast<float*>(region0);
  float* const t_mem = a_mem + 10 * kBlk;
  float* const p_mem = t_mem + 10 * kBlk;
  // Element (r, c) of a block sits at 16 (r % 16) + ((c % 16) ^ 4 ((r % 16) / 4)): the MFMA operand reads (16 rows x 4
  // columns, or 4 rows x 16 columns, per instruction) fall on 64 distinct banks, and column pairs (2c, 2c + 1) stay
  // adjacent. Block (bi, bj), bj <= bi, is block bi (bi + 1) / 2 + bj of its matrix.
  auto in_blk = [](int r, int c) { return (r & 15) * 16 + ((c & 15) ^ (4 * ((r & 15) >> 2))); };
  auto tri = [](int r, int c) { return ((r >> 4) * ((r >> 4) + 1) / 2 + (c >> 4)) * kBlk; };
  auto a_lds = [=](int r, int c) -> float& { return a_mem[tri(r, c) + in_blk(r, c)]; };
  auto t_lds = [=](int r, int c) -> float& { return t_mem[tri(r, c) + in_blk(r, c)]; };
  auto p_lds = [=](int r, int c) -> float& { return p_mem[w * kBlk + in_blk(r, c)]; };  // this wavefront's block

  // Q operands of this wavefront's token tile: bq[s] = q[16w + r16][32s + 8kq .. +8], zero past the chunk's end.
  uint4 bq[4];
  {  // Raw k rows into LDS, q rows into registers (zero past the chunk's end), and their sums of squares. Every load
     // is issued unconditionally from a clamped row and masked afterwards, so that all of them are in flight together.
    const int row = tid >> 2, part = tid & 3;
    const uint32_t keep = row < n ? ~0u : 0u;
    const uint64_t tok = static_cast<uint64_t>(t0 + min(row, n - 1));
    const uint16_t* kp = a.k + tok * a.k_stride + kh * kDim + part * 32;
    const int qrow = 16 * w + r16;
    const uint32_t qkeep = qrow < n ? ~0u : 0u;
    const uint16_t* qp = a.q + static_cast<uint64_t>(t0 + min(qrow, n - 1)) * a.q_stride + kh * kDim + 8 * kq;
    const GateRaw gr = GateRequest(a, static_cast<uint64_t>(t0 + min(lane, n - 1)), h);  // in flight with the rows
    uint4 kv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kv[i] = Load8<kVec>(kp + 8 * i);
      bq[i] = Load8<kVec>(qp + 32 * i);
    }
    float graw, braw;
    GateFrom(a, GateWiden(a, gr), graw, braw);
    float kk = 0.0f, qq = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kv[i] = make_uint4(kv[i].x & keep, kv[i].y & keep, kv[i].z & keep, kv[i].w & keep);
      bq[i] = make_uint4(bq[i].x & qkeep, bq[i].y & qkeep, bq[i].z & qkeep, bq[i].w & qkeep);
      kk += SumSq8(kv[i]);
      qq += SumSq8(bq[i]);
      *reinterpret_cast<uint4*>(&kt[row][part * 32 + 8 * i]) = kv[i];
    }
    kk = QuadSum(kk);
    qq += __shfl_xor(qq, 16, 64);  // the 4 lanes r16 + 16kq hold disjoint quarters of q row 16w + r16
    qq += __shfl_xor(qq, 32, 64);
    if (part == 0) rk_lds[row] = 1.0f / sqrtf(kk + 1e-6f);
    if (kq == 0) rq_lds[qrow] = a.scale / sqrtf(qq + 1e-6f);
    if (w == 0) {  // cumulative log-decay (zero increments past the end) and beta
      float gv = lane < n ? graw : 0.0f;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const float y = __shfl_up(gv, d, 64);
        if (lane >= d) gv += y;
      }
      g_lds[lane] = gv * kLog2e;  // cumulative log-decay in log2 units: every factor below is one exp2
      b_lds[lane] = lane < n ? braw : 0.0f;
    }
  }
  __syncthreads();

  // kk4[c] = k.k^T at rows 16w.., columns 16c..; pt4[c] = k.q^T at rows 16c.. (key tokens j), columns 16w.. (query
  // tokens t), i.e. P^T, whose result lanes hold four consecutive j of one t. A row-major 16 x 32 tile supplies the A and
  // the B operand in the same lane layout, so the k rows of tile c serve as both.
  f32x4_t kk4[4], pt4[4];
  {
    uint4 ak[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) ak[s] = *reinterpret_cast<const uint4*>(&kt[16 * w + r16][32 * s + 8 * kq]);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      kk4[c] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      pt4[c] = kk4[c];
      if (c <= w) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const uint4 kc = *reinterpret_cast<const uint4*>(&kt[16 * c + r16][32 * s + 8 * kq]);
          kk4[c] = Mfma(ak[s], kc, kk4[c]);
          pt4[c] = Mfma(kc, bq[s], pt4[c]);
        }
      }
    }
  }
  __syncthreads();  // the k tile is dead: region0 becomes A and T

  // P operands of wave w's token tile: lane (kq, r16) holds P[t = 16w + r16][j = 16c + 4kq + i] in pt4[c], which is
  // exactly its share of the operand of pair (w, s') for c = 2s' (slots 8kq..8kq+3) and c = 2s' + 1 (slots +4..+7).
  {
    float pv[4][4];
    const int t = 16 * w + r16;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = 16 * c + 4 * kq + i;
        pv[c][i] = (c <= w && j <= t) ? pt4[c][i] * rq_lds[t] * rk_lds[j] * Exp2(g_lds[t] - g_lds[j]) : 0.0f;
      }
#pragma unroll
    for (int sp = 0; sp < 2; ++sp) {
      if (sp <= w / 2) {
        const uint4 op = make_uint4(PackRne(pv[2 * sp][0], pv[2 * sp][1]), PackRne(pv[2 * sp][2], pv[2 * sp][3]),
                                    PackRne(pv[2 * sp + 1][0], pv[2 * sp + 1][1]),
                                    PackRne(pv[2 * sp + 1][2], pv[2 * sp + 1][3]));
        *reinterpret_cast<uint4*>(rec + kRecP + Pair(w, sp) * 1024 + 16 * lane) = op;
      }
    }
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    if (c > w) continue;  // blocks above the diagonal are not stored
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // A[r][j], r = 16w + 4kq + i, j = 16c + r16 (strictly lower; zero above the diagonal of the diagonal block)
      const int r = 16 * w + 4 * kq + i, j = 16 * c + r16;
      float av = 0.0f;
      if (j < r) av = b_lds[r] * Exp2(g_lds[r] - g_lds[j]) * kk4[c][i] * rk_lds[r] * rk_lds[j];
      a_lds(r, j) = av;
    }
  }
  __syncthreads();

  // T = (I + A)^-1. Diagonal 16 x 16 blocks by forward substitution (wave w, one column per lane) ...
  if (lane < 16) {
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float acc = i == lane ? 1.0f : 0.0f;
#pragma unroll
      for (int j = 0; j < i; ++j) acc = fmaf(-a_lds(16 * w + i, 16 * w + j), x[j], acc);
      x[i] = acc;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) t_lds(16 * w + i, 16 * w + lane) = x[i];
  }
  __syncthreads();
  // ... then the blocks below it, T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj, in order of distance d = i - j from the
  // diagonal, one block per wave, on fp32 MFMA. The partial sum goes through the wavefront's own block of LDS.
#pragma unroll
  for (int d = 1; d < 4; ++d) {
    if (w < 4 - d) {
      const int j = w, i = w + d;
      f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int k = j; k < i; ++k) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          acc = MfmaF32(a_lds(16 * i + r16, 16 * k + 4 * kk + kq), t_lds(16 * k + 4 * kk + kq, 16 * j + r16), acc);
        }
      }
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) p_lds(4 * kq + ii, r16) = acc[ii];
      f32x4_t tij = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        tij = MfmaF32(t_lds(16 * i + r16, 16 * i + 4 * kk + kq), p_lds(4 * kk + kq, r16), tij);
      }
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) t_lds(16 * i + 4 * kq + ii, 16 * j + r16) = -tij[ii];
    }
    __syncthreads();
  }
  // T operands, hi and lo, of wave w's token tile: lane (kq, r16) holds T[16w + r16][32s' + 16hh + 4kq + i].
#pragma unroll
  for (int sp = 0; sp < 2; ++sp) {
    if (sp <= w / 2) {
      const int tr = 16 * w + r16, tc = 32 * sp + 4 * kq;
      // T is zero above its diagonal blocks, which are not stored.
      auto tv = [&](int c) { return (c >> 4) > w ? 0.0f : t_lds(tr, c); };
      uint4 hi, lo;
      Split2(tv(tc), tv(tc + 1), hi.x, lo.x);
      Split2(tv(tc + 2), tv(tc + 3), hi.y, lo.y);
      Split2(tv(tc + 16), tv(tc + 17), hi.z, lo.z);
      Split2(tv(tc + 18), tv(tc + 19), hi.w, lo.w);
      *reinterpret_cast<uint4*>(rec + kRecTHi + Pair(w, sp) * 1024 + 16 * lane) = hi;
      *reinterpret_cast<uint4*>(rec + kRecTLo + Pair(w, sp) * 1024 + 16 * lane) = lo;
    }
  }
  if (tid < 64) {
    float* sc = reinterpret_cast<float*>(rec + kRecScal);
    const float gt = g_lds[tid], gn = g_lds[63];
    const float e = Exp2(gt);
    sc[tid] = e * rk_lds[tid];
    sc[64 + tid] = b_lds[tid];
    sc[128 + tid] = rq_lds[tid] * e;
    sc[192 + tid] = tid < n ? Exp2(gn - gt) * rk_lds[tid] : 0.0f;
    if (tid == 0) sc[256] = Exp2(gn);
  }
}

template <bool kVec>
__global__ void __launch_bounds__(256, 6) WyPrepKernel(ChunkArgs ca) {
  WyPrepChunk<kVec>(ca, blockIdx.x, blockIdx.y);
}

// The recurrent variant's routed calls: the prep workgroups (the first prep_x x heads of a 1-D grid, every head of a
// chunk in turn) and, behind them, one workgroup per (sequence, value head, column quarter) for the recurrence of the
// sequences shorter than a.route_min. One launch instead of two streams: the recurrent work fills the CUs the prep
// leaves idle, and the scan that follows has the chip to itself. The prep workgroups come first in dispatch order, so
// that none of them waits behind recurrent ones for a slot.
template <bool kVec, bool kPreGate>
__global__ void __launch_bounds__(256, 6) WyPrepRecurrentKernel(ChunkArgs ca) {
  static_assert(kRecThreads == 256, "the prep and recurrent workgroups share one size");
  const uint32_t vh = ca.a.vh, i = blockIdx.x, preps = ca.prep_x * vh;
  if (i < preps) {
    WyPrepChunk<kVec>(ca, i / vh, i % vh);
  } else {
    const uint32_t j = i - preps, per_seq = vh * kRecQuarters;
    RecurrentUnit<kVec, false, kPreGate>(ca.a, j / per_seq, (j % per_seq) / kRecQuarters, j % kRecQuarters);
  }
}

namespace wy {

// One chunk's LDS stage: its record, the raw k and q rows (swizzled 16-byte pieces) and the v block.
struct Stage {
  uint8_t rec[kRecBytes];
  uint8_t kt[64 * 256];
  uint8_t qt[64 * 256];
  uint8_t vt[64 * 64];  // [64 tokens][32 columns] bf16
  uint8_t ob[64 * 64];  // the chunk's outputs [64 tokens][32 columns] bf16, written by the compute wavefronts
};

// Starts the copies of chunk (t0, n)'s record and rows into `st`; copier 0 copies the record and v, copier 1 k and q.
// Rows past the chunk's end repeat its last row (their factors are zero).
// global -> LDS copy with a wave-uniform 64-bit base in SGPRs and a 32-bit per-lane byte offset: lane l's 16 bytes land
// at lds + 16 l. M0 carries the LDS address and is restored.
__device__ __forceinline__ void DmaS(const void* sbase, uint32_t voff, uint32_t lds) {
  uint32_t save;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\tglobal_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
               : "=&s"(save) : "v"(voff), "s"(sbase), "s"(lds));
}

// The same copy with the non-temporal hint, for rows one workgroup alone reads (its v block): kept out of L2, they leave
// room there for the k, q and record lines the chain's four value-block workgroups share (config 4: 0.160 against
// 0.166 ms).
__device__ __forceinline__ void DmaSNt(const void* sbase, uint32_t voff, uint32_t lds) {
  uint32_t save;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\tglobal_load_lds_dwordx4 %1, %2 nt\n\ts_mov_b32 m0, %0"
               : "=&s"(save) : "v"(voff), "s"(sbase), "s"(lds));
}

__device__ __forceinline__ uint32_t Uniform(uint32_t x) { return __builtin_amdgcn_readfirstlane(x); }

// Per-lane byte offsets of a full chunk's copies, fixed for the whole scan. Instruction i of the k (or q) copy fills
// rows 4i .. 4i + 3: lane l takes row 4i + l / 16 and fetches the piece that lands at position l % 16, which is
// (l % 16) ^ Hsw(row) = (l % 16) ^ 4 (l / 16) ^ (i % 4); the row part 4i * stride is wave-uniform and goes into the base.
struct CopyOffsets {
  uint32_t k[4], q[4];  // by i % 4
  uint32_t v;           // v block: instruction i copies tokens 16i .. 16i + 15, 4 lanes x 16 bytes per token
  uint32_t rec;         // 16 bytes per lane of each 1 KB record block
};

__device__ __forceinline__ CopyOffsets MakeCopyOffsets(const GdnArgs& a, uint32_t h, uint32_t vb, int lane) {
  CopyOffsets o;
  const uint32_t rr = static_cast<uint32_t>(lane) >> 4, pos = static_cast<uint32_t>(lane) & 15;
#pragma unroll
  for (uint32_t j = 0; j < 4; ++j) {
    const uint32_t piece = pos ^ (rr << 2) ^ j;
    o.k[j] = static_cast<uint32_t>(rr * a.k_stride * 2) + (h / a.group) * 256 + 16 * piece;
    o.q[j] = static_cast<uint32_t>(rr * a.q_stride * 2) + (h / a.group) * 256 + 16 * piece;
  }
  o.v = static_cast<uint32_t>((static_cast<uint32_t>(lane) >> 2) * a.v_stride * 2) + h * 256 + vb * 64 +
        16 * VSw(static_cast<uint32_t>(lane) >> 2, static_cast<uint32_t>(lane) & 3);
  o.rec = 16 * static_cast<uint32_t>(lane);
  return o;
}

// Views that are not 16-byte aligned (kVec false) are read into registers and written to LDS instead; so are the rows
// of a chunk shorter than 64 tokens, whose rows past the end repeat its last row (their factors are zero).
template <bool kVec>
__device__ __forceinline__ void Copy16(const uint16_t* src, uint8_t* tile, uint32_t tile_lds, int block, int lane) {
  if constexpr (kVec) {
    Dma16(src, tile_lds + 1024 * block);
  } else {
    *reinterpret_cast<uint4*>(tile + 1024 * block + 16 * lane) = Load8<false>(src);
  }
}

// Copies chunk (t0, n)'s record and rows into `st`: copier 0 the record and the v block, copier 1 the k and q rows.
// `lds` is the LDS byte address of `st` (computed once, outside the loop, from the stage array).
template <bool kVec>
__device__ __forceinline__ void Fetch(const GdnArgs& a, const CopyOffsets& co, const uint8_t* recp, int t0, int n,
                                      uint32_t h, uint32_t vb, int copier, int lane, Stage& st, uint32_t lds) {
  const bool full = kVec && n == 64;
  const uint32_t l_rec = lds + offsetof(Stage, rec), l_kt = lds + offsetof(Stage, kt), l_qt = lds + offsetof(Stage, qt),
                 l_vt = lds + offsetof(Stage, vt);
  if (copier == 0) {
#pragma unroll
    for (int b = 0; b < kRecBytes / 1024; ++b) DmaS(recp + 1024 * b, co.rec, l_rec + 1024 * b);
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // 16 tokens of 4 x 16 bytes per instruction
      if (full) {
        const auto* vbase = reinterpret_cast<const uint8_t*>(a.v) + static_cast<uint64_t>(t0 + 16 * i) * a.v_stride * 2;
        DmaSNt(vbase, co.v, l_vt + 1024 * i);
      } else {
        const int row = 16 * i + (lane >> 2);
        const uint16_t* src = a.v + static_cast<uint64_t>(t0 + min(row, n - 1)) * a.v_stride + h * kDim + vb * 32 +
                              8 * VSw(row, lane & 3);
        Copy16<kVec>(src, st.vt, l_vt, i, lane);
      }
    }
  } else if (full) {
    const auto* kb = reinterpret_cast<const uint8_t*>(a.k) + static_cast<uint64_t>(t0) * a.k_stride * 2;
    const auto* qb = reinterpret_cast<const uint8_t*>(a.q) + static_cast<uint64_t>(t0) * a.q_stride * 2;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      DmaS(kb + 4ull * i * a.k_stride * 2, co.k[i & 3], l_kt + 1024 * i);
      DmaS(qb + 4ull * i * a.q_stride * 2, co.q[i & 3], l_qt + 1024 * i);
    }
  } else {
    const int rr = lane >> 4, pos = lane & 15;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = 4 * i + rr;
      const int piece = pos ^ Hsw(row);
      const uint64_t tok = static_cast<uint64_t>(t0 + min(row, n - 1));
      Copy16<kVec>(a.k + tok * a.k_stride + (h / a.group) * kDim + 8 * piece, st.kt, l_kt, i, lane);
      Copy16<kVec>(a.q + tok * a.q_stride + (h / a.group) * kDim + 8 * piece, st.qt, l_qt, i, lane);
    }
  }
}

// The workgroup barrier of the storer wavefront. `__syncthreads()` releases at workgroup scope, which waits for every
// global store of the wavefront to complete (`vmcnt(0)`): a store's round trip at every chunk. Nothing in the workgroup
// reads the outputs, so the storer only waits for its LDS reads (the block it read may be overwritten after the
// barrier); the empty asm's memory clobber keeps the compiler from moving memory operations across it.
__device__ __forceinline__ void BarrierAfterLdsReads() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left at their maxima
  asm volatile("s_barrier" ::: "memory");
}

// Writes a chunk's outputs from its LDS block to the output rows (the storer): 16 tokens of 4 x 16 bytes per
// instruction.
__device__ __forceinline__ void StoreOut(const GdnArgs& a, const Stage& st, int t0, int n, uint32_t h, uint32_t vb,
                                         int lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = 16 * i + (lane >> 2);
    const uint4 v = *reinterpret_cast<const uint4*>(st.ob + t * 64 + 16 * VSw(t, lane & 3));
    if (t < n) {  // non-temporal: the outputs are not read here again, and kept out of L2 they leave the chain's
                  // shared k, q and record lines there (config 4: 0.167 against 0.176 ms)
      typedef uint32_t u32x4_nt __attribute__((ext_vector_type(4)));
      __builtin_nontemporal_store(u32x4_nt{v.x, v.y, v.z, v.w},
                                  reinterpret_cast<u32x4_nt*>(a.out + (static_cast<uint64_t>(t0 + t) * a.vh + h) * kDim +
                                                              vb * 32 + 8 * (lane & 3)));
    }
  }
}

// One chunk of the scan for one wavefront's 16 state columns. With one wavefront per SIMD nothing hides an LDS read's
// latency but the wavefront's own work, so every phase keeps its operand reads a few multiplies ahead (register rings
// whose order sched_group_barrier pins) and loads the next phase's factors while the current one multiplies.
__device__ __forceinline__ void Advance(Stage& sg, f32x4_t (&st)[8], int w, int lane) {
  const int g = lane >> 4, m = lane & 15;
  const float* sc = reinterpret_cast<const float*>(sg.rec + kRecScal);
  // Per-lane LDS offsets of the k / q operand of (row tile r, k-step s): row 16r + m, piece 4s + g.
  auto kq_off = [&](int r, int s) { return T16(16 * r + m, 4 * s + g); };

  // (1) S as bf16 hi / lo B operands: k-step s covers state rows 32s .. 32s + 31.
  uint4 sh[4], sl[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    Split2(st[2 * s][0], st[2 * s][1], sh[s].x, sl[s].x);
    Split2(st[2 * s][2], st[2 * s][3], sh[s].y, sl[s].y);
    Split2(st[2 * s + 1][0], st[2 * s + 1][1], sh[s].z, sl[s].z);
    Split2(st[2 * s + 1][2], st[2 * s + 1][3], sh[s].w, sl[s].w);
  }
  // (2) X = k S as hi and lo partial sums and (q S)^T, token tile by token tile (r-major), so that (3) for tile r can
  // run while tile r + 1 multiplies; within a tile the three accumulators alternate. A ring keeps the k / q reads kRing
  // steps ahead.
  constexpr int kRing = 3;
  f32x4_t xh[4], xl[4], oq[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) xh[r] = xl[r] = oq[r] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  uint4 rk[kRing], rq[kRing];
#pragma unroll
  for (int j = 0; j < kRing; ++j) {
    rk[j] = Lds<uint4>(sg.kt, kq_off(j >> 2, j & 3));
    rq[j] = Lds<uint4>(sg.qt, kq_off(j >> 2, j & 3));
  }
  // The factors of phase (3), the v block and the T operands of phase (4), read while the multiplies run.
  float4 xf[4], bf[4];
  u32x2_t vr[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    xf[r] = *reinterpret_cast<const float4*>(sc + 16 * r + 4 * g);
    bf[r] = *reinterpret_cast<const float4*>(sc + 64 + 16 * r + 4 * g);
    vr[r] = TrRead(sg.vt + (16 * r + 4 * g + (m >> 2)) * 64 + 16 * VSw(16 * r + 4 * g + (m >> 2), 2 * w + ((m & 3) >> 1)) +
                   8 * (m & 1));
  }
  uint4 th[kPairs], tl[kPairs];
#pragma unroll
  for (int q = 0; q < kPairs; ++q) {
    th[q] = Lds<uint4>(sg.rec, kRecTHi + q * 1024 + 16 * lane);
    tl[q] = Lds<uint4>(sg.rec, kRecTLo + q * 1024 + 16 * lane);
  }
  // (3) Y = beta (v - e^G rk X) as hi / lo B operands of k-steps s' (tokens 32s' ..).
  uint4 yh[2], yl[2];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int r = j >> 2, s = j & 3;
    const uint4 ak = rk[j % kRing], aq = rq[j % kRing];
    if (j + kRing < 16) {
      rk[j % kRing] = Lds<uint4>(sg.kt, kq_off((j + kRing) >> 2, (j + kRing) & 3));
      rq[j % kRing] = Lds<uint4>(sg.qt, kq_off((j + kRing) >> 2, (j + kRing) & 3));
    }
    xh[r] = Mfma(ak, sh[s], xh[r]);
    xl[r] = Mfma(ak, sl[s], xl[r]);
    oq[r] = Mfma(sh[s], aq, oq[r]);  // (q S)^T: lane (g, m) gets columns 4g .. 4g + 3 of token 16r + m
    if (s == 3) {
      const float v4[4] = {Bf16LoToF32(vr[r][0]), Bf16HiToF32(vr[r][0]), Bf16LoToF32(vr[r][1]),
                           Bf16HiToF32(vr[r][1])};
      float y[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] = F4(bf[r], i) * (v4[i] - F4(xf[r], i) * (xh[r][i] + xl[r][i]));
      uint32_t* dh = reinterpret_cast<uint32_t*>(&yh[r >> 1]) + 2 * (r & 1);
      uint32_t* dl = reinterpret_cast<uint32_t*>(&yl[r >> 1]) + 2 * (r & 1);
      Split2(y[0], y[1], dh[0], dl[0]);
      Split2(y[2], y[3], dh[1], dl[1]);
    }
  }
  // Factors of phases (5) and (7); the output is transposed, so lane (g, m) scales token 16r + m.
  float4 wf[4];
  float of[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    wf[r] = *reinterpret_cast<const float4*>(sc + 192 + 16 * r + 4 * g);
    of[r] = sc[128 + 16 * r + m];
  }
  const float decay = sc[256];
  // (4) V = T Y on and below the diagonal (hi.hi + hi.lo + lo.hi), pairs in an order that alternates accumulators.
  f32x4_t vn[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) vn[r] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int term = 0; term < 3; ++term) {
#pragma unroll
    for (int q = 0; q < kPairs; ++q) {
      const int r = q < 2 ? q : 2 + (q - 2) / 2, sp = q < 2 ? 0 : (q - 2) % 2;
      const uint4 ta = term == 2 ? tl[q] : th[q];
      const uint4 yb = term == 1 ? yl[sp] : yh[sp];
      vn[r] = Mfma(ta, yb, vn[r]);
    }
  }
  // The transposed k operands of phase (6): tiles mt = 2s + hf, k-steps s' (two 8-byte reads each).
  const int e = m >> 2, q4 = m & 3;
  auto kt_op = [&](int mt, int sp) {
    const int s = mt >> 1, hf = mt & 1;
    const u32x2_t lo = TrRead(sg.kt + T16(32 * sp + 4 * g + e, 4 * s + q4) + 8 * hf);
    const u32x2_t hi = TrRead(sg.kt + T16(32 * sp + 16 + 4 * g + e, 4 * s + q4) + 8 * hf);
    return make_uint4(lo[0], lo[1], hi[0], hi[1]);
  };
  constexpr int kKtRing = 4;  // (mt, s') operands in flight
  uint4 kr[kKtRing];
#pragma unroll
  for (int j = 0; j < kKtRing; ++j) kr[j] = kt_op(j >> 1, j & 1);
  // (5) V as single bf16 operands for P V, and ws V as hi / lo for the state update.
  uint4 vb[2], wh[2], wl[2];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    uint32_t* db = reinterpret_cast<uint32_t*>(&vb[r >> 1]) + 2 * (r & 1);
    uint32_t* dh = reinterpret_cast<uint32_t*>(&wh[r >> 1]) + 2 * (r & 1);
    uint32_t* dl = reinterpret_cast<uint32_t*>(&wl[r >> 1]) + 2 * (r & 1);
    db[0] = PackRne(vn[r][0], vn[r][1]);
    db[1] = PackRne(vn[r][2], vn[r][3]);
    Split2(vn[r][0] * wf[r].x, vn[r][1] * wf[r].y, dh[0], dl[0]);
    Split2(vn[r][2] * wf[r].z, vn[r][3] * wf[r].w, dh[1], dl[1]);
  }
  // (6) S = e^Gn S + k^T (ws V), hi + lo, over (mt, s') with the transposed reads kKtRing operands ahead; two state
  // tiles are advanced side by side so that consecutive multiplies hit different accumulators.
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) st[mt] = st[mt] * decay;
#pragma unroll
  for (int pr = 0; pr < 4; ++pr) {  // state tiles 2pr and 2pr + 1
#pragma unroll
    for (int sp = 0; sp < 2; ++sp) {
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int mt = 2 * pr + hf, j = 4 * pr + 2 * hf + sp;  // operand index in (mt, s') order: j = 2 mt + s'
        const uint4 ak = kr[j % kKtRing];
        if (j + kKtRing < 16) kr[j % kKtRing] = kt_op((j + kKtRing) >> 1, (j + kKtRing) & 1);
        st[mt] = Mfma(ak, wh[sp], st[mt]);
        st[mt] = Mfma(ak, wl[sp], st[mt]);
      }
    }
  }
  // (7) o^T = rq e^G (q S0)^T + V^T P^T, rounded to bf16 (round to nearest even); written to the chunk's LDS output block.
  // The C layout of V is the A layout of V^T and P's A operand is the B layout of P^T, so the operands are the same
  // registers as P V's with their roles swapped; lane (g, m) ends up with 4 consecutive columns of token 16r + m.
  uint4 pa[kPairs];
#pragma unroll
  for (int q = 0; q < kPairs; ++q) pa[q] = Lds<uint4>(sg.rec, kRecP + q * 1024 + 16 * lane);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    f32x4_t o = oq[r] * of[r];
#pragma unroll
    for (int sp = 0; sp <= r / 2; ++sp) o = Mfma(vb[sp], pa[Pair(r, sp)], o);
    *reinterpret_cast<uint2*>(sg.ob + (16 * r + m) * 64 + 16 * VSw(16 * r + m, 2 * w + (g >> 1)) + 8 * (g & 1)) =
        make_uint2(PackRne(o[0], o[1]), PackRne(o[2], o[3]));
  }
}

}  // namespace wy

// One workgroup of five wavefronts per (sequence, head, value block of 32 columns): wavefronts 0 and 1 compute
// (columns 16w .. 16w + 15 of the block each) and never touch global memory inside the loop; wavefronts 2 and 3 copy
// the next chunk into LDS while they compute, so that the copies, which are bound by HBM, never hold the compute
// wavefronts at the memory pipeline; wavefront 4 stores the previous chunk's outputs. The storer passes its barriers
// without waiting for its stores: with the stores on a copier, the wait for them came back at every chunk
// (config 4: 0.176 ms against 0.165 with the storer and non-temporal stores). blockIdx -> (chain, block) keeps the four
// value blocks of a chain on one XCD (workgroups are dealt to the 8 XCDs round-robin): they share the chain's rows and
// records in L2.
template <bool kVec>
__global__ void __launch_bounds__(320, 1) WyScanKernel(ChunkArgs ca) {
  using namespace wy;
  const GdnArgs& a = ca.a;
  const uint32_t x = blockIdx.x;
  const uint32_t chain = (x & 7) + 8 * (x >> 5);
  const uint32_t vb = (x >> 3) & 3;
  if (chain >= ca.chains) return;
  const int32_t listed = ca.seq_list != nullptr ? ca.seq_list[chain / a.vh] : static_cast<int32_t>(chain / a.vh);
  if (listed < 0) return;
  const uint32_t seq = static_cast<uint32_t>(listed), h = chain % a.vh;
  const int4 sq = ca.seqs[seq];
  const int chunks = sq.y;
  if (chunks == 0) return;  // an empty (or unrouted) sequence leaves its slot untouched
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, m = lane & 15;
  __shared__ __align__(16) Stage stage[2];

  auto t0_of = [&](int c) { return sq.z + 64 * c; };
  auto n_of = [&](int c) { return min(64, sq.w - t0_of(c)); };
  auto rec_of = [&](int c) {
    return ca.recs + (static_cast<uint64_t>(sq.x + c) * a.vh + h) * kRecBytes;
  };

  const uint32_t lds0 = Uniform(LdsAddr(&stage[0]));  // LDS byte address of stage[0]; stage[1] follows it
  if (w == 4) {  // storer: the previous chunk's outputs, from LDS, while the next chunk is computed
    __syncthreads();
    for (int c = 0; c < chunks; ++c) {
      if (c > 0) StoreOut(a, stage[(c - 1) & 1], t0_of(c - 1), n_of(c - 1), h, vb, lane);
      BarrierAfterLdsReads();
    }
    StoreOut(a, stage[(chunks - 1) & 1], t0_of(chunks - 1), n_of(chunks - 1), h, vb, lane);
    return;
  }
  if (w >= 2) {  // copiers
    const int copier = w - 2;
    const CopyOffsets co = MakeCopyOffsets(a, h, vb, lane);
    Fetch<kVec>(a, co, rec_of(0), t0_of(0), n_of(0), h, vb, copier, lane, stage[0], lds0);
    WaitVmem();
    __syncthreads();
    for (int c = 0; c < chunks; ++c) {
      if (c + 1 < chunks) {
        const int nb = (c + 1) & 1;
        Fetch<kVec>(a, co, rec_of(c + 1), t0_of(c + 1), n_of(c + 1), h, vb, copier, lane, stage[nb],
                    lds0 + nb * static_cast<uint32_t>(sizeof(Stage)));
      }
      WaitVmem();
      __syncthreads();
    }
    return;
  }

  const int32_t slot = a.slots[seq];
  const bool has_slot = slot >= 0 && static_cast<uint64_t>(slot) < a.pool_slots;
  const uint32_t col = vb * 32 + 16 * w + m;
  float* sp = has_slot ? a.state + (static_cast<uint64_t>(slot) * a.vh + h) * kDim * kDim : nullptr;
  // st[mt][i] = S[32 (mt >> 1) + 8g + 4 (mt & 1) + i][col]
  f32x4_t st[8];
#pragma unroll
  for (int mt = 0; mt < 8; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = 32 * (mt >> 1) + 8 * g + 4 * (mt & 1) + i;
      st[mt][i] = (has_slot && a.use_initial_state) ? sp[d * kDim + col] : 0.0f;
    }
  __syncthreads();
  for (int c = 0; c < chunks; ++c) {
    Advance(stage[c & 1], st, w, lane);
    __syncthreads();
  }
  if (has_slot) {
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 32 * (mt >> 1) + 8 * g + 4 * (mt & 1) + i;
        sp[d * kDim + col] = st[mt][i];
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

ChunkArena MakeArena(uint64_t max_chunks, uint64_t batch, uint64_t heads, uint64_t max_long = 0) {
  ChunkArena l{};
  l.max_chunks = static_cast<uint32_t>(max_chunks);
  l.max_long = static_cast<uint32_t>(max_long);
  l.chunk_table = 0;
  l.seq_table = roost::RoundUp(16ull * l.max_chunks, 256);
  l.seq_list = l.seq_table + 16ull * batch;
  l.tables_bytes = roost::RoundUp(l.seq_list + 4ull * max_long, 256);
  l.records = l.tables_bytes;
  l.total = l.records + uint64_t{l.max_chunks} * heads * wy::kRecBytes;
  return l;
}

// Every sequence may be chunked (chunk variant): at most tokens / 64 + batch chunks.
ChunkArena MakeChunkArena(uint64_t tokens, uint64_t batch, uint64_t heads) {
  return MakeArena(tokens / kChunk + batch, batch, heads);
}

// Only sequences of kRouteMinTokens or more are chunked (recurrent variant): sum ceil(len / 64) over them is at most
// tokens / 64 plus their number, which is at most min(batch, tokens / kRouteMinTokens).
ChunkArena MakeRouteArena(uint64_t tokens, uint64_t batch, uint64_t heads) {
  const uint64_t max_long = std::min<uint64_t>(batch, tokens / kRouteMinTokens);
  return MakeArena(tokens / kChunk + max_long, batch, heads, max_long);
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

// with_recurrent: the prep launch also runs the recurrence of the sequences shorter than kRouteMinTokens.
RoostStatus LaunchChunk(const RoostGatedDeltaRuleParams& p, const RoostWorkspace* ws, const ChunkArena& l,
                        uint32_t chunks, hipStream_t stream, bool fold = false, bool with_recurrent = false,
                        const GateSource& gs = GateSource{}) {
  ChunkArgs ca{};
  ca.a = MakeArgs(p, gs);
  auto* base = static_cast<uint8_t*>(ws->device);
  ca.chunks = reinterpret_cast<const int4*>(base + l.chunk_table);
  ca.seqs = reinterpret_cast<const int4*>(base + l.seq_table);
  ca.recs = base + l.records;
  // The recurrent variant's calls list their chunked sequences; the chunk variant's chains are every sequence.
  ca.seq_list = l.max_long > 0 ? reinterpret_cast<const int32_t*>(base + l.seq_list) : nullptr;
  ca.chains = (l.max_long > 0 ? l.max_long : p.batch) * p.v_heads;
  if (fold) {
    ca.fold_cu = static_cast<const int32_t*>(p.cu_seqlens.address);
    ca.fold_seqs = reinterpret_cast<int4*>(base + l.seq_table);
    ca.fold_list = reinterpret_cast<int32_t*>(base + l.seq_list);
    ca.fold_batch = p.batch;
    ca.fold_max_chunks = l.max_chunks;
    ca.fold_max_long = l.max_long;
  }
  const dim3 prep(chunks, p.v_heads);
  const dim3 scan((ca.chains + 7) / 8 * 8 * kVBlocks);
  if (with_recurrent) {
    ca.a.route_min = static_cast<int32_t>(kRouteMinTokens);
    ca.prep_x = chunks;
    const dim3 both((chunks + p.batch * kRecQuarters) * p.v_heads);
    // The gate inputs are requested before the state when the launch computes the gates itself.
    const bool pre_gate = gs.a != nullptr;
    if (Vec16(p)) {
      auto* prep = pre_gate ? WyPrepRecurrentKernel<true, true> : WyPrepRecurrentKernel<true, false>;
      hipLaunchKernelGGL(prep, both, dim3(256), 0, stream, ca);
      hipLaunchKernelGGL(WyScanKernel<true>, scan, dim3(320), 0, stream, ca);
    } else {
      auto* prep = pre_gate ? WyPrepRecurrentKernel<false, true> : WyPrepRecurrentKernel<false, false>;
      hipLaunchKernelGGL(prep, both, dim3(256), 0, stream, ca);
      hipLaunchKernelGGL(WyScanKernel<false>, scan, dim3(320), 0, stream, ca);
    }
  } else if (Vec16(p)) {
    hipLaunchKernelGGL(WyPrepKernel<true>, prep, dim3(256), 0, stream, ca);
    hipLaunchKernelGGL(WyScanKernel<true>, scan, dim3(320), 0, stream, ca);
  } else {
    hipLaunchKernelGGL(WyPrepKernel<false>, prep, dim3(256), 0, stream, ca);
    hipLaunchKernelGGL(WyScanKernel<false>, scan, dim3(320), 0, stream, ca);
  }
  return roost::HipStatus(hipGetLastError(), kOp, "chunk launch");
}

// The recurrent variant's routed path over a device region laid out as `l`: the sequences of kRouteMinTokens or more
// tokens are cut into chunks (by the prep launch itself up to kFoldBatch sequences, else by RouteKernel from the device
// cu_seqlens), and the prep launch also runs the recurrence of the shorter ones in workgroups of its own, beside the
// prep workgroups: the chunks' chains leave most of the chip idle. The scan follows on the same stream. Short
// sequences that share a slot run in batch order (RecurrentUnit); a chunked sequence must have its slot to itself:
// otherwise the two race (they may run at the same time), as they do in the reference's gather / scatter of the slots.
RoostStatus LaunchRouted(const RoostGatedDeltaRuleParams& p, uint8_t* base, const ChunkArena& l, hipStream_t s,
                         const GateSource& gs = GateSource{}) {
  const bool fold = p.batch <= kFoldBatch;
  if (!fold) {
    hipLaunchKernelGGL(RouteKernel, dim3(1), dim3(1024), 0, s, static_cast<const int32_t*>(p.cu_seqlens.address),
                       p.batch, l.max_chunks, reinterpret_cast<int4*>(base + l.chunk_table),
                       reinterpret_cast<int4*>(base + l.seq_table), reinterpret_cast<int32_t*>(base + l.seq_list),
                       l.max_long);
    ROOST_RETURN_IF_FAILED(roost::HipStatus(hipGetLastError(), kOp, "route launch"));
  }
  RoostWorkspace ws{};
  ws.device = base;
  ws.device_bytes = l.total;
  return LaunchChunk(p, &ws, l, l.max_chunks, s, fold, /*with_recurrent=*/true, gs);
}

// The GatedDeltaRuleGates inputs of a call that folds the gates in, checked against the (admitted) GDN call.
RoostStatus GateSourceOf(const RoostGatedDeltaRuleGatesParams& gp, const RoostGatedDeltaRuleParams& p, GateSource* gs) {
  roost::Gate gate(kOp);
  gate.Expect(gp.tokens == p.tokens && gp.v_heads == p.v_heads, ROOST_STATUS_INVALID_ARGUMENT,
              "the gates cover %u tokens x %u heads; the call has %u x %u", gp.tokens, gp.v_heads, p.tokens, p.v_heads);
  ROOST_GATE_RETURN(gate);
  auto float_span = [&](const char* name, const RoostDeviceSpan& sp, uint64_t elements) {
    gate.Expect(sp.dtype == ROOST_DTYPE_BF16 || sp.dtype == ROOST_DTYPE_F32, ROOST_STATUS_UNSUPPORTED,
                "%s is %s; the gates read bf16 or f32", name, roost::Describe(sp.dtype).name);
    if (gate.ok()) gate.Tensor(name, sp, sp.dtype, elements).Aligned(name, sp.address, roost::ElementBytes(sp.dtype));
  };
  const uint64_t as = gp.a_stride == 0 ? gp.v_heads : gp.a_stride, bs = gp.b_stride == 0 ? gp.v_heads : gp.b_stride;
  gate.Expect(as >= gp.v_heads && bs >= gp.v_heads, ROOST_STATUS_INVALID_ARGUMENT,
              "a_stride %llu, b_stride %llu: rows hold %u heads", static_cast<unsigned long long>(as),
              static_cast<unsigned long long>(bs), gp.v_heads);
  const uint64_t t = gp.tokens;
  float_span("a", gp.a, t == 0 ? 0 : (t - 1) * as + gp.v_heads);
  float_span("b", gp.b, t == 0 ? 0 : (t - 1) * bs + gp.v_heads);
  float_span("a_log", gp.a_log, gp.v_heads);
  float_span("dt_bias", gp.dt_bias, gp.v_heads);
  ROOST_GATE_RETURN(gate);
  gs->a = gp.a.address;
  gs->b = gp.b.address;
  gs->a_log = gp.a_log.address;
  gs->dt_bias = gp.dt_bias.address;
  gs->a_t = gp.a.dtype;
  gs->b_t = gp.b.dtype;
  gs->alog_t = gp.a_log.dtype;
  gs->dtb_t = gp.dt_bias.dtype;
  gs->a_stride = as;
  gs->b_stride = bs;
  if (t > 0 && gs->a == nullptr) return roost::Report(ROOST_STATUS_INVALID_ARGUMENT, kOp, "a: address is NULL");
  return ROOST_STATUS_OK;
}

// The recurrent variant's run() over its admitted call, with g and beta read from the call or computed from gs.
RoostStatus RecurrentRun(const RoostGatedDeltaRuleParams& p, const RoostWorkspace* ws, hipStream_t s,
                         const GateSource& gs) {
  roost::Gate gate(kOp);
  if (p.batch == 0 || p.tokens == 0) return ROOST_STATUS_OK;
  if (p.tokens < kRouteMinTokens) return LaunchRecurrent(p, s, 0, gs);
  if (p.cu_seqlens_host != nullptr) {
    // The host copy says whether any sequence reaches kRouteMinTokens; if none does, the recurrent kernel runs every
    // sequence (so a graph captured from this call stays correct whatever lengths it is replayed with).
    bool any_long = false;
    for (uint32_t b = 0; b < p.batch && !any_long; ++b) {
      any_long = p.cu_seqlens_host[b + 1] - p.cu_seqlens_host[b] >= static_cast<int32_t>(kRouteMinTokens);
    }
    if (!any_long) return LaunchRecurrent(p, s, 0, gs);
  }
  // Every launch size below follows from tokens and batch alone, so the call can be captured into a graph.
  const ChunkArena l = MakeRouteArena(p.tokens, p.batch, p.v_heads);
  gate.Expect(roost::HasDeviceRegion(ws, l.total), ROOST_STATUS_WORKSPACE_TOO_SMALL,
              "%u tokens may route sequences to the chunk kernels, which need %llu device workspace bytes", p.tokens,
              static_cast<unsigned long long>(l.total));
  ROOST_GATE_RETURN(gate);
  return LaunchRouted(p, static_cast<uint8_t*>(ws->device), l, s, gs);
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
  sizes->device_bytes = p.tokens >= kRouteMinTokens ? MakeRouteArena(p.tokens, p.batch, p.v_heads).total : 0;
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
    return RecurrentRun(p, ws, roost::Stream(stream), GateSource{});
  });
}

extern "C" ROOST_API RoostStatus roost_amd_gdn_recurrent_gated_run(RoostContext* ctx, const void* params,
                                                                   const void* gates, const RoostWorkspace* ws,
                                                                   void* stream) {
  roost::Gate gate(kOp);
  gate.Expect(ctx != nullptr && params != nullptr && gates != nullptr, ROOST_STATUS_INVALID_ARGUMENT,
              "a context, the GDN params and the gates params are required");
  ROOST_GATE_RETURN(gate);
  ROOST_GATE_RETURN(gate.Header(gates, sizeof(RoostGatedDeltaRuleGatesParams)));
  const auto& p = *static_cast<const RoostGatedDeltaRuleParams*>(params);
  const auto& gp = *static_cast<const RoostGatedDeltaRuleGatesParams*>(gates);
  return roost::CatchAll(kOp, [&]() -> RoostStatus {
    ROOST_RETURN_IF_FAILED(Admit(p, false, /*fused_gates=*/true));
    GateSource gs;
    ROOST_RETURN_IF_FAILED(GateSourceOf(gp, p, &gs));
    return RecurrentRun(p, ws, roost::Stream(stream), gs);
  });
}

// CausalConv1d + GatedDeltaRuleGates + the recurrent GatedDeltaRule + GatedRmsNorm of one decode step in two launches
// (ConvRecurrentKernel, then the norm with the convolution's state update): the four ops' results bit for bit.
namespace {

// What the two layer calls (decode and chunk) read from their four params structs once admitted.
struct LayerViews {
  GateSource gs;
  uint32_t cq = 0, ck = 0, cv = 0;  // first channel of the q, k and v columns in the convolution's output rows
  bool row_form = false;            // the norm runs on GatedRmsNorm's single-pass bf16 form
  bool empty = false;               // no sequence has a token: nothing is read or written
};

// The layer calls' pointers and struct headers: a context and the conv, GDN and norm params are required; the gates
// params may be NULL (g and beta are then read from the GDN params).
RoostStatus LayerHeaders(const char* op, const RoostContext* ctx, const void* conv_params, const void* gates_params,
                         const void* gdn_params, const void* norm_params) {
  roost::Gate gate(op);
  gate.Expect(ctx != nullptr && conv_params != nullptr && gdn_params != nullptr && norm_params != nullptr,
              ROOST_STATUS_INVALID_ARGUMENT, "a context and the conv, GDN and norm params are required (the gates "
              "params may be NULL: g and beta are then read from the GDN params)");
  ROOST_GATE_RETURN(gate);
  gate.Header(conv_params, sizeof(RoostCausalConv1dParams))
      .Header(gdn_params, sizeof(RoostGatedDeltaRuleParams))
      .Header(norm_params, sizeof(RoostGatedRmsNormParams));
  if (gates_params != nullptr) gate.Header(gates_params, sizeof(RoostGatedDeltaRuleGatesParams));
  return gate.status();
}

// The rules the layer calls share: each op's own admission; the convolution over the GDN call's batch, bf16, at most
// kLayerMaxWidth taps, and q, k and v column views of its output (where the GDN op reads them); the norm over the GDN
// output's 128-column rows; and the norm's output apart from every input and state the layer reads.
RoostStatus AdmitLayer(const char* op, const RoostCausalConv1dParams& cp, const void* gates_params,
                       const RoostGatedDeltaRuleParams& p, const RoostGatedRmsNormParams& np, LayerViews* v) {
  roost::Gate gate(op);
  ROOST_RETURN_IF_FAILED(Admit(p, false, /*fused_gates=*/gates_params != nullptr));
  if (gates_params != nullptr) {
    ROOST_RETURN_IF_FAILED(GateSourceOf(*static_cast<const RoostGatedDeltaRuleGatesParams*>(gates_params), p, &v->gs));
  }
  ROOST_RETURN_IF_FAILED(roost_layer::AdmitConv(cp, op));
  ROOST_RETURN_IF_FAILED(roost_layer::AdmitNorm(np, op, &v->row_form));
  if (p.batch == 0 || p.tokens == 0) {  // nothing to read or write, as for the four ops
    v->empty = true;
    return ROOST_STATUS_OK;
  }
  const uint64_t ch = cp.channels;
  gate.Expect(cp.batch == p.batch && cp.tokens == p.tokens && cp.cu_seqlens.address == p.cu_seqlens.address,
              ROOST_STATUS_INVALID_ARGUMENT,
              "the convolution covers %u sequences / %u tokens (cu_seqlens %p); the GDN call %u / %u (%p)", cp.batch,
              cp.tokens, cp.cu_seqlens.address, p.batch, p.tokens, p.cu_seqlens.address)
      .Expect(cp.input.dtype == ROOST_DTYPE_BF16 && cp.width <= kLayerMaxWidth, ROOST_STATUS_UNSUPPORTED,
              "convolution of %s with %u taps: the layer calls are built for bf16 and up to %u taps",
              roost::Describe(cp.input.dtype).name, cp.width, kLayerMaxWidth);
  ROOST_GATE_RETURN(gate);
  auto view = [&](const char* name, const RoostDeviceSpan& sp, uint32_t stride, uint64_t heads, uint32_t* first) {
    const auto at = reinterpret_cast<intptr_t>(sp.address) - reinterpret_cast<intptr_t>(cp.output.address);
    const uint64_t width = heads * kDim;
    const bool ok = at >= 0 && at % 2 == 0 && static_cast<uint64_t>(at / 2) + width <= ch && Stride(stride, width) == ch;
    gate.Expect(ok, ROOST_STATUS_INVALID_ARGUMENT,
                "%s is not a column view of the convolution's output (offset %lld bytes, row stride %llu; rows of "
                "%llu channels)", name, static_cast<long long>(at),
                static_cast<unsigned long long>(Stride(stride, width)), static_cast<unsigned long long>(ch));
    *first = ok ? static_cast<uint32_t>(at / 2) : 0;
  };
  view("q", p.q, p.q_stride, p.k_heads, &v->cq);
  view("k", p.k, p.k_stride, p.k_heads, &v->ck);
  view("v", p.v, p.v_stride, p.v_heads, &v->cv);
  ROOST_GATE_RETURN(gate);
  gate.Expect(np.input.address == p.output.address && np.rows == uint64_t{p.tokens} * p.v_heads && np.dim == kDim,
              ROOST_STATUS_INVALID_ARGUMENT,
              "the norm reads %u rows x %u at %p; the GDN output is %llu rows x %u at %p", np.rows, np.dim,
              np.input.address, static_cast<unsigned long long>(uint64_t{p.tokens} * p.v_heads), kDim,
              p.output.address);
  ROOST_GATE_RETURN(gate);
  // What the kernels read may not be what they write: the norm's output against the layer's other inputs and states.
  auto range = [](const void* a, uint64_t bytes) {
    const auto x = reinterpret_cast<uintptr_t>(a);
    return std::pair<uintptr_t, uintptr_t>{x, x + bytes};
  };
  const auto out = range(np.output.address, np.rows * uint64_t{kDim} * 2);
  auto clear = [&](const char* name, const void* a, uint64_t bytes) {
    const auto r = range(a, bytes);
    gate.Expect(a == nullptr || bytes == 0 || r.second <= out.first || out.second <= r.first,
                ROOST_STATUS_INVALID_ARGUMENT, "the norm's output overlaps %s", name);
  };
  const uint64_t sl = cp.width - 1ull;
  clear("the convolution's input", cp.input.address, uint64_t{cp.tokens} * ch * 2);
  clear("the convolution's weights", cp.weight.address, ch * cp.width * 2);
  clear("the convolution's bias", cp.bias.address, ch * 2);
  clear("the convolution's state", sl == 0 ? nullptr : cp.conv_state.address,
        cp.conv_state.length * roost::ElementBytes(cp.conv_state.dtype == ROOST_DTYPE_UNDEFINED ? cp.input.dtype
                                                                                            : cp.conv_state.dtype));
  clear("the recurrent state", p.state.address, p.state.length * 4);
  ROOST_GATE_RETURN(gate);
  return ROOST_STATUS_OK;
}

// The decode layer's launch for an admitted call whose sequences are all shorter than kRouteMinTokens and whose norm
// is the single-pass bf16 form: ConvRecurrentKernel, then the norm and the convolution's state update.
RoostStatus LaunchDecodeLayer(const char* op, const RoostCausalConv1dParams& cp, const RoostGatedDeltaRuleParams& p,
                              const RoostGatedRmsNormParams& np, const LayerViews& lv, hipStream_t s) {
  const uint64_t sl = cp.width - 1ull;
  LayerArgs L{};
  L.cq = lv.cq;
  L.ck = lv.ck;
  L.cv = lv.cv;
  L.a = MakeArgs(p, lv.gs);
  L.x = static_cast<const uint16_t*>(cp.input.address);
  L.conv_w = static_cast<const uint16_t*>(cp.weight.address);
  L.conv_b = static_cast<const uint16_t*>(cp.bias.address);
  L.conv_state = cp.conv_state.address;
  L.conv_slots = static_cast<const int32_t*>(cp.state_slots.address);
  L.conv_state_t = cp.conv_state.dtype == ROOST_DTYPE_UNDEFINED ? cp.input.dtype : cp.conv_state.dtype;
  L.conv_pool_slots = sl == 0 ? 0 : cp.conv_state.length / (uint64_t{cp.channels} * sl);
  L.channels = cp.channels;
  L.width = cp.width;
  L.silu = cp.silu != 0 ? 1u : 0u;
  const dim3 grid(p.batch, p.v_heads * kRecQuarters);
  const bool bf16_state = L.conv_state_t == ROOST_DTYPE_BF16;
  switch (cp.width * 2 + (bf16_state ? 1 : 0)) {
    case 3: hipLaunchKernelGGL((ConvRecurrentKernel<1, uint16_t>), grid, dim3(kRecThreads), 0, s, L); break;
    case 2: hipLaunchKernelGGL((ConvRecurrentKernel<1, float>), grid, dim3(kRecThreads), 0, s, L); break;
    case 5: hipLaunchKernelGGL((ConvRecurrentKernel<2, uint16_t>), grid, dim3(kRecThreads), 0, s, L); break;
    case 4: hipLaunchKernelGGL((ConvRecurrentKernel<2, float>), grid, dim3(kRecThreads), 0, s, L); break;
    case 7: hipLaunchKernelGGL((ConvRecurrentKernel<3, uint16_t>), grid, dim3(kRecThreads), 0, s, L); break;
    case 6: hipLaunchKernelGGL((ConvRecurrentKernel<3, float>), grid, dim3(kRecThreads), 0, s, L); break;
    case 9: hipLaunchKernelGGL((ConvRecurrentKernel<4, uint16_t>), grid, dim3(kRecThreads), 0, s, L); break;
    default: hipLaunchKernelGGL((ConvRecurrentKernel<4, float>), grid, dim3(kRecThreads), 0, s, L); break;
  }
  ROOST_RETURN_IF_FAILED(roost::HipStatus(hipGetLastError(), op, "layer launch"));
  return roost_layer::RunNormAndConvState(np, cp, s, op);
}

}  // namespace

extern "C" ROOST_API RoostStatus roost_amd_gdn_decode_layer_run(RoostContext* ctx, const void* conv_params,
                                                                const void* gates_params, const void* gdn_params,
                                                                const void* norm_params, void* stream) {
  constexpr char kLayerOp[] = "gdn_decode_layer";
  roost::Gate gate(kLayerOp);
  ROOST_RETURN_IF_FAILED(LayerHeaders(kLayerOp, ctx, conv_params, gates_params, gdn_params, norm_params));
  const auto& cp = *static_cast<const RoostCausalConv1dParams*>(conv_params);
  const auto& p = *static_cast<const RoostGatedDeltaRuleParams*>(gdn_params);
  const auto& np = *static_cast<const RoostGatedRmsNormParams*>(norm_params);
  return roost::CatchAll(kLayerOp, [&]() -> RoostStatus {
    LayerViews lv;
    ROOST_RETURN_IF_FAILED(AdmitLayer(kLayerOp, cp, gates_params, p, np, &lv));
    if (lv.empty) return ROOST_STATUS_OK;
    // Every sequence on the token-serial recurrence: longer ones are the chunk kernels' in the recurrent variant.
    gate.Expect(p.cu_seqlens_host != nullptr, ROOST_STATUS_INVALID_ARGUMENT,
                "the decode layer checks the sequence lengths in cu_seqlens_host, which is NULL");
    ROOST_GATE_RETURN(gate);
    for (uint32_t b = 0; b < p.batch; ++b) {
      const int64_t n = int64_t{p.cu_seqlens_host[b + 1]} - p.cu_seqlens_host[b];
      gate.Expect(n < static_cast<int64_t>(kRouteMinTokens), ROOST_STATUS_UNSUPPORTED,
                  "sequence %u has %lld tokens; sequences of %u or more run on the chunk kernels, so this call covers "
                  "decode steps only (run the four ops one by one, or the chunk layer call)", b,
                  static_cast<long long>(n), kRouteMinTokens);
      if (!gate.ok()) return gate.status();
    }
    gate.Expect(np.rows == 0 || (np.input.dtype == ROOST_DTYPE_BF16 && lv.row_form), ROOST_STATUS_UNSUPPORTED,
                "the decode layer's norm is GatedRmsNorm's single-pass bf16 form: 16-byte aligned input, gate and "
                "output of bf16");
    ROOST_GATE_RETURN(gate);
    return LaunchDecodeLayer(kLayerOp, cp, p, np, lv, roost::Stream(stream));
  });
}

// One GDN layer over the recurrent variant for any step (no reference counterpart; the Qwen3.5 worker runs the four
// ops one after another, Qwen35EagerModel.cs:89-92, and names the recurrent variant for every length): a step whose
// sequences are all shorter than kRouteMinTokens, with the norm in its single-pass bf16 form, runs as the decode
// layer (ConvRecurrentKernel, then the norm and the convolution's state); any other step runs the conv op, the recurrent variant with the gates computed where
// they are read (its longer sequences on the chunk kernels, in `ws`), and the norm op. Either way the results equal
// the four ops'.
extern "C" ROOST_API RoostStatus roost_amd_gdn_layer_run(RoostContext* ctx, const void* conv_params,
                                                         const void* gates_params, const void* gdn_params,
                                                         const void* norm_params, const RoostWorkspace* ws,
                                                         void* stream) {
  constexpr char kLayerOp[] = "gdn_layer";
  ROOST_RETURN_IF_FAILED(LayerHeaders(kLayerOp, ctx, conv_params, gates_params, gdn_params, norm_params));
  const auto& cp = *static_cast<const RoostCausalConv1dParams*>(conv_params);
  const auto& p = *static_cast<const RoostGatedDeltaRuleParams*>(gdn_params);
  const auto& np = *static_cast<const RoostGatedRmsNormParams*>(norm_params);
  return roost::CatchAll(kLayerOp, [&]() -> RoostStatus {
    LayerViews lv;
    ROOST_RETURN_IF_FAILED(AdmitLayer(kLayerOp, cp, gates_params, p, np, &lv));
    if (lv.empty) return ROOST_STATUS_OK;
    // Short sequences only: known from the token count, or from the host copy of cu_seqlens.
    bool short_only = p.tokens < kRouteMinTokens;
    if (!short_only && p.cu_seqlens_host != nullptr) {
      short_only = true;
      for (uint32_t b = 0; b < p.batch && short_only; ++b) {
        short_only = p.cu_seqlens_host[b + 1] - p.cu_seqlens_host[b] < static_cast<int32_t>(kRouteMinTokens);
      }
    }
    hipStream_t s = roost::Stream(stream);
    if (short_only && np.input.dtype == ROOST_DTYPE_BF16 && lv.row_form) {
      return LaunchDecodeLayer(kLayerOp, cp, p, np, lv, s);
    }
    ROOST_RETURN_IF_FAILED(roost_causal_conv1d_run(ctx, conv_params, nullptr, stream));
    ROOST_RETURN_IF_FAILED(RecurrentRun(p, ws, s, lv.gs));
    return roost_gated_rms_norm_run(ctx, norm_params, nullptr, stream);
  });
}

// ---- Chunk entry points ---------------------------------------------------------------------------------------------

extern "C" ROOST_API RoostStatus roost_gdn_chunk_workspace(RoostContext*, const void* params, RoostWorkspaceSizes* sizes) {
  ROOST_RETURN_IF_FAILED(AdmitForSizing(params, sizes));
  const auto& p = *static_cast<const RoostGatedDeltaRuleParams*>(params);
  const ChunkArena l = MakeChunkArena(p.tokens, p.batch, p.v_heads);
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

namespace {

// plan() of the chunk variant: the chunk and sequence tables from cu_seqlens_host, copied to the workspace on the
// stream, and the stamp run() checks. With fused_gates the GDN params' g and beta are not read (a layer call computes
// them from the gates' inputs).
RoostStatus ChunkPlan(const RoostGatedDeltaRuleParams& p, const RoostWorkspace* ws, void* stream, bool fused_gates) {
  roost::Gate gate(kOp);
  ROOST_RETURN_IF_FAILED(Admit(p, true, fused_gates));
  const ChunkArena l = MakeChunkArena(p.tokens, p.batch, p.v_heads);
  gate.Expect(roost::HasDeviceRegion(ws, l.total) && ws->pinned_host != nullptr &&
                  ws->pinned_host_bytes >= l.tables_bytes && ws->plan != nullptr && ws->plan_bytes >= sizeof(ChunkStamp),
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
}

}  // namespace

extern "C" ROOST_API RoostStatus roost_gdn_chunk_plan(RoostContext* ctx, const void* params, const RoostWorkspace* ws,
                                                      void* stream) {
  roost::Gate gate(kOp);
  gate.Expect(ctx != nullptr && params != nullptr && ws != nullptr, ROOST_STATUS_INVALID_ARGUMENT,
              "plan() needs a context, params and a workspace");
  ROOST_GATE_RETURN(gate);
  const auto& p = *static_cast<const RoostGatedDeltaRuleParams*>(params);
  return roost::CatchAll(kOp, [&]() -> RoostStatus { return ChunkPlan(p, ws, stream, false); });
}

// plan() for roost_amd_gdn_chunk_layer_run: the chunk variant's plan of the GDN params, whose g and beta are not read
// when the gates params are given (the layer computes them).
extern "C" ROOST_API RoostStatus roost_amd_gdn_chunk_layer_plan(RoostContext* ctx, const void* gates_params,
                                                                const void* gdn_params, const RoostWorkspace* ws,
                                                                void* stream) {
  roost::Gate gate(kOp);
  gate.Expect(ctx != nullptr && gdn_params != nullptr && ws != nullptr, ROOST_STATUS_INVALID_ARGUMENT,
              "plan() needs a context, the GDN params and a workspace");
  ROOST_GATE_RETURN(gate);
  if (gates_params != nullptr) gate.Header(gates_params, sizeof(RoostGatedDeltaRuleGatesParams));
  ROOST_GATE_RETURN(gate);
  const auto& p = *static_cast<const RoostGatedDeltaRuleParams*>(gdn_params);
  return roost::CatchAll(kOp, [&]() -> RoostStatus {
    if (gates_params != nullptr) {
      ROOST_RETURN_IF_FAILED(Admit(p, true, true));
      GateSource gs;
      ROOST_RETURN_IF_FAILED(GateSourceOf(*static_cast<const RoostGatedDeltaRuleGatesParams*>(gates_params), p, &gs));
    }
    return ChunkPlan(p, ws, stream, gates_params != nullptr);
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
    const ChunkArena l = MakeChunkArena(p.tokens, p.batch, p.v_heads);
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

// One prefill pass of a GDN layer over the chunk variant (no reference counterpart; the Qwen3.5 worker runs
// CausalConv1d, GatedDeltaRuleGates, GatedDeltaRule and GatedRmsNorm one after another, Qwen35EagerModel.cs:89-92) in
// one call: the convolution, the chunk kernels computing g and beta where they read them (the gates op's arithmetic,
// so g and beta never reach memory), and the norm. The workspace is the chunk variant's (roost_gdn_chunk_workspace),
// planned by roost_amd_gdn_chunk_layer_plan.
extern "C" ROOST_API RoostStatus roost_amd_gdn_chunk_layer_run(RoostContext* ctx, const void* conv_params,
                                                               const void* gates_params, const void* gdn_params,
                                                               const void* norm_params, const RoostWorkspace* ws,
                                                               void* stream) {
  constexpr char kLayerOp[] = "gdn_chunk_layer";
  roost::Gate gate(kLayerOp);
  ROOST_RETURN_IF_FAILED(LayerHeaders(kLayerOp, ctx, conv_params, gates_params, gdn_params, norm_params));
  const auto& cp = *static_cast<const RoostCausalConv1dParams*>(conv_params);
  const auto& p = *static_cast<const RoostGatedDeltaRuleParams*>(gdn_params);
  const auto& np = *static_cast<const RoostGatedRmsNormParams*>(norm_params);
  return roost::CatchAll(kLayerOp, [&]() -> RoostStatus {
    LayerViews lv;
    ROOST_RETURN_IF_FAILED(AdmitLayer(kLayerOp, cp, gates_params, p, np, &lv));
    if (lv.empty) return ROOST_STATUS_OK;
    const ChunkArena l = MakeChunkArena(p.tokens, p.batch, p.v_heads);
    gate.Expect(roost::HasDeviceRegion(ws, l.total) && ws->plan != nullptr && ws->plan_bytes >= sizeof(ChunkStamp),
                ROOST_STATUS_WORKSPACE_TOO_SMALL, "the call needs %llu device bytes and its plan record",
                static_cast<unsigned long long>(l.total));
    ROOST_GATE_RETURN(gate);
    ChunkStamp stamp;
    std::memcpy(&stamp, ws->plan, sizeof(stamp));
    if (stamp.magic != kPlanMagic || stamp.batch != p.batch || stamp.tokens != p.tokens || stamp.chunks > l.max_chunks) {
      return roost::Report(ROOST_STATUS_NOT_PLANNED, kLayerOp,
                           "no roost_amd_gdn_chunk_layer_plan() for %u tokens in %u sequences in this workspace", p.tokens,
                           p.batch);
    }
    // The convolution (with its state update; the GDN kernels do not read the convolution's state), the chunk kernels
    // with the gates computed where they are read, then the norm, all on the caller's stream.
    ROOST_RETURN_IF_FAILED(roost_causal_conv1d_run(ctx, conv_params, nullptr, stream));
    if (stamp.chunks > 0) {
      ROOST_RETURN_IF_FAILED(LaunchChunk(p, ws, l, stamp.chunks, roost::Stream(stream), false, false, lv.gs));
    }
    // The norm's input is normally the scan's output, which the scan stores past the caches: the norm streams it and
    // its gate in the same way (config 4's layer: 0.286-0.287 against 0.289 ms; the standalone op keeps plain loads,
    // which are faster when its inputs are still cached).
    return roost_layer::RunNorm(np, roost::Stream(stream), true, kLayerOp);
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

constexpr uint64_t kStaticScratchBytes = 24ull << 20;  // 24 MiB per device, held until the process ends
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
    ChunkArena l = MakeRouteArena(p.tokens, p.batch, p.v_heads);
    if (p.cu_seqlens_host != nullptr) {
      // The host copy bounds the routing exactly: its long sequences and their chunks (a decode batch has none and
      // runs on the recurrent kernel alone, whatever its size).
      uint64_t long_seqs = 0, chunks = 0;
      for (uint32_t b = 0; b < p.batch; ++b) {
        const int64_t len = int64_t{p.cu_seqlens_host[b + 1]} - p.cu_seqlens_host[b];
        if (len >= static_cast<int64_t>(kRouteMinTokens)) {
          ++long_seqs;
          chunks += roost::CeilDiv(static_cast<uint64_t>(len), uint64_t{kChunk});
        }
      }
      if (long_seqs == 0) return LaunchRecurrent(p, s);
      l = MakeArena(std::min<uint64_t>(chunks, l.max_chunks), p.batch, p.v_heads,
                    std::min<uint64_t>(long_seqs, l.max_long));
    }
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



