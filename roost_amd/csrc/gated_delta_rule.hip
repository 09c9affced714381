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

#include <cmath>
#include <cstring>

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
constexpr uint32_t kPlanMagic = 0x50444752;  // "RGDP"

uint32_t Stride(uint32_t s) { return s == 0 ? kRow : s; }

// Checks shared by both variants (reference: kernels/src/ops/gated_delta_rule.cu:231-278), same statuses.
RoostStatus Validate(const RoostGatedDeltaRuleParams& p, bool need_host_cu) {
  using roost::Aligned;
  using roost::Fail;
  if (p.struct_size < sizeof(RoostGatedDeltaRuleParams) || p.abi_minor > ROOST_ABI_MINOR) {
    return Fail(ROOST_STATUS_ABI_MISMATCH, "GatedDeltaRule: params struct_size or abi_minor is not supported by this library");
  }
  if (p.k_heads != kHeads || p.v_heads != kHeads || p.k_dim != kDim || p.v_dim != kDim) {
    return Fail(ROOST_STATUS_UNSUPPORTED,
                "GatedDeltaRule: built for 16 key heads, 16 value heads and head size 128 (Qwen3.5-0.8B)");
  }
  if (p.l2_norm_qk == 0) return Fail(ROOST_STATUS_UNSUPPORTED, "GatedDeltaRule: only l2_norm_qk != 0 is built");
  if (p.tokens > kMaxTokens || p.batch > kMaxBatch) {
    return Fail(ROOST_STATUS_INVALID_ARGUMENT, "GatedDeltaRule: too many tokens or sequences for one call");
  }
  const uint64_t qs = Stride(p.q_stride), ks = Stride(p.k_stride), vs = Stride(p.v_stride);
  if (qs < kRow || ks < kRow || vs < kRow) {
    return Fail(ROOST_STATUS_INVALID_ARGUMENT, "GatedDeltaRule: a q, k or v stride is smaller than the row width");
  }
  auto span_ok = [](const RoostDeviceSpan& s, uint32_t dtype, uint64_t n) {
    return s.reserved0 == 0 && s.dtype == dtype && s.length >= n && (n == 0 || s.address != nullptr);
  };
  const uint64_t t = p.tokens;
  const uint64_t tail = t == 0 ? 0 : t - 1;
  if (!span_ok(p.q, ROOST_DTYPE_BF16, t == 0 ? 0 : tail * qs + kRow) ||
      !span_ok(p.k, ROOST_DTYPE_BF16, t == 0 ? 0 : tail * ks + kRow) ||
      !span_ok(p.v, ROOST_DTYPE_BF16, t == 0 ? 0 : tail * vs + kRow)) {
    return Fail(ROOST_STATUS_INVALID_ARGUMENT,
                "GatedDeltaRule: q, k and v must be bf16 spans reaching (tokens - 1) * stride + 2048 elements");
  }
  if (!span_ok(p.g, ROOST_DTYPE_F32, t * kHeads) || !span_ok(p.beta, ROOST_DTYPE_BF16, t * kHeads) ||
      !span_ok(p.output, ROOST_DTYPE_BF16, t * kRow)) {
    return Fail(ROOST_STATUS_UNSUPPORTED, "GatedDeltaRule: g must be float32, beta and output bf16, each long enough");
  }
  if (!span_ok(p.state, ROOST_DTYPE_F32, kStateElems) || p.state.length % kStateElems != 0) {
    return Fail(ROOST_STATUS_INVALID_ARGUMENT, "GatedDeltaRule: state must be a float32 pool of whole [16, 128, 128] slots");
  }
  if (!span_ok(p.state_slots, ROOST_DTYPE_I32, p.batch) || !span_ok(p.cu_seqlens, ROOST_DTYPE_I32, uint64_t{p.batch} + 1)) {
    return Fail(ROOST_STATUS_INVALID_ARGUMENT,
                "GatedDeltaRule: state_slots and cu_seqlens must be int32 spans of batch and batch + 1");
  }
  if (!Aligned(p.g.address, 16) || !Aligned(p.beta.address, 16) || !Aligned(p.output.address, 16) ||
      !Aligned(p.state.address, 16)) {
    return Fail(ROOST_STATUS_INVALID_ARGUMENT, "GatedDeltaRule: g, beta, output and state must be 16-byte aligned");
  }
  if (!Aligned(p.q.address, 2) || !Aligned(p.k.address, 2) || !Aligned(p.v.address, 2)) {
    return Fail(ROOST_STATUS_INVALID_ARGUMENT, "GatedDeltaRule: q, k and v must be 2-byte aligned");
  }
  if (need_host_cu && p.cu_seqlens_host == nullptr && p.batch > 0 && p.tokens > 0) {
    return Fail(ROOST_STATUS_INVALID_ARGUMENT, "GatedDeltaRule plan: cu_seqlens_host is required");
  }
  return ROOST_STATUS_OK;
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
    for (int i = 0; i < 32; ++i) s[i] = *reinterpret_cast<const float4*>(sp + (rq * 32 + i) * kDim + cg * 4);
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
    for (int i = 0; i < 32; ++i) *reinterpret_cast<float4*>(sp + (rq * 32 + i) * kDim + cg * 4) = s[i];
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
  using roost::Aligned;
  const uint64_t qs = Stride(p.q_stride), ks = Stride(p.k_stride), vs = Stride(p.v_stride);
  return Aligned(p.q.address, 16) && Aligned(p.k.address, 16) && Aligned(p.v.address, 8) && qs % 8 == 0 &&
         ks % 8 == 0 && vs % 4 == 0;
}

RoostStatus LaunchRecurrent(const RoostGatedDeltaRuleParams& p, hipStream_t stream) {
  const GdnArgs a = MakeArgs(p);
  const dim3 grid(p.batch, kHeads);
  if (Vec16(p)) {
    hipLaunchKernelGGL(RecurrentKernel<true>, grid, dim3(128), 0, stream, a);
  } else {
    hipLaunchKernelGGL(RecurrentKernel<false>, grid, dim3(128), 0, stream, a);
  }
  return roost::FromHip(hipGetLastError(), "GatedDeltaRule recurrent launch");
}

// ---- Chunk variant: plan tables ---------------------------------------------------------------------------------------

struct PlanRecord {
  uint32_t magic;
  uint32_t batch;
  uint32_t tokens;
  uint32_t chunks;
};

struct ChunkLayout {
  uint64_t chunk_table;  // [chunks] int2 (sequence, first token)
  uint64_t tables_bytes;
  uint64_t total;
  uint32_t max_chunks;
};

ChunkLayout MakeChunkLayout(uint64_t tokens, uint64_t batch) {
  ChunkLayout l{};
  l.max_chunks = static_cast<uint32_t>(tokens / kChunk + batch);
  l.chunk_table = 0;
  l.tables_bytes = roost::AlignUp(8ull * l.max_chunks, 256);
  l.total = l.tables_bytes;
  return l;
}

}  // namespace

// ---- Recurrent entry points ---------------------------------------------------------------------------------------

extern "C" ROOST_API RoostStatus roost_gdn_recurrent_workspace(RoostContext*, const void* params,
                                                               RoostWorkspaceSizes* sizes) {
  using namespace roost;
  if (params == nullptr || sizes == nullptr) return Fail(ROOST_STATUS_INVALID_ARGUMENT, "GatedDeltaRule: params or sizes is NULL");
  const auto& p = *static_cast<const RoostGatedDeltaRuleParams*>(params);
  if (p.struct_size < sizeof(RoostGatedDeltaRuleParams) || p.abi_minor > ROOST_ABI_MINOR) {
    return Fail(ROOST_STATUS_ABI_MISMATCH, "GatedDeltaRule: params struct_size or abi_minor is not supported by this library");
  }
  if (p.tokens > kMaxTokens || p.batch > kMaxBatch) {
    return Fail(ROOST_STATUS_INVALID_ARGUMENT, "GatedDeltaRule: too many tokens or sequences for one call");
  }
  sizes->device_bytes = 0;  // the views and the pool slots are read in place
  sizes->pinned_host_bytes = 0;
  sizes->plan_bytes = 0;
  sizes->device_alignment = 256;
  return ROOST_STATUS_OK;
}

extern "C" ROOST_API RoostStatus roost_gdn_recurrent_run(RoostContext* ctx, const void* params, const RoostWorkspace*,
                                                         void* stream) {
  using namespace roost;
  if (ctx == nullptr || params == nullptr) return Fail(ROOST_STATUS_INVALID_ARGUMENT, "GatedDeltaRule: ctx or params is NULL");
  const auto& p = *static_cast<const RoostGatedDeltaRuleParams*>(params);
  return Guarded("GatedDeltaRule", [&]() -> RoostStatus {
    ROOST_TRY(Validate(p, false));
    if (p.batch == 0 || p.tokens == 0) return ROOST_STATUS_OK;
    return LaunchRecurrent(p, Stream(stream));
  });
}

// ---- Chunk entry points ---------------------------------------------------------------------------------------------

extern "C" ROOST_API RoostStatus roost_gdn_chunk_workspace(RoostContext*, const void* params, RoostWorkspaceSizes* sizes) {
  using namespace roost;
  if (params == nullptr || sizes == nullptr) return Fail(ROOST_STATUS_INVALID_ARGUMENT, "GatedDeltaRule: params or sizes is NULL");
  const auto& p = *static_cast<const RoostGatedDeltaRuleParams*>(params);
  if (p.struct_size < sizeof(RoostGatedDeltaRuleParams) || p.abi_minor > ROOST_ABI_MINOR) {
    return Fail(ROOST_STATUS_ABI_MISMATCH, "GatedDeltaRule: params struct_size or abi_minor is not supported by this library");
  }
  if (p.tokens > kMaxTokens || p.batch > kMaxBatch) {
    return Fail(ROOST_STATUS_INVALID_ARGUMENT, "GatedDeltaRule: too many tokens or sequences for one call");
  }
  const ChunkLayout l = MakeChunkLayout(p.tokens, p.batch);
  sizes->device_bytes = l.total;
  sizes->pinned_host_bytes = l.tables_bytes;
  sizes->plan_bytes = sizeof(PlanRecord);
  sizes->device_alignment = 256;
  return ROOST_STATUS_OK;
}

extern "C" ROOST_API RoostStatus roost_gdn_chunk_plan(RoostContext* ctx, const void* params, const RoostWorkspace* ws,
                                                      void* stream) {
  using namespace roost;
  if (ctx == nullptr || params == nullptr || ws == nullptr) {
    return Fail(ROOST_STATUS_INVALID_ARGUMENT, "GatedDeltaRule plan: ctx, params or workspace is NULL");
  }
  const auto& p = *static_cast<const RoostGatedDeltaRuleParams*>(params);
  return Guarded("GatedDeltaRule", [&]() -> RoostStatus {
    ROOST_TRY(Validate(p, true));
    const ChunkLayout l = MakeChunkLayout(p.tokens, p.batch);
    if (!DeviceWorkspaceOk(ws, l.total) || ws->pinned_host == nullptr || ws->pinned_host_bytes < l.tables_bytes ||
        ws->plan == nullptr || ws->plan_bytes < sizeof(PlanRecord)) {
      return Fail(ROOST_STATUS_WORKSPACE_TOO_SMALL,
                  "GatedDeltaRule plan: workspace is missing or smaller than the workspace query said");
    }
    PlanRecord rec{kPlanMagic, p.batch, p.tokens, 0};
    if (p.batch == 0 || p.tokens == 0) {
      std::memcpy(ws->plan, &rec, sizeof(rec));
      return ROOST_STATUS_OK;
    }
    const int32_t* cu = p.cu_seqlens_host;
    if (cu[0] != 0 || static_cast<uint32_t>(cu[p.batch]) != p.tokens) {
      return Fail(ROOST_STATUS_INVALID_ARGUMENT, "GatedDeltaRule plan: cu_seqlens_host must start at 0 and end at tokens");
    }
    auto* table = static_cast<int32_t*>(ws->pinned_host);
    uint32_t n = 0;
    for (uint32_t b = 0; b < p.batch; ++b) {
      if (cu[b + 1] < cu[b]) return Fail(ROOST_STATUS_INVALID_ARGUMENT, "GatedDeltaRule plan: cu_seqlens_host decreases");
      for (int32_t t = cu[b]; t < cu[b + 1]; t += kChunk) {
        table[2 * n] = static_cast<int32_t>(b);
        table[2 * n + 1] = t;
        ++n;
      }
    }
    rec.chunks = n;
    ROOST_TRY(FromHip(hipMemcpyAsync(ws->device, table, 8ull * n, hipMemcpyHostToDevice, Stream(stream)),
                      "GatedDeltaRule plan copy"));
    std::memcpy(ws->plan, &rec, sizeof(rec));
    return ROOST_STATUS_OK;
  });
}

extern "C" ROOST_API RoostStatus roost_gdn_chunk_run(RoostContext* ctx, const void* params, const RoostWorkspace* ws,
                                                     void* stream) {
  using namespace roost;
  if (ctx == nullptr || params == nullptr) return Fail(ROOST_STATUS_INVALID_ARGUMENT, "GatedDeltaRule: ctx or params is NULL");
  const auto& p = *static_cast<const RoostGatedDeltaRuleParams*>(params);
  return Guarded("GatedDeltaRule", [&]() -> RoostStatus {
    ROOST_TRY(Validate(p, false));
    if (p.batch == 0 || p.tokens == 0) return ROOST_STATUS_OK;
    const ChunkLayout l = MakeChunkLayout(p.tokens, p.batch);
    if (!DeviceWorkspaceOk(ws, l.total) || ws->plan == nullptr || ws->plan_bytes < sizeof(PlanRecord)) {
      return Fail(ROOST_STATUS_WORKSPACE_TOO_SMALL, "GatedDeltaRule: workspace or plan is missing or too small");
    }
    PlanRecord rec;
    std::memcpy(&rec, ws->plan, sizeof(rec));
    if (rec.magic != kPlanMagic || rec.batch != p.batch || rec.tokens != p.tokens || rec.chunks > l.max_chunks) {
      return Fail(ROOST_STATUS_NOT_PLANNED, "GatedDeltaRule: plan() has not run for these tokens and sequences");
    }
    return LaunchRecurrent(p, Stream(stream));
  });
}
