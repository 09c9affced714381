// The attention layer's input ops for gfx950: QkNorm (ROOST_OP_QK_NORM), Rope (ROOST_OP_ROPE) and the fused
// QkvQkNormRopeCacheWrite (ROOST_OP_QKV_QK_NORM_ROPE_CACHE_WRITE) that feeds PagedAttention.
//
// Semantics: src/Starlings.Roost.Ops/CpuOps.cs:63-175 (QkNorm, Rope) and CpuOps.Fused.cs:37-95 (the fused op, defined
// as its unfused parts in order), with the refusal rules of the reference's QkNormRun and RopeRun
// (kernels/src/m0_ops.cu:89-255). Every element is computed in fp32 and rounded into its span's type where CpuOps
// stores it: the fused op rounds the normalised head before rotating it, as the unfused calls do.
//
// One (token, head) row is served by G lanes of a wavefront (G a power of two, 64 / G rows per wavefront); a lane
// holds kJ chunks of kV consecutive elements (16-byte loads and stores when the rows allow them). The sum of squares
// is reduced over the G lanes by a fixed xor butterfly. The rotation partner of each element (i +- R/2 for NeoX halves,
// i ^ 1 for interleaved pairs) is read from a per-wavefront copy of the rounded row in LDS. Angles follow the
// reference's own rope kernel: frequencies theta^(-2i/R) (Llama 3 scaled when asked) in double in an LDS table,
// position * frequency in double reduced modulo 2 pi in double, then sincosf of the reduced angle.
//
// Nothing here allocates, synchronises the host or reads host memory; each call is one launch on the caller's stream.

#include <cmath>

#include "common.h"

namespace {

using namespace roost_dev;

constexpr int kMaxHeadDim = 1024;

template <typename T>
__device__ __forceinline__ float LoadT(const T* p) {
  if constexpr (sizeof(T) == 2) {
    return Bf16ToF32(*reinterpret_cast<const uint16_t*>(p));
  } else {
    return *reinterpret_cast<const float*>(p);
  }
}
template <typename T>
__device__ __forceinline__ void StoreT(T* p, float v) {
  if constexpr (sizeof(T) == 2) {
    *reinterpret_cast<uint16_t*>(p) = static_cast<uint16_t>(PackBf16Rne(v, 0.0f));
  } else {
    *reinterpret_cast<float*>(p) = v;
  }
}
// v rounded to T and widened back (what CpuOps reads after storing v in T).
template <typename T>
__device__ __forceinline__ float RoundT(float v) {
  if constexpr (sizeof(T) == 2) {
    return Bf16LoToF32(PackBf16Rne(v, 0.0f));
  } else {
    return v;
  }
}

// Elements e and e + 1 of v rounded to T (bf16: one v_cvt_pk_bf16_f32, round to nearest even).
template <typename T>
__device__ __forceinline__ void RoundPairT(float* v) {
  if constexpr (sizeof(T) == 2) {
    const uint32_t w = PackBf16Rne(v[0], v[1]);
    v[0] = Bf16LoToF32(w);
    v[1] = Bf16HiToF32(w);
  }
}

// kV consecutive elements at p as floats (one 16-byte load when kV * sizeof(T) == 16).
template <typename T, int kV>
__device__ __forceinline__ void LoadChunk(const T* p, float* v) {
  if constexpr (kV * sizeof(T) == 16) {
    const uint4 q = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int e = 0; e < kV; ++e) {
      v[e] = sizeof(T) == 2 ? ((e & 1) ? Bf16HiToF32(w[e >> 1]) : Bf16LoToF32(w[e >> 1])) : __uint_as_float(w[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < kV; ++e) v[e] = LoadT(p + e);
  }
}
template <typename T, int kV>
__device__ __forceinline__ void StoreChunk(T* p, const float* v) {
  if constexpr (kV * sizeof(T) == 16) {
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) w[q] = sizeof(T) == 2 ? PackBf16Rne(v[2 * q], v[2 * q + 1]) : __float_as_uint(v[q]);
    *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  } else {
#pragma unroll
    for (int e = 0; e < kV; ++e) StoreT(p + e, v[e]);
  }
}

// What a rope launch needs besides the rows.
struct RopeSpec {
  const int32_t* positions;
  uint32_t rot;  // rotated dims R (even, <= head_dim)
  uint32_t interleaved;
  uint32_t llama3;
  float theta, factor, low_ff, high_ff;
  uint32_t original_max;
  uint32_t chunk_pairs;  // every pair lies within one chunk (interleaved) or pairs whole chunks (NeoX)
};

// Frequency i of R rotary dims (CpuOps.cs:141-163): theta^(-2i/R), Llama 3 scaled when asked; in double.
__device__ double Frequency(const RopeSpec& r, uint32_t i) {
  double f = pow(static_cast<double>(r.theta), -2.0 * i / r.rot);
  if (r.llama3) {
    const double orig = r.original_max;
    const double wavelen = 2.0 * 3.14159265358979323846 / f;
    const double low = orig / static_cast<double>(r.low_ff), high = orig / static_cast<double>(r.high_ff);
    if (wavelen < high) {
      // kept
    } else if (wavelen > low) {
      f = f / static_cast<double>(r.factor);
    } else {
      const double smooth = (orig / wavelen - static_cast<double>(r.low_ff)) /
                            (static_cast<double>(r.high_ff) - static_cast<double>(r.low_ff));
      f = (1.0 - smooth) * f / static_cast<double>(r.factor) + smooth * f;
    }
  }
  return f;
}

// The workgroup's angle table: cs[t * R/2 + i] = (cos, sin) of positions[t0 + t] * f_i for its tokens t < count. The
// angle is formed and reduced to [-pi, pi] in double, then sincosf of the reduced angle. Every head of a token reads
// the same entries, so each is computed once per token. Two barriers: frequencies, then angles.
__device__ void BuildAngles(const RopeSpec& r, uint64_t t0, uint32_t count, double* freq, float2* cs) {
  constexpr double kTwoPi = 6.283185307179586476925286766559;
  constexpr double kInvTwoPi = 0.15915494309189533576888376337251;
  const uint32_t half = r.rot / 2;
  for (uint32_t i = threadIdx.x; i < half; i += blockDim.x) freq[i] = Frequency(r, i);
  __syncthreads();
  for (uint32_t idx = threadIdx.x; idx < count * half; idx += blockDim.x) {
    const uint32_t t = idx / half, i = idx - t * half;
    const double a = static_cast<double>(r.positions[t0 + t]) * freq[i];
    const double red = fma(-kTwoPi, rint(a * kInvTwoPi), a);
    float sn, c;
    sincosf(static_cast<float>(red), &sn, &c);
    cs[idx] = make_float2(c, sn);
  }
  __syncthreads();
}

// One row's values held by the G lanes serving it: chunk c = sub + G * j of kV elements for j < kJ.
template <int kV, int kJ>
struct RowRegs {
  float v[kJ][kV];
};

// v of lane (lane ^ M): ds_swizzle's bit-mask mode within each 32 lanes for M < 32 (one instruction, no address), a
// full-wave permute for M = 32.
template <int M>
__device__ __forceinline__ float XorLanes(float v) {
  if constexpr (M < 32) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), (M << 10) | 0x1F));
  } else {
    return __shfl_xor(v, M, 64);
  }
}

// RmsNorm of the row in place: v * rsqrt(mean(v^2) + eps) * w, then rounded to T (CpuOps.cs:89-103). Lanes whose
// chunks lie beyond head_dim hold zeros and contribute nothing; w holds the lane's chunks of the weight. The sum of
// squares is reduced over the g lanes of the row by an xor butterfly with constant masks (DPP / swizzle moves).
template <typename T, int kV, int kJ>
__device__ __forceinline__ void NormRow(RowRegs<kV, kJ>& r, const RowRegs<kV, kJ>& w, uint32_t sub, uint32_t g,
                                        uint32_t chunks, float inv_dim, float eps) {
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < kJ; ++j)
#pragma unroll
    for (int e = 0; e < kV; ++e) ss = fmaf(r.v[j][e], r.v[j][e], ss);
  if (g > 1) ss += XorLanes<1>(ss);
  if (g > 2) ss += XorLanes<2>(ss);
  if (g > 4) ss += XorLanes<4>(ss);
  if (g > 8) ss += XorLanes<8>(ss);
  if (g > 16) ss += XorLanes<16>(ss);
  if (g > 32) ss += XorLanes<32>(ss);
  const float inv = rsqrtf(ss * inv_dim + eps);
#pragma unroll
  for (int j = 0; j < kJ; ++j) {
    const uint32_t c = sub + g * j;
    if (c < chunks) {
#pragma unroll
      for (int e = 0; e < kV; ++e) r.v[j][e] = r.v[j][e] * inv * w.v[j][e];
      if constexpr (kV % 2 == 0) {
#pragma unroll
        for (int e = 0; e < kV; e += 2) RoundPairT<T>(&r.v[j][e]);
      } else {
#pragma unroll
        for (int e = 0; e < kV; ++e) r.v[j][e] = RoundT<T>(r.v[j][e]);
      }
    }
  }
}

// The rotation with whole chunks (vector rows, host-checked layout): interleaved pairs lie inside a chunk; NeoX pairs
// chunk c with chunk c +- R/(2 kV), read from the row's LDS copy as vectors. Same arithmetic, element for element, as
// the general form below.
template <typename T, int kV, int kJ>
__device__ __forceinline__ void RopeRowChunks(RowRegs<kV, kJ>& r, float* row, const float2* cs, const RopeSpec& rs,
                                              uint32_t sub, uint32_t g, uint32_t chunks) {
  static_assert(kV % 4 == 0, "vector chunks hold 4 or 8 elements");
  if (rs.interleaved) {
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
      const uint32_t c = sub + g * j, i0 = c * kV;
      if (c >= chunks || i0 >= rs.rot) continue;
      const float4* a4 = reinterpret_cast<const float4*>(cs + i0 / 2);
#pragma unroll
      for (int q = 0; q < kV / 4; ++q) {
        const float4 a = a4[q];  // pairs (2q, 2q + 1) of the chunk: (cos, sin) twice
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int e = 4 * q + 2 * h;
          const float c0 = h ? a.z : a.x, s0 = h ? a.w : a.y;
          const float x1 = r.v[j][e], x2 = r.v[j][e + 1];
          r.v[j][e] = fmaf(x1, c0, -(x2 * s0));
          r.v[j][e + 1] = fmaf(x2, c0, x1 * s0);
          RoundPairT<T>(&r.v[j][e]);
        }
      }
    }
    return;
  }
  const uint32_t half = rs.rot / 2;
#pragma unroll
  for (int j = 0; j < kJ; ++j) {
    const uint32_t c = sub + g * j;
    if (c < chunks && c * kV < rs.rot) {
#pragma unroll
      for (int q = 0; q < kV / 4; ++q) {
        reinterpret_cast<float4*>(row + c * kV)[q] =
            make_float4(r.v[j][4 * q], r.v[j][4 * q + 1], r.v[j][4 * q + 2], r.v[j][4 * q + 3]);
      }
    }
  }
  __builtin_amdgcn_wave_barrier();  // the row's lanes are all in this wavefront: LDS order within it is program order
#pragma unroll
  for (int j = 0; j < kJ; ++j) {
    const uint32_t c = sub + g * j, i0 = c * kV;
    if (c >= chunks || i0 >= rs.rot) continue;
    const bool first = i0 < half;
    const uint32_t p0 = first ? i0 + half : i0 - half, k0 = first ? i0 : i0 - half;
    float xp[kV];
    float2 a[kV];
#pragma unroll
    for (int q = 0; q < kV / 4; ++q) {
      const float4 v = reinterpret_cast<const float4*>(row + p0)[q];
      xp[4 * q] = v.x; xp[4 * q + 1] = v.y; xp[4 * q + 2] = v.z; xp[4 * q + 3] = v.w;
    }
#pragma unroll
    for (int q = 0; q < kV / 2; ++q) {
      const float4 v = reinterpret_cast<const float4*>(cs + k0)[q];
      a[2 * q] = make_float2(v.x, v.y);
      a[2 * q + 1] = make_float2(v.z, v.w);
    }
#pragma unroll
    for (int e = 0; e < kV; ++e) {
      const float x = r.v[j][e];
      r.v[j][e] = first ? fmaf(x, a[e].x, -(xp[e] * a[e].y)) : fmaf(x, a[e].x, xp[e] * a[e].y);
    }
#pragma unroll
    for (int e = 0; e < kV; e += 2) RoundPairT<T>(&r.v[j][e]);
  }
  __builtin_amdgcn_wave_barrier();
}

// Rotation of the row in place (CpuOps.cs:111-139, 165-175): pair (x1, x2) -> (x1 c - x2 s, x2 c + x1 s), NeoX
// partners i +- R/2 or interleaved i ^ 1, elements at and beyond R kept; rounded to T. `row` is this row's LDS copy.
template <typename T, int kV, int kJ>
__device__ __forceinline__ void RopeRow(RowRegs<kV, kJ>& r, float* row, const float2* cs, const RopeSpec& rs,
                                        uint32_t sub, uint32_t g, uint32_t chunks) {
  if constexpr (kV > 1) {
    if (rs.chunk_pairs) {
      RopeRowChunks<T, kV, kJ>(r, row, cs, rs, sub, g, chunks);
      return;
    }
  }
#pragma unroll
  for (int j = 0; j < kJ; ++j) {
    const uint32_t c = sub + g * j;
    if (c < chunks) {
#pragma unroll
      for (int e = 0; e < kV; ++e) row[c * kV + e] = r.v[j][e];
    }
  }
  __builtin_amdgcn_wave_barrier();  // the row's lanes are all in this wavefront: LDS order within it is program order
  const uint32_t half = rs.rot / 2;
#pragma unroll
  for (int j = 0; j < kJ; ++j) {
    const uint32_t c = sub + g * j;
    if (c >= chunks) continue;
#pragma unroll
    for (int e = 0; e < kV; ++e) {
      const uint32_t i = c * kV + e;
      if (i >= rs.rot) continue;
      uint32_t pair, partner;
      bool first;
      if (rs.interleaved) {
        pair = i >> 1;
        partner = i ^ 1u;
        first = (i & 1u) == 0;
      } else {
        first = i < half;
        pair = first ? i : i - half;
        partner = first ? i + half : i - half;
      }
      const float2 a = cs[pair];
      const float x = r.v[j][e], xp = row[partner];
      // Explicit fused multiply-adds: every kernel that rotates a row rounds it the same way.
      r.v[j][e] = RoundT<T>(first ? fmaf(x, a.x, -(xp * a.y)) : fmaf(x, a.x, xp * a.y));
    }
  }
  __builtin_amdgcn_wave_barrier();
}

template <typename T, int kV, int kJ>
__device__ __forceinline__ void LoadRow(RowRegs<kV, kJ>& r, const T* src, uint32_t sub, uint32_t g, uint32_t chunks,
                                        bool live) {
#pragma unroll
  for (int j = 0; j < kJ; ++j) {
    const uint32_t c = sub + g * j;
    if (live && c < chunks) {
      LoadChunk<T, kV>(src + c * kV, r.v[j]);
    } else {
#pragma unroll
      for (int e = 0; e < kV; ++e) r.v[j][e] = 0.0f;
    }
  }
}
// A lane's chunks of one row as fetched: the 16-byte words of vector rows (unpacked only when the row is used, so a
// fetched row stays in flight while the previous one is computed), or the floats of scalar rows.
template <typename T, int kV, int kJ>
struct RowRaw {
  static constexpr bool kVec = kV * sizeof(T) == 16;
  uint4 w[kVec ? kJ : 1];
  RowRegs<kV, kVec ? 1 : kJ> f;
};
// Fetches the row at src (when live) or, for lanes without a row or past head_dim, the harmless address `safe`
// (their values are zeroed on unpacking).
template <typename T, int kV, int kJ>
__device__ __forceinline__ void FetchRow(RowRaw<T, kV, kJ>& raw, const T* src, const T* safe, uint32_t sub, uint32_t g,
                                         uint32_t chunks, bool live) {
  if constexpr (RowRaw<T, kV, kJ>::kVec) {
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
      const uint32_t c = sub + g * j;
      const bool ok = live && c < chunks;
      raw.w[j] = *reinterpret_cast<const uint4*>(ok ? src + c * kV : safe);
    }
  } else {
    LoadRow<T, kV, kJ>(raw.f, src, sub, g, chunks, live);
  }
}
template <typename T, int kV, int kJ>
__device__ __forceinline__ void UnpackRow(const RowRaw<T, kV, kJ>& raw, RowRegs<kV, kJ>& r, uint32_t sub, uint32_t g,
                                          uint32_t chunks, bool live) {
  if constexpr (RowRaw<T, kV, kJ>::kVec) {
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
      const bool ok = live && sub + g * j < chunks;
      const uint32_t wd[4] = {raw.w[j].x, raw.w[j].y, raw.w[j].z, raw.w[j].w};
#pragma unroll
      for (int e = 0; e < kV; ++e) {
        const float v = sizeof(T) == 2 ? ((e & 1) ? Bf16HiToF32(wd[e >> 1]) : Bf16LoToF32(wd[e >> 1]))
                                       : __uint_as_float(wd[e]);
        r.v[j][e] = ok ? v : 0.0f;
      }
    }
  } else {
    r = raw.f;
  }
}

template <typename T, int kV, int kJ>
__device__ __forceinline__ void StoreRow(const RowRegs<kV, kJ>& r, T* dst, uint32_t sub, uint32_t g, uint32_t chunks) {
#pragma unroll
  for (int j = 0; j < kJ; ++j) {
    const uint32_t c = sub + g * j;
    if (c < chunks) StoreChunk<T, kV>(dst + c * kV, r.v[j]);
  }
}

// The lane's place: row index (over the whole launch), lane within the row.
struct Lane {
  uint64_t row;
  uint32_t sub;
};
__device__ __forceinline__ Lane Place(uint32_t g) {
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  Lane l;
  l.sub = lane % g;
  l.row = (static_cast<uint64_t>(blockIdx.x) * (blockDim.x >> 6) + wave) * (64 / g) + lane / g;
  return l;
}

// Rope launches: workgroup b serves tokens [b * tpb, b * tpb + tpb) (tpb tokens per block), all of their head rows;
// wavefront w takes row groups w, w + 4, ... of 64 / g rows each. Dynamic LDS, sized by RopeLdsBytes: the frequency
// table (R/2 doubles), the angle table (tpb x R/2 (cos, sin) pairs) and each wavefront's row copies (64 / g rows).
constexpr uint32_t kMaxTpb = 8;

__host__ __device__ constexpr uint64_t RopeLdsBytes(uint32_t half, uint32_t tpb, uint32_t g, uint32_t head_dim) {
  return uint64_t{half} * 8 + uint64_t{tpb} * half * 8 + uint64_t{4} * (64 / g) * head_dim * 4;
}
__device__ __forceinline__ void CarveLds(uint32_t half, uint32_t tpb, uint32_t g, uint32_t head_dim, double** freq,
                                         float2** cs, float** rows) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  *freq = reinterpret_cast<double*>(lds_raw);
  *cs = reinterpret_cast<float2*>(lds_raw + uint64_t{half} * 8);
  *rows = reinterpret_cast<float*>(lds_raw + uint64_t{half} * 8 + uint64_t{tpb} * half * 8);
  (void)g;
  (void)head_dim;
}

struct TokenRows {
  uint64_t t0;     // first token of the workgroup
  uint32_t count;  // its tokens
  uint32_t rows;   // count * heads
};
__device__ __forceinline__ TokenRows BlockTokens(uint32_t tokens, uint32_t tpb, uint32_t heads) {
  TokenRows tr;
  tr.t0 = static_cast<uint64_t>(blockIdx.x) * tpb;
  tr.count = static_cast<uint32_t>(min(static_cast<uint64_t>(tpb), tokens - tr.t0));
  tr.rows = tr.count * heads;
  return tr;
}

// ---- QkNorm: rows are (token, head) over q heads then k heads, in place. --------------------------------------------
template <typename T, int kV, int kJ>
__global__ void __launch_bounds__(256) QkNormKernel(T* q, T* k, const T* qw, const T* kw, uint32_t tokens,
                                                    uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim,
                                                    uint64_t q_stride, uint64_t k_stride, float eps, uint32_t g) {
  const Lane l = Place(g);
  const uint32_t heads = q_heads + kv_heads;
  const uint64_t rows = static_cast<uint64_t>(tokens) * heads;
  const bool live = l.row < rows;
  const uint64_t t = live ? l.row / heads : 0;
  const uint32_t h = live ? static_cast<uint32_t>(l.row - t * heads) : 0;
  const bool is_q = h < q_heads;
  T* x = is_q ? q + t * q_stride + static_cast<uint64_t>(h) * head_dim
              : k + t * k_stride + static_cast<uint64_t>(h - q_heads) * head_dim;
  const uint32_t chunks = head_dim / kV;
  // The row and the weight requested together, without a branch around either (lanes past the row read the weight's
  // first chunk instead), and unpacked after: a request made and used inside a branch waited for everything before it.
  const T* wp = is_q ? qw : kw;
  RowRaw<T, kV, kJ> rr, wr;
  FetchRow<T, kV, kJ>(rr, x, wp, l.sub, g, chunks, live);
  FetchRow<T, kV, kJ>(wr, wp, wp, l.sub, g, chunks, true);
  RowRegs<kV, kJ> r, w;
  UnpackRow<T, kV, kJ>(rr, r, l.sub, g, chunks, live);
  UnpackRow<T, kV, kJ>(wr, w, l.sub, g, chunks, true);
  NormRow<T, kV, kJ>(r, w, l.sub, g, chunks, 1.0f / static_cast<float>(head_dim), eps);
  if (live) StoreRow<T, kV, kJ>(r, x, l.sub, g, chunks);
}

// ---- Rope: rows are (token, head) over q heads then k heads, contiguous [tokens, heads, head_dim], in place. --------
template <typename T, int kV, int kJ>
__global__ void __launch_bounds__(256) RopeKernel(T* q, T* k, RopeSpec rs, uint32_t tokens, uint32_t q_heads,
                                                  uint32_t kv_heads, uint32_t head_dim, uint32_t g, uint32_t tpb) {
  const uint32_t heads = q_heads + kv_heads;
  const TokenRows tr = BlockTokens(tokens, tpb, heads);
  double* freq;
  float2* cs;
  float* lds;
  CarveLds(rs.rot / 2, tpb, g, head_dim, &freq, &cs, &lds);
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, per = 64 / g, sub = lane % g;
  const uint32_t chunks = head_dim / kV, half = rs.rot / 2;
  float* row_lds = lds + (wave * per + lane / g) * head_dim;
  // Row r of the workgroup: its address, and whether this lane's row exists.
  auto row_at = [&](uint32_t grp, bool* live, uint32_t* lt) -> T* {
    const uint32_t r = grp * per + lane / g;
    *live = r < tr.rows;
    *lt = *live ? r / heads : 0;
    const uint32_t h = *live ? r - *lt * heads : 0;
    const uint64_t t = tr.t0 + *lt;
    return h < q_heads ? q + (t * q_heads + h) * head_dim : k + (t * kv_heads + (h - q_heads)) * head_dim;
  };
  // Software pipeline: the first group's rows are requested before the angle table is built, and each group's
  // successor before the group is computed.
  bool live;
  uint32_t lt;
  T* x = row_at(wave, &live, &lt);
  RowRaw<T, kV, kJ> raw;
  FetchRow<T, kV, kJ>(raw, x, q, sub, g, chunks, live);
  BuildAngles(rs, tr.t0, tr.count, freq, cs);
  for (uint32_t grp = wave; grp * per < tr.rows; grp += 4) {
    RowRegs<kV, kJ> cur;
    UnpackRow<T, kV, kJ>(raw, cur, sub, g, chunks, live);
    bool live_n;
    uint32_t lt_n;
    T* x_n = row_at(grp + 4, &live_n, &lt_n);
    FetchRow<T, kV, kJ>(raw, x_n, q, sub, g, chunks, live_n);
    RopeRow<T, kV, kJ>(cur, row_lds, cs + lt * half, rs, sub, g, chunks);
    if (live) StoreRow<T, kV, kJ>(cur, x, sub, g, chunks);
    x = x_n;
    live = live_n;
    lt = lt_n;
  }
}

// ---- QkvQkNormRopeCacheWrite: rows are (token, head) over q, k and v heads of each [q | k | v] row. ----------------
struct QkvArgs {
  const void* qkv;
  void* q;
  const void* qw;
  const void* kw;
  void* k_cache;
  void* v_cache;
  const int64_t* slots;
  uint64_t pool_rows;  // (page, offset) rows both pools hold
  uint32_t tokens, q_heads, kv_heads, head_dim;
  float eps;
};

// A v row goes to the cache as stored (CacheWrite copies it; a wider cache type widens it exactly).
template <typename T, typename C, int kV, int kJ>
__device__ __forceinline__ void CopyVRow(const T* src, C* dst, uint32_t sub, uint32_t g, uint32_t chunks) {
#pragma unroll
  for (int j = 0; j < kJ; ++j) {
    const uint32_t c = sub + g * j;
    if (c >= chunks) continue;
    if constexpr (sizeof(C) == sizeof(T) && kV * sizeof(T) == 16) {
      *reinterpret_cast<uint4*>(dst + c * kV) = *reinterpret_cast<const uint4*>(src + c * kV);
    } else if constexpr (sizeof(C) == sizeof(T)) {
#pragma unroll
      for (int e = 0; e < kV; ++e) dst[c * kV + e] = src[c * kV + e];
    } else {
      float v[kV];
      LoadChunk<T, kV>(src + c * kV, v);
#pragma unroll
      for (int e = 0; e < kV; ++e) StoreT(dst + c * kV + e, v[e]);
    }
  }
}

// Workgroup b serves tokens [b * tpb, b * tpb + tpb). Its wavefronts first take the v rows (plain copies), then the q
// and k rows (norm, rounding, rotation), so a wavefront's rows share one path.
template <typename T, typename C, int kV, int kJ>
__global__ void __launch_bounds__(256) QkvKernel(QkvArgs a, RopeSpec rs, uint32_t g, uint32_t tpb) {
  double* freq;
  float2* cs;
  float* lds;
  CarveLds(rs.rot / 2, tpb, g, a.head_dim, &freq, &cs, &lds);
  const uint32_t qk_heads = a.q_heads + a.kv_heads, heads = qk_heads + a.kv_heads;
  const TokenRows tr = BlockTokens(a.tokens, tpb, heads);
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, per = 64 / g, sub = lane % g;
  const uint32_t chunks = a.head_dim / kV, half = rs.rot / 2;
  const T* qkv = static_cast<const T*>(a.qkv);
  RowRaw<T, kV, kJ> wq, wk;  // this lane's chunks of the two norm weights, fetched once
  FetchRow<T, kV, kJ>(wq, static_cast<const T*>(a.qw), static_cast<const T*>(a.qw), sub, g, chunks, true);
  FetchRow<T, kV, kJ>(wk, static_cast<const T*>(a.kw), static_cast<const T*>(a.kw), sub, g, chunks, true);
  // v rows (no angles needed): tr.count * kv_heads of them.
  const uint32_t v_rows = tr.count * a.kv_heads;
  for (uint32_t grp = wave; grp * per < v_rows; grp += 4) {
    const uint32_t r = grp * per + lane / g;
    if (r >= v_rows) continue;
    const uint32_t lt = r / a.kv_heads, h = r - lt * a.kv_heads;
    const uint64_t t = tr.t0 + lt;
    const int64_t slot = a.slots[t];
    if (slot < 0 || static_cast<uint64_t>(slot) >= a.pool_rows) continue;
    CopyVRow<T, C, kV, kJ>(qkv + (t * heads + qk_heads + h) * a.head_dim,
                           static_cast<C*>(a.v_cache) + (static_cast<uint64_t>(slot) * a.kv_heads + h) * a.head_dim,
                           sub, g, chunks);
  }
  float* row_lds = lds + (wave * per + lane / g) * a.head_dim;
  const uint32_t qk_rows = tr.count * qk_heads;
  struct RowAt {
    bool live, is_q;
    uint32_t lt, h;
    int64_t slot;  // k rows: the token's cache slot, read with the row (one iteration ahead)
  };
  auto row_at = [&](uint32_t grp) {
    RowAt w;
    const uint32_t r = grp * per + lane / g;
    w.live = r < qk_rows;
    w.lt = w.live ? r / qk_heads : 0;
    w.h = w.live ? r - w.lt * qk_heads : 0;
    w.is_q = w.h < a.q_heads;
    w.slot = a.slots[tr.t0 + w.lt];
    return w;
  };
  auto src_of = [&](const RowAt& w) { return qkv + ((tr.t0 + w.lt) * heads + w.h) * a.head_dim; };
  // Software pipeline: the first group's rows are requested before the angle table is built, and each group's
  // successor before the group is computed.
  RowAt w = row_at(wave);
  RowRaw<T, kV, kJ> raw;
  FetchRow<T, kV, kJ>(raw, src_of(w), qkv, sub, g, chunks, w.live);
  BuildAngles(rs, tr.t0, tr.count, freq, cs);
  const float inv_dim = 1.0f / static_cast<float>(a.head_dim);
  for (uint32_t grp = wave; grp * per < qk_rows; grp += 4) {
    RowRegs<kV, kJ> cur;
    UnpackRow<T, kV, kJ>(raw, cur, sub, g, chunks, w.live);
    const RowAt wn = row_at(grp + 4);
    FetchRow<T, kV, kJ>(raw, src_of(wn), qkv, sub, g, chunks, wn.live);
    RowRegs<kV, kJ> wt;
    UnpackRow<T, kV, kJ>(w.is_q ? wq : wk, wt, sub, g, chunks, true);
    NormRow<T, kV, kJ>(cur, wt, sub, g, chunks, inv_dim, a.eps);
    RopeRow<T, kV, kJ>(cur, row_lds, cs + w.lt * half, rs, sub, g, chunks);
    const uint64_t t = tr.t0 + w.lt;
    if (w.live && w.is_q) {
      StoreRow<T, kV, kJ>(cur, static_cast<T*>(a.q) + (t * a.q_heads + w.h) * a.head_dim, sub, g, chunks);
    } else if (w.live) {
      const int64_t slot = w.slot;
      if (slot >= 0 && static_cast<uint64_t>(slot) < a.pool_rows) {
        C* dst = static_cast<C*>(a.k_cache) + (static_cast<uint64_t>(slot) * a.kv_heads + (w.h - a.q_heads)) * a.head_dim;
        if constexpr (sizeof(C) == sizeof(T)) {
          StoreRow<T, kV, kJ>(cur, reinterpret_cast<T*>(dst), sub, g, chunks);
        } else {
#pragma unroll
          for (int j = 0; j < kJ; ++j) {
            const uint32_t c = sub + g * j;
            if (c < chunks) {
#pragma unroll
              for (int e = 0; e < kV; ++e) StoreT(dst + c * kV + e, cur.v[j][e]);
            }
          }
        }
      }
    }
    w = wn;
  }
}

// ---- Host side ------------------------------------------------------------------------------------------------------

uint64_t ElemBytes(uint32_t dt) { return dt == ROOST_DTYPE_BF16 ? 2 : 4; }
bool ActType(uint32_t dt) { return dt == ROOST_DTYPE_BF16 || dt == ROOST_DTYPE_F32; }
uintptr_t Addr(const void* p) { return reinterpret_cast<uintptr_t>(p); }
bool Overlap(const RoostDeviceSpan& x, uint64_t xn, const RoostDeviceSpan& y, uint64_t yn) {
  return Addr(x.address) < Addr(y.address) + yn * ElemBytes(y.dtype) &&
         Addr(y.address) < Addr(x.address) + xn * ElemBytes(x.dtype);
}

// How a row of head_dim elements maps onto lanes: kV elements per chunk (16 / element bytes when every row start is
// 16-byte aligned, else 1), kJ chunks per lane, g lanes per row.
struct RowShape {
  bool vec;
  int kj;  // 1, 2 (vector) or 1, 16 (scalar)
  uint32_t g;
};
uint32_t Pow2AtLeast(uint32_t n) {
  uint32_t p = 1;
  while (p < n) p <<= 1;
  return p;
}
RowShape ShapeFor(uint32_t head_dim, uint32_t elem_bytes, bool aligned16) {
  const uint32_t v = 16 / elem_bytes;
  RowShape s{};
  s.vec = aligned16 && head_dim % v == 0 && head_dim / v <= 128;  // two 16-byte chunks per lane at most
  const uint32_t chunks = s.vec ? head_dim / v : head_dim;
  if (chunks <= 64) {
    s.kj = 1;
    s.g = Pow2AtLeast(chunks);
  } else {
    s.kj = s.vec ? 2 : 16;
    s.g = 64;
  }
  return s;
}
// Every row start base + t * stride + h * head_dim (elements) is 16-byte aligned when these are.
bool RowsAligned16(const void* base, uint64_t stride, uint32_t head_dim, uint32_t elem_bytes) {
  return roost::IsAligned(base, 16) && (stride * elem_bytes) % 16 == 0 && (uint64_t{head_dim} * elem_bytes) % 16 == 0;
}
// Whether the rotation can take whole chunks (vector rows only): interleaved pairs never straddle a chunk when R is a
// multiple of the chunk, NeoX halves pair whole chunks when R/2 is.
uint32_t ChunkPairs(const RowShape& s, uint32_t elem_bytes, uint32_t rot, bool interleaved) {
  const uint32_t v = 16 / elem_bytes;
  if (!s.vec) return 0u;
  return (interleaved ? rot % v == 0 : (rot / 2) % v == 0) ? 1u : 0u;
}
uint32_t Blocks(uint64_t items, uint32_t per) { return static_cast<uint32_t>(roost::CeilDiv(items, per)); }
// Tokens per rope workgroup: about a thousand workgroups for large calls, one token each for small ones.
uint32_t TokensPerBlock(uint32_t tokens) { return std::min<uint32_t>(kMaxTpb, std::max<uint32_t>(1, tokens / 1024)); }
uint32_t GridFor(uint64_t rows, uint32_t g) {
  return static_cast<uint32_t>(roost::CeilDiv(rows, uint64_t{4} * (64 / g)));
}

// Instantiates `launch` for (T, kV, kJ) from the dtype and the row shape.
template <typename F>
void DispatchShape(uint32_t dt, const RowShape& s, F&& launch) {
  auto by_kj = [&](auto t_tag, auto kv_tag) {
    using T = decltype(t_tag);
    constexpr int kV = decltype(kv_tag)::value;
    if constexpr (kV == 1) {
      if (s.kj == 1) launch(T{}, std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{});
      else launch(T{}, std::integral_constant<int, 1>{}, std::integral_constant<int, 16>{});
    } else {
      if (s.kj == 1) launch(T{}, std::integral_constant<int, kV>{}, std::integral_constant<int, 1>{});
      else launch(T{}, std::integral_constant<int, kV>{}, std::integral_constant<int, 2>{});
    }
  };
  if (dt == ROOST_DTYPE_BF16) {
    if (s.vec) by_kj(uint16_t{}, std::integral_constant<int, 8>{});
    else by_kj(uint16_t{}, std::integral_constant<int, 1>{});
  } else {
    if (s.vec) by_kj(float{}, std::integral_constant<int, 4>{});
    else by_kj(float{}, std::integral_constant<int, 1>{});
  }
}

// The rotation's own rules: a known kind, an even rotary width of at most the head, theta > 0, and for Llama 3 a
// positive factor, 0 < low < high and an original context length.
void AdmitRope(roost::Gate& gate, uint32_t head_dim, uint32_t rot, uint32_t kind, float theta, float factor, float low,
               float high, uint32_t orig) {
  gate.Expect(kind == ROOST_ROPE_DEFAULT || kind == ROOST_ROPE_LLAMA3, ROOST_STATUS_INVALID_ARGUMENT,
              "rope kind %u is neither DEFAULT nor LLAMA3", kind)
      .Expect(rot > 0 && rot <= head_dim && rot % 2 == 0, ROOST_STATUS_INVALID_ARGUMENT,
              "rotary width %u: an even width between 2 and head_dim = %u is required", rot, head_dim)
      .Expect(theta > 0.0f, ROOST_STATUS_INVALID_ARGUMENT, "theta = %g; the frequency base must be > 0", theta)
      .Expect(kind != ROOST_ROPE_LLAMA3 || (factor > 0.0f && low > 0.0f && high > low && orig > 0),
              ROOST_STATUS_INVALID_ARGUMENT,
              "Llama 3 scaling with factor %g, low %g, high %g, original length %u; it needs factor > 0, "
              "0 < low < high and a non-zero length", factor, low, high, orig);
}

// A row tensor of the activation type `dt`: the span rules plus natural alignment.
roost::Gate& RowTensor(roost::Gate& gate, const char* name, const RoostDeviceSpan& s, uint32_t dt, uint64_t elems) {
  return gate.Tensor(name, s, dt, elems).Aligned(name, s.address, static_cast<uint32_t>(ElemBytes(dt)));
}

template <typename Params>
const Params* Preamble(roost::Gate& gate, RoostContext* ctx, const void* params) {
  gate.Expect(ctx != nullptr, ROOST_STATUS_INVALID_ARGUMENT, "no context was passed").Header(params, sizeof(Params));
  return gate.ok() ? static_cast<const Params*>(params) : nullptr;
}

}  // namespace

// ---- Entry points ---------------------------------------------------------------------------------------------------

extern "C" ROOST_API RoostStatus roost_qk_norm_run(RoostContext* ctx, const void* params, const RoostWorkspace*,
                                                   void* stream) {
  constexpr char kOp[] = "qk_norm";
  roost::Gate gate(kOp);
  const auto* pp = Preamble<RoostQkNormParams>(gate, ctx, params);
  ROOST_GATE_RETURN(gate);
  const auto& p = *pp;
  return roost::CatchAll(kOp, [&]() -> RoostStatus {
    const uint64_t qrow = uint64_t{p.q_heads} * p.head_dim, krow = uint64_t{p.kv_heads} * p.head_dim;
    const uint64_t qs = p.q_stride == 0 ? qrow : p.q_stride, ks = p.k_stride == 0 ? krow : p.k_stride;
    gate.Expect(p.reserved0 == 0, ROOST_STATUS_INVALID_ARGUMENT, "reserved0 = %u, must be 0", p.reserved0)
        .Expect(p.head_dim > 0 && p.q_heads > 0 && p.kv_heads > 0, ROOST_STATUS_INVALID_ARGUMENT,
                "head_dim = %u, q_heads = %u, kv_heads = %u: each must be positive", p.head_dim, p.q_heads, p.kv_heads)
        .Expect(qs >= qrow && ks >= krow, ROOST_STATUS_INVALID_ARGUMENT,
                "token strides q %llu, k %llu are narrower than their rows of heads (%llu, %llu)",
                static_cast<unsigned long long>(qs), static_cast<unsigned long long>(ks),
                static_cast<unsigned long long>(qrow), static_cast<unsigned long long>(krow));
    ROOST_GATE_RETURN(gate);
    if (p.tokens == 0) return ROOST_STATUS_OK;
    const uint32_t dt = p.q.dtype;
    gate.Expect(ActType(dt), ROOST_STATUS_UNSUPPORTED, "q is %s; built for bf16 and f32", roost::Describe(dt).name)
        .Expect(p.head_dim <= kMaxHeadDim, ROOST_STATUS_UNSUPPORTED, "head_dim = %u exceeds the built maximum of %u",
                p.head_dim, kMaxHeadDim);
    ROOST_GATE_RETURN(gate);
    const uint64_t q_len = (p.tokens - 1ull) * qs + qrow, k_len = (p.tokens - 1ull) * ks + krow;
    const uint64_t rows = uint64_t{p.tokens} * (p.q_heads + p.kv_heads);
    RowTensor(gate, "q", p.q, dt, q_len);
    RowTensor(gate, "k", p.k, dt, k_len);
    RowTensor(gate, "q_weight", p.q_weight, dt, p.head_dim);
    RowTensor(gate, "k_weight", p.k_weight, dt, p.head_dim);
    gate.Expect(rows <= (uint64_t{1} << 40), ROOST_STATUS_INVALID_ARGUMENT, "%llu head rows exceed one launch",
                static_cast<unsigned long long>(rows));
    ROOST_GATE_RETURN(gate);
    const uint32_t eb = static_cast<uint32_t>(ElemBytes(dt));
    const bool a16 = RowsAligned16(p.q.address, qs, p.head_dim, eb) && RowsAligned16(p.k.address, ks, p.head_dim, eb) &&
                     roost::IsAligned(p.q_weight.address, 16) && roost::IsAligned(p.k_weight.address, 16);
    const RowShape s = ShapeFor(p.head_dim, eb, a16);
    DispatchShape(dt, s, [&](auto t_tag, auto kv, auto kj) {
      using T = decltype(t_tag);
      hipLaunchKernelGGL((QkNormKernel<T, decltype(kv)::value, decltype(kj)::value>), dim3(GridFor(rows, s.g)),
                         dim3(256), 0, roost::Stream(stream), static_cast<T*>(p.q.address), static_cast<T*>(p.k.address),
                         static_cast<const T*>(p.q_weight.address), static_cast<const T*>(p.k_weight.address),
                         p.tokens, p.q_heads, p.kv_heads, p.head_dim, qs, ks, p.eps, s.g);
    });
    return roost::HipStatus(hipGetLastError(), kOp, "kernel launch");
  });
}

extern "C" ROOST_API RoostStatus roost_rope_run(RoostContext* ctx, const void* params, const RoostWorkspace*,
                                                void* stream) {
  constexpr char kOp[] = "rope";
  roost::Gate gate(kOp);
  const auto* pp = Preamble<RoostRopeParams>(gate, ctx, params);
  ROOST_GATE_RETURN(gate);
  const auto& p = *pp;
  return roost::CatchAll(kOp, [&]() -> RoostStatus {
    const uint32_t rot = p.rotary_dim == 0 ? p.head_dim : p.rotary_dim;
    gate.Expect(p.kind == ROOST_ROPE_DEFAULT || p.kind == ROOST_ROPE_LLAMA3, ROOST_STATUS_INVALID_ARGUMENT,
                "rope kind %u is neither DEFAULT nor LLAMA3", p.kind)
        .Expect(p.head_dim > 0 && p.q_heads > 0 && p.kv_heads > 0, ROOST_STATUS_INVALID_ARGUMENT,
                "head_dim = %u, q_heads = %u, kv_heads = %u: each must be positive", p.head_dim, p.q_heads, p.kv_heads);
    AdmitRope(gate, p.head_dim, rot, p.kind, p.theta, p.llama3_factor, p.llama3_low_freq_factor,
              p.llama3_high_freq_factor, p.llama3_original_max_position);
    gate.Expect(p.head_dim <= kMaxHeadDim, ROOST_STATUS_UNSUPPORTED, "head_dim = %u exceeds the built maximum of %u",
                p.head_dim, kMaxHeadDim);
    ROOST_GATE_RETURN(gate);
    if (p.tokens == 0) return ROOST_STATUS_OK;
    const uint32_t dt = p.q.dtype;
    gate.Expect(ActType(dt), ROOST_STATUS_UNSUPPORTED, "q is %s; built for bf16 and f32", roost::Describe(dt).name);
    ROOST_GATE_RETURN(gate);
    const uint64_t q_len = uint64_t{p.tokens} * p.q_heads * p.head_dim;
    const uint64_t k_len = uint64_t{p.tokens} * p.kv_heads * p.head_dim;
    const uint64_t rows = uint64_t{p.tokens} * (p.q_heads + p.kv_heads);
    RowTensor(gate, "q", p.q, dt, q_len);
    RowTensor(gate, "k", p.k, dt, k_len);
    gate.Tensor("positions", p.positions, ROOST_DTYPE_I32, p.tokens)
        .Aligned("positions", p.positions.address, 4)
        .Expect(rows <= (uint64_t{1} << 40), ROOST_STATUS_INVALID_ARGUMENT, "%llu head rows exceed one launch",
                static_cast<unsigned long long>(rows));
    ROOST_GATE_RETURN(gate);
    const uint32_t eb = static_cast<uint32_t>(ElemBytes(dt));
    RopeSpec rs{static_cast<const int32_t*>(p.positions.address), rot, p.interleaved != 0u,
                p.kind == ROOST_ROPE_LLAMA3, p.theta, p.llama3_factor, p.llama3_low_freq_factor,
                p.llama3_high_freq_factor, p.llama3_original_max_position, 0u};
    const bool a16 = RowsAligned16(p.q.address, uint64_t{p.q_heads} * p.head_dim, p.head_dim, eb) &&
                     RowsAligned16(p.k.address, uint64_t{p.kv_heads} * p.head_dim, p.head_dim, eb);
    const RowShape s = ShapeFor(p.head_dim, eb, a16);
    rs.chunk_pairs = ChunkPairs(s, eb, rot, p.interleaved != 0u);
    const uint32_t tpb = TokensPerBlock(p.tokens);
    DispatchShape(dt, s, [&](auto t_tag, auto kv, auto kj) {
      using T = decltype(t_tag);
      hipLaunchKernelGGL((RopeKernel<T, decltype(kv)::value, decltype(kj)::value>), dim3(Blocks(p.tokens, tpb)),
                         dim3(256), RopeLdsBytes(rot / 2, tpb, s.g, p.head_dim), roost::Stream(stream),
                         static_cast<T*>(p.q.address), static_cast<T*>(p.k.address), rs, p.tokens, p.q_heads,
                         p.kv_heads, p.head_dim, s.g, tpb);
    });
    return roost::HipStatus(hipGetLastError(), kOp, "kernel launch");
  });
}

extern "C" ROOST_API RoostStatus roost_qkv_qk_norm_rope_cache_write_run(RoostContext* ctx, const void* params,
                                                                        const RoostWorkspace*, void* stream) {
  constexpr char kOp[] = "qkv_qk_norm_rope_cache_write";
  roost::Gate gate(kOp);
  const auto* pp = Preamble<RoostQkvQkNormRopeCacheWriteParams>(gate, ctx, params);
  ROOST_GATE_RETURN(gate);
  const auto& p = *pp;
  return roost::CatchAll(kOp, [&]() -> RoostStatus {
    gate.Expect(p.reserved0 == 0, ROOST_STATUS_INVALID_ARGUMENT, "reserved0 = %u, must be 0", p.reserved0)
        .Expect(p.head_dim > 0 && p.q_heads > 0 && p.kv_heads > 0 && p.page_size > 0, ROOST_STATUS_INVALID_ARGUMENT,
                "head_dim = %u, q_heads = %u, kv_heads = %u, page_size = %u: each must be positive", p.head_dim,
                p.q_heads, p.kv_heads, p.page_size);
    AdmitRope(gate, p.head_dim, p.head_dim, ROOST_ROPE_DEFAULT, p.theta, 0.0f, 0.0f, 0.0f, 0);
    ROOST_GATE_RETURN(gate);
    if (p.tokens == 0) return ROOST_STATUS_OK;
    const uint32_t dt = p.qkv.dtype, ct = p.k_cache.dtype;
    gate.Expect(ActType(dt), ROOST_STATUS_UNSUPPORTED, "qkv is %s; built for bf16 and f32", roost::Describe(dt).name)
        .Expect(ct == dt || (dt == ROOST_DTYPE_BF16 && ct == ROOST_DTYPE_F32), ROOST_STATUS_UNSUPPORTED,
                "%s pages under %s rows: pages hold the row type, or f32 under bf16 rows", roost::Describe(ct).name,
                roost::Describe(dt).name)
        .Expect(p.head_dim <= kMaxHeadDim, ROOST_STATUS_UNSUPPORTED, "head_dim = %u exceeds the built maximum of %u",
                p.head_dim, kMaxHeadDim);
    ROOST_GATE_RETURN(gate);
    const uint64_t qw = uint64_t{p.q_heads} * p.head_dim, kw = uint64_t{p.kv_heads} * p.head_dim;
    const uint64_t row = qw + 2 * kw, tokens = p.tokens;
    RowTensor(gate, "qkv", p.qkv, dt, tokens * row);
    RowTensor(gate, "q", p.q, dt, tokens * qw);
    RowTensor(gate, "q_weight", p.q_weight, dt, p.head_dim);
    RowTensor(gate, "k_weight", p.k_weight, dt, p.head_dim);
    RowTensor(gate, "k_cache", p.k_cache, ct, kw);
    RowTensor(gate, "v_cache", p.v_cache, ct, kw);
    gate.Tensor("positions", p.positions, ROOST_DTYPE_I32, tokens)
        .Aligned("positions", p.positions.address, 4)
        .Tensor("slot_mapping", p.slot_mapping, ROOST_DTYPE_I64, tokens)
        .Aligned("slot_mapping", p.slot_mapping.address, 8);
    ROOST_GATE_RETURN(gate);
    const uint64_t kc_len = p.k_cache.length, vc_len = p.v_cache.length;
    const bool clash = Overlap(p.q, tokens * qw, p.qkv, tokens * row) || Overlap(p.q, tokens * qw, p.k_cache, kc_len) ||
                       Overlap(p.q, tokens * qw, p.v_cache, vc_len) || Overlap(p.qkv, tokens * row, p.k_cache, kc_len) ||
                       Overlap(p.qkv, tokens * row, p.v_cache, vc_len) || Overlap(p.k_cache, kc_len, p.v_cache, vc_len);
    const uint64_t rows = tokens * (p.q_heads + 2ull * p.kv_heads);
    gate.Expect(!clash, ROOST_STATUS_INVALID_ARGUMENT,
                "q, qkv, k_cache and v_cache must be four disjoint buffers (the op is never computed in place)")
        .Expect(rows <= (uint64_t{1} << 40), ROOST_STATUS_INVALID_ARGUMENT, "%llu head rows exceed one launch",
                static_cast<unsigned long long>(rows));
    ROOST_GATE_RETURN(gate);
    const uint32_t eb = static_cast<uint32_t>(ElemBytes(dt)), cb = static_cast<uint32_t>(ElemBytes(ct));
    QkvArgs a{p.qkv.address, p.q.address, p.q_weight.address, p.k_weight.address, p.k_cache.address,
              p.v_cache.address, static_cast<const int64_t*>(p.slot_mapping.address), std::min(kc_len, vc_len) / kw,
              p.tokens, p.q_heads, p.kv_heads, p.head_dim, p.eps};
    RopeSpec rs{static_cast<const int32_t*>(p.positions.address), p.head_dim, 0u, 0u, p.theta, 0.0f, 0.0f, 0.0f, 0u, 0u};
    // 16-byte rows need every row start aligned: qkv rows, q rows, cache rows and the weights.
    const bool a16 = RowsAligned16(p.qkv.address, row, p.head_dim, eb) && RowsAligned16(p.q.address, qw, p.head_dim, eb) &&
                     RowsAligned16(p.k_cache.address, kw, p.head_dim, cb) &&
                     RowsAligned16(p.v_cache.address, kw, p.head_dim, cb) && roost::IsAligned(p.q_weight.address, 16) &&
                     roost::IsAligned(p.k_weight.address, 16);
    const RowShape s = ShapeFor(p.head_dim, eb, a16);
    rs.chunk_pairs = ChunkPairs(s, eb, p.head_dim, false);
    const bool widen = ct != dt;
    const uint32_t tpb = TokensPerBlock(p.tokens);
    const dim3 grid(Blocks(p.tokens, tpb));
    const uint64_t lds = RopeLdsBytes(p.head_dim / 2, tpb, s.g, p.head_dim);
    DispatchShape(dt, s, [&](auto t_tag, auto kv, auto kj) {
      using T = decltype(t_tag);
      constexpr int kV = decltype(kv)::value, kJ = decltype(kj)::value;
      if (widen) {
        if constexpr (sizeof(T) == 2) {
          hipLaunchKernelGGL((QkvKernel<T, float, kV, kJ>), grid, dim3(256), lds, roost::Stream(stream), a, rs, s.g, tpb);
        }
      } else {
        hipLaunchKernelGGL((QkvKernel<T, T, kV, kJ>), grid, dim3(256), lds, roost::Stream(stream), a, rs, s.g, tpb);
      }
    });
    return roost::HipStatus(hipGetLastError(), kOp, "kernel launch");
  });
}
