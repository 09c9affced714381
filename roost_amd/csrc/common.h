// Internal helpers shared by the translation units of the gfx950 Roost kernel library. Not part of the C ABI.
// Host-side admission of calls (statuses, messages, span rules) lives in contract.h; this file adds the per-device
// context and the device-side element helpers.
#ifndef ROOST_AMD_COMMON_H_
#define ROOST_AMD_COMMON_H_

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "contract.h"

// Per-library, per-device state. The gfx950 kernels need no handles or loaded modules; the context records the
// device, the creation flags and the device's compute-unit count (the decode planner sizes its grid to it).
struct RoostContext {
  int32_t device;
  uint32_t flags;
  uint32_t compute_units;
};

// ---- Device-side helpers -------------------------------------------------------------------------------------------

namespace roost_dev {

// bf16 <-> f32. bf16 is the top half of an IEEE binary32; widening is exact. Narrowing rounds to nearest, ties to
// even, and maps any NaN to the quiet NaN 0x7FC0 (the same bit pattern CpuElements.ToBFloat16 stores for NaN).
__device__ __forceinline__ float Bf16ToF32(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }
__device__ __forceinline__ float Bf16LoToF32(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float Bf16HiToF32(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

__device__ __forceinline__ uint16_t F32ToBf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ uint32_t PackBf16(float lo, float hi) {
  return static_cast<uint32_t>(F32ToBf16(lo)) | (static_cast<uint32_t>(F32ToBf16(hi)) << 16);
}

// Two floats to packed bf16 with gfx950's v_cvt_pk_bf16_f32: round to nearest, ties to even, as F32ToBf16 does, in one
// instruction instead of a dozen. Only a NaN may come out with other NaN bits than F32ToBf16's 0x7FC0.
__device__ __forceinline__ uint32_t PackBf16Rne(float lo, float hi) {
  typedef float F2 __attribute__((ext_vector_type(2)));
  typedef __bf16 B2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((F2){lo, hi}, B2));
}

// An element of a span whose type (bf16 or f32) is chosen at run time; the branch is uniform across a launch.
__device__ __forceinline__ float LoadF(const void* p, uint32_t dt, int64_t i) {
  return dt == ROOST_DTYPE_BF16 ? Bf16ToF32(static_cast<const uint16_t*>(p)[i]) : static_cast<const float*>(p)[i];
}

// sigmoid with the hardware reciprocal (v_rcp_f32, about 1 ulp) instead of a full-precision divide.
__device__ __forceinline__ float SigmoidF(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
// SiLU, x * sigmoid(x), with the same reciprocal; the conv and gated-norm kernels and the fused GDN layer share it.
__device__ __forceinline__ float SiluF(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// SigmoidMul's arithmetic (CpuOps.Gating.cs, out = x * sigmoid(gate)): each element in fp32, rounded once to the
// element type. The SigmoidMul op and the attention kernels' gated epilogue both use these, so the fused and the
// separate calls agree bit for bit.
__device__ __forceinline__ uint32_t GateMulBf16x2(uint32_t x, uint32_t g) {
  return PackBf16Rne(Bf16LoToF32(x) * SigmoidF(Bf16LoToF32(g)), Bf16HiToF32(x) * SigmoidF(Bf16HiToF32(g)));
}
__device__ __forceinline__ uint16_t GateMul(uint16_t x, uint16_t g) {
  return static_cast<uint16_t>(GateMulBf16x2(x, g));
}
__device__ __forceinline__ float GateMul(float x, float g) { return x * SigmoidF(g); }

// GatedDeltaRuleGates for one (token, value head) (CpuOps.Gating.cs): g = -exp(a_log) * softplus(a + dt_bias), with
// softplus(x) = x above 20, and beta = sigmoid(b), in fp32. The gates op stores these; the GDN kernels' fused-gates
// path uses them directly, so both paths compute bit-identical values.
__device__ __forceinline__ void GateValues(float a, float dt_bias, float a_log, float b, float& g, float& beta) {
  const float x = a + dt_bias;
  const float sp = x > 20.0f ? x : log1pf(__expf(x));
  g = -__expf(a_log) * sp;
  beta = SigmoidF(b);
}

}  // namespace roost_dev

#endif  // ROOST_AMD_COMMON_H_
