// Internal helpers shared by the translation units of the gfx950 Roost kernel library. Not part of the C ABI.
//
// Validation follows the contract's rules (reference: kernels/src/op_common.h:55-103): a params struct smaller than
// this library needs, or from a newer minor, is an ABI mismatch; spans are checked for dtype, reserved field, NULL
// address and length; no exception ever crosses the C ABI; a failing call leaves its message in roost_last_error().
#ifndef ROOST_AMD_COMMON_H_
#define ROOST_AMD_COMMON_H_

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <exception>
#include <string>

#include "../../include/roost_amd.h"
#include "../../include/roost_kernels.h"

// Per-library, per-device state. The gfx950 kernels need no handles or loaded modules; the context records the
// device, the creation flags and the device's compute-unit count (the decode planner sizes its grid to it).
struct RoostContext {
  int32_t device;
  uint32_t flags;
  uint32_t compute_units;
};

void roost_set_error(const char* message);

namespace roost {

constexpr uint64_t DtypeBit(uint32_t dtype) { return uint64_t{1} << dtype; }

inline uint32_t DtypeBytes(uint32_t dtype) {
  switch (dtype) {
    case ROOST_DTYPE_F64:
    case ROOST_DTYPE_I64:
    case ROOST_DTYPE_U64: return 8;
    case ROOST_DTYPE_F32:
    case ROOST_DTYPE_I32:
    case ROOST_DTYPE_U32: return 4;
    case ROOST_DTYPE_F16:
    case ROOST_DTYPE_BF16:
    case ROOST_DTYPE_I16: return 2;
    case ROOST_DTYPE_I8:
    case ROOST_DTYPE_U8:
    case ROOST_DTYPE_F8E4M3:
    case ROOST_DTYPE_F8E5M2: return 1;
    default: return 0;
  }
}

inline RoostStatus Fail(RoostStatus status, const std::string& message) {
  roost_set_error(message.c_str());
  return status;
}

inline RoostStatus FromHip(hipError_t err, const char* what) {
  if (err == hipSuccess) return ROOST_STATUS_OK;
  std::string m = std::string(what) + ": " + hipGetErrorString(err);
  roost_set_error(m.c_str());
  return ROOST_STATUS_CUDA_ERROR;
}

// The leading (struct_size, abi_minor) pair of every params struct.
inline RoostStatus CheckHeader(const void* params, uint32_t needed, const char* op) {
  if (params == nullptr) return Fail(ROOST_STATUS_INVALID_ARGUMENT, std::string(op) + ": params is NULL");
  const auto* h = static_cast<const uint32_t*>(params);
  if (h[0] < needed || h[1] > ROOST_ABI_MINOR) {
    return Fail(ROOST_STATUS_ABI_MISMATCH,
                std::string(op) + ": params struct_size or abi_minor is not supported by this library");
  }
  return ROOST_STATUS_OK;
}

// A span the op reads or writes: reserved field zero, the expected dtype, non-NULL when it must hold elements, and at
// least `elements` long. An optional span may be NULL (then it is unused).
inline RoostStatus CheckSpan(const RoostDeviceSpan& s, uint32_t dtype, uint64_t elements, const char* op,
                             const char* name, bool optional = false) {
  if (s.reserved0 != 0) return Fail(ROOST_STATUS_INVALID_ARGUMENT, std::string(op) + ": " + name + ".reserved0 must be zero");
  if (optional && s.address == nullptr) return ROOST_STATUS_OK;
  if (s.dtype != dtype) return Fail(ROOST_STATUS_INVALID_ARGUMENT, std::string(op) + ": " + name + " has an unexpected dtype");
  if (elements > 0 && s.address == nullptr) {
    return Fail(ROOST_STATUS_INVALID_ARGUMENT, std::string(op) + ": " + name + " has a NULL address");
  }
  if (s.length < elements) {
    return Fail(ROOST_STATUS_INVALID_ARGUMENT, std::string(op) + ": " + name + " is shorter than the shape needs");
  }
  return ROOST_STATUS_OK;
}

inline bool Aligned(const void* p, uint64_t bytes) { return reinterpret_cast<uintptr_t>(p) % bytes == 0; }
constexpr uint64_t AlignUp(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }
constexpr uint64_t CeilDiv(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

inline hipStream_t Stream(void* s) { return static_cast<hipStream_t>(s); }

// Runs `body`, turning an escaping C++ exception into ROOST_STATUS_INTERNAL.
template <typename F>
RoostStatus Guarded(const char* op, F&& body) {
  try {
    return body();
  } catch (const std::exception& e) {
    return Fail(ROOST_STATUS_INTERNAL, std::string(op) + ": " + e.what());
  } catch (...) {
    return Fail(ROOST_STATUS_INTERNAL, std::string(op) + ": unknown exception");
  }
}

// Workspace check shared by the ops: a workspace pointer with a device region of at least `bytes`.
inline bool DeviceWorkspaceOk(const RoostWorkspace* ws, uint64_t bytes, uint64_t align = 256) {
  if (bytes == 0) return true;
  return ws != nullptr && ws->device != nullptr && ws->device_bytes >= bytes && Aligned(ws->device, align);
}

}  // namespace roost

#define ROOST_TRY(expr)                       \
  do {                                        \
    const RoostStatus roost_s_ = (expr);      \
    if (roost_s_ != ROOST_STATUS_OK) return roost_s_; \
  } while (0)

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

}  // namespace roost_dev

#endif  // ROOST_AMD_COMMON_H_
