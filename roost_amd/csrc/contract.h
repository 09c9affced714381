// Host-side admission of C-ABI calls for the gfx950 Roost kernel library. Not part of the C ABI.
//
// Every entry point admits its call through a Gate before it touches the device: the gate walks the call's rules in
// order and the first broken rule decides the call's RoostStatus, whose message the caller reads back through
// roost_last_error(). The rules themselves are the contract of kernels/include/roost_kernels.h (ABI 1.3): a params
// struct must be at least as large as this library's and no newer than its minor (ABI_MISMATCH); device spans carry a
// dtype, an element count and a reserved word that must be zero; shapes the kernels do not cover are UNSUPPORTED;
// malformed calls are INVALID_ARGUMENT. No C++ exception may reach the caller: CatchAll turns one into INTERNAL.
//
// Messages name the op, the offending field and the value seen, e.g.
//   "paged_attention: head_dim = 96 has no kernel here (built: 64, 128, 256)".
#ifndef ROOST_AMD_CONTRACT_H_
#define ROOST_AMD_CONTRACT_H_

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <exception>
#include <string>

#include "../../include/roost_amd.h"
#include "../../include/roost_kernels.h"

void roost_set_error(const char* message);

namespace roost {

// ---- Dtypes -----------------------------------------------------------------------------------------------------------

// Bit `dtype` of a constraints dtype mask.
constexpr uint64_t DtypeMask(uint32_t dtype) { return uint64_t{1} << dtype; }

struct DtypeInfo {
  const char* name;
  uint32_t bytes;  // 0 for sub-byte and undefined types
};

inline DtypeInfo Describe(uint32_t dtype) {
  static constexpr DtypeInfo kTable[ROOST_DTYPE_COUNT] = {
      {"undefined", 0}, {"f32", 4}, {"f16", 2},  {"bf16", 2}, {"f64", 8}, {"f8e4m3", 1},
      {"f8e5m2", 1},    {"i8", 1},  {"u8", 1},   {"i16", 2},  {"i32", 4}, {"u32", 4},
      {"i64", 8},       {"u64", 8}, {"i4", 0},   {"u4", 0},   {"f4e2m1", 0}};
  return dtype < ROOST_DTYPE_COUNT ? kTable[dtype] : DtypeInfo{"unknown", 0};
}

inline uint32_t ElementBytes(uint32_t dtype) { return Describe(dtype).bytes; }

// ---- Small arithmetic -------------------------------------------------------------------------------------------------

inline bool IsAligned(const void* p, uint64_t bytes) { return reinterpret_cast<uintptr_t>(p) % bytes == 0; }
constexpr uint64_t RoundUp(uint64_t v, uint64_t multiple) { return (v + multiple - 1) / multiple * multiple; }
constexpr uint64_t CeilDiv(uint64_t a, uint64_t b) { return (a + b - 1) / b; }
constexpr bool IsPow2(uint64_t v) { return v != 0 && (v & (v - 1)) == 0; }

inline hipStream_t Stream(void* s) { return static_cast<hipStream_t>(s); }

// ---- Reporting --------------------------------------------------------------------------------------------------------

// Formats "<op>: <detail>" into the calling thread's last-error slot and returns `status`.
inline RoostStatus Report(RoostStatus status, const char* op, const char* fmt, ...) __attribute__((format(printf, 3, 4)));
inline RoostStatus Report(RoostStatus status, const char* op, const char* fmt, ...) {
  char detail[384];
  va_list args;
  va_start(args, fmt);
  std::vsnprintf(detail, sizeof detail, fmt, args);
  va_end(args);
  roost_set_error((std::string(op) + ": " + detail).c_str());
  return status;
}

// A HIP runtime error as ROOST_STATUS_CUDA_ERROR (the ABI's name for any GPU runtime failure).
inline RoostStatus HipStatus(hipError_t err, const char* op, const char* step) {
  if (err == hipSuccess) return ROOST_STATUS_OK;
  return Report(ROOST_STATUS_CUDA_ERROR, op, "%s failed in the HIP runtime: %s", step, hipGetErrorString(err));
}

// ---- The gate ---------------------------------------------------------------------------------------------------------

class Gate {
 public:
  explicit Gate(const char* op) : op_(op) {}

  bool ok() const { return status_ == ROOST_STATUS_OK; }
  RoostStatus status() const { return status_; }
  const char* op() const { return op_; }

  // The rule holds, or the call is refused with `status` and the formatted reason. Once a rule has failed, later
  // rules are not evaluated further (their arguments are, so a rule must not dereference what an earlier one guards:
  // split such chains with `if (!gate.ok()) return gate.status();`).
  Gate& Expect(bool holds, RoostStatus status, const char* fmt, ...) __attribute__((format(printf, 4, 5))) {
    if (!ok() || holds) return *this;
    char detail[384];
    va_list args;
    va_start(args, fmt);
    std::vsnprintf(detail, sizeof detail, fmt, args);
    va_end(args);
    status_ = Report(status, op_, "%s", detail);
    return *this;
  }

  // The leading (struct_size, abi_minor) words of a params struct.
  Gate& Header(const void* params, uint32_t this_size) {
    if (!ok()) return *this;
    if (params == nullptr) return Expect(false, ROOST_STATUS_INVALID_ARGUMENT, "no params struct was passed");
    const auto* words = static_cast<const uint32_t*>(params);
    return Expect(words[0] >= this_size && words[1] <= ROOST_ABI_MINOR, ROOST_STATUS_ABI_MISMATCH,
                  "params struct of %u bytes at ABI minor %u; this library reads %u bytes at minor <= %u", words[0],
                  words[1], this_size, static_cast<uint32_t>(ROOST_ABI_MINOR));
  }

  // A device span the op reads or writes: zero reserved word, the dtype the op computes in, an address whenever
  // elements are needed, and room for `elements`.
  Gate& Tensor(const char* name, const RoostDeviceSpan& s, uint32_t dtype, uint64_t elements) {
    if (!ok()) return *this;
    Expect(s.reserved0 == 0, ROOST_STATUS_INVALID_ARGUMENT, "%s: reserved word is %u, must be 0", name, s.reserved0);
    Expect(s.dtype == dtype, ROOST_STATUS_INVALID_ARGUMENT, "%s: dtype %s where %s is required", name,
           Describe(s.dtype).name, Describe(dtype).name);
    Expect(elements == 0 || s.address != nullptr, ROOST_STATUS_INVALID_ARGUMENT, "%s: address is NULL", name);
    return Expect(s.length >= elements, ROOST_STATUS_INVALID_ARGUMENT,
                  "%s: %llu elements given, the shape needs %llu", name, static_cast<unsigned long long>(s.length),
                  static_cast<unsigned long long>(elements));
  }

  // As Tensor, for a span the op may go without: a NULL address means "not wanted".
  Gate& OptionalTensor(const char* name, const RoostDeviceSpan& s, uint32_t dtype, uint64_t elements) {
    if (!ok()) return *this;
    if (s.address == nullptr) {
      return Expect(s.reserved0 == 0, ROOST_STATUS_INVALID_ARGUMENT, "%s: reserved word is %u, must be 0", name,
                    s.reserved0);
    }
    return Tensor(name, s, dtype, elements);
  }

  Gate& Aligned(const char* name, const void* p, uint32_t bytes) {
    return Expect(IsAligned(p, bytes), ROOST_STATUS_INVALID_ARGUMENT, "%s: address %p is not %u-byte aligned", name, p,
                  bytes);
  }

 private:
  const char* op_;
  RoostStatus status_ = ROOST_STATUS_OK;
};

// Returns from the enclosing function when the gate has refused the call.
#define ROOST_GATE_RETURN(gate)                  \
  do {                                           \
    if (!(gate).ok()) return (gate).status();    \
  } while (0)

// Returns from the enclosing function on any status other than OK.
#define ROOST_RETURN_IF_FAILED(expr)                 \
  do {                                               \
    const RoostStatus roost_status_ = (expr);        \
    if (roost_status_ != ROOST_STATUS_OK) return roost_status_; \
  } while (0)

// Runs `body`; an exception that escapes it becomes ROOST_STATUS_INTERNAL with its text.
template <typename Body>
RoostStatus CatchAll(const char* op, Body&& body) noexcept {
  try {
    return body();
  } catch (const std::exception& e) {
    return Report(ROOST_STATUS_INTERNAL, op, "internal error: %s", e.what());
  } catch (...) {
    return Report(ROOST_STATUS_INTERNAL, op, "internal error of unknown type");
  }
}

// The device region of a workspace: present, large enough for `bytes`, aligned to `align`.
inline bool HasDeviceRegion(const RoostWorkspace* ws, uint64_t bytes, uint64_t align = 256) {
  if (bytes == 0) return true;
  return ws != nullptr && ws->device != nullptr && ws->device_bytes >= bytes && IsAligned(ws->device, align);
}

}  // namespace roost

#endif  // ROOST_AMD_CONTRACT_H_
