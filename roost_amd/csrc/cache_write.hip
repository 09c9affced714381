// CacheWrite (ROOST_OP_CACHE_WRITE) for gfx950: new K and V rows scattered into the paged pools at slot_mapping.
//
// Semantics (reference: src/Starlings.Roost.Ops/CpuOps.cs:515-555 and kernels/src/m0_ops.cu:362-429): token t with
// slot s >= 0 goes to page s / page_size, offset s % page_size; row (page*page_size + offset)*kv_heads + h in an NHD
// pool, ((page*kv_heads + h)*page_size + offset) in an HND pool; the bytes are copied unchanged (cache dtype ==
// activation dtype; quantised KV is refused). A negative slot skips the token; a slot past the end of the pool is
// skipped on the device rather than faulting, because slots are device data and are not range-checked on the host.
//
// Design: the copy is pure HBM traffic (2 * tokens * kv_heads * head_dim * elem bytes each way). One work item moves
// one 16-byte vector of one head row (the common case: head rows are multiples of 16 bytes and the buffers are
// 16-byte aligned) or one 16-bit word otherwise, so consecutive lanes touch consecutive bytes of a row on both sides.

#include "common.h"

namespace {

template <typename W>
__global__ void __launch_bounds__(256) CacheWriteKernel(const W* __restrict__ k, const W* __restrict__ v,
                                                        W* __restrict__ k_cache, W* __restrict__ v_cache,
                                                        const int64_t* __restrict__ slots, uint64_t pool_rows,
                                                        uint32_t kv_heads, uint32_t words_per_head, uint32_t page_size,
                                                        uint32_t hnd, uint64_t total_words) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total_words) return;
  const uint64_t words_per_token = static_cast<uint64_t>(kv_heads) * words_per_head;
  const uint64_t token = i / words_per_token;
  const uint64_t rem = i - token * words_per_token;
  const int64_t slot = slots[token];
  if (slot < 0) return;
  const uint64_t page = static_cast<uint64_t>(slot) / page_size;
  const uint64_t off = static_cast<uint64_t>(slot) - page * page_size;
  if (page * page_size + off >= pool_rows) return;
  const uint64_t h = rem / words_per_head;
  const uint64_t w = rem - h * words_per_head;
  const uint64_t row = hnd ? (page * kv_heads + h) * page_size + off : (page * page_size + off) * kv_heads + h;
  const uint64_t dst = row * words_per_head + w;
  k_cache[dst] = k[i];
  v_cache[dst] = v[i];
}

}  // namespace

extern "C" ROOST_API RoostStatus roost_cache_write_run(RoostContext*, const void* params, const RoostWorkspace*,
                                                       void* stream) {
  using namespace roost;
  constexpr char kOp[] = "CacheWrite";
  ROOST_TRY(CheckHeader(params, sizeof(RoostCacheWriteParams), kOp));
  const auto& p = *static_cast<const RoostCacheWriteParams*>(params);
  return Guarded(kOp, [&]() -> RoostStatus {
    if (p.reserved0 != 0) return Fail(ROOST_STATUS_INVALID_ARGUMENT, "CacheWrite: reserved0 must be zero");
    if (p.kv_layout != ROOST_LAYOUT_PAGED_NHD && p.kv_layout != ROOST_LAYOUT_PAGED_HND) {
      return Fail(ROOST_STATUS_INVALID_ARGUMENT, "CacheWrite: kv_layout must be PAGED_NHD or PAGED_HND");
    }
    if (p.kv_heads == 0 || p.head_dim == 0 || p.page_size == 0) {
      return Fail(ROOST_STATUS_INVALID_ARGUMENT, "CacheWrite: kv_heads, head_dim and page_size must be non-zero");
    }
    const uint32_t dt = p.k.dtype;
    if (dt != ROOST_DTYPE_BF16 && dt != ROOST_DTYPE_F16 && dt != ROOST_DTYPE_F32) {
      return Fail(ROOST_STATUS_UNSUPPORTED, "CacheWrite: k dtype must be bf16, f16 or f32");
    }
    if (p.v.dtype != dt || p.k_cache.dtype != dt || p.v_cache.dtype != dt) {
      return Fail(ROOST_STATUS_UNSUPPORTED, "CacheWrite: quantised KV (cache dtype != activation dtype) is not built");
    }
    if (p.k_scale != 1.0f || p.v_scale != 1.0f) {
      return Fail(ROOST_STATUS_UNSUPPORTED, "CacheWrite: k_scale and v_scale must be 1 without quantised KV");
    }
    if (p.tokens == 0) return ROOST_STATUS_OK;
    const uint64_t per_token = static_cast<uint64_t>(p.kv_heads) * p.head_dim;
    ROOST_TRY(CheckSpan(p.k, dt, p.tokens * per_token, kOp, "k"));
    ROOST_TRY(CheckSpan(p.v, dt, p.tokens * per_token, kOp, "v"));
    ROOST_TRY(CheckSpan(p.k_cache, dt, per_token, kOp, "k_cache"));
    ROOST_TRY(CheckSpan(p.v_cache, dt, per_token, kOp, "v_cache"));
    ROOST_TRY(CheckSpan(p.slot_mapping, ROOST_DTYPE_I64, p.tokens, kOp, "slot_mapping"));
    if (!Aligned(p.k.address, 2) || !Aligned(p.v.address, 2) || !Aligned(p.k_cache.address, 2) ||
        !Aligned(p.v_cache.address, 2) || !Aligned(p.slot_mapping.address, 8)) {
      return Fail(ROOST_STATUS_INVALID_ARGUMENT, "CacheWrite: k, v and the pools must be 2-byte aligned, slots 8-byte");
    }
    const uint64_t pool_rows = std::min(p.k_cache.length, p.v_cache.length) / per_token;
    const uint64_t head_bytes = static_cast<uint64_t>(p.head_dim) * DtypeBytes(dt);
    const bool vec16 = head_bytes % 16 == 0 && Aligned(p.k.address, 16) && Aligned(p.v.address, 16) &&
                       Aligned(p.k_cache.address, 16) && Aligned(p.v_cache.address, 16);
    const uint32_t word = vec16 ? 16 : 2;
    const uint32_t words_per_head = static_cast<uint32_t>(head_bytes / word);
    const uint64_t total = static_cast<uint64_t>(p.tokens) * p.kv_heads * words_per_head;
    const uint64_t blocks = CeilDiv(total, 256);
    if (blocks > 0x7FFFFFFFull) return Fail(ROOST_STATUS_INVALID_ARGUMENT, "CacheWrite: too many tokens for one call");
    const auto* slots = static_cast<const int64_t*>(p.slot_mapping.address);
    const uint32_t hnd = p.kv_layout == ROOST_LAYOUT_PAGED_HND ? 1u : 0u;
    if (vec16) {
      hipLaunchKernelGGL(CacheWriteKernel<uint4>, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, Stream(stream),
                         static_cast<const uint4*>(p.k.address), static_cast<const uint4*>(p.v.address),
                         static_cast<uint4*>(p.k_cache.address), static_cast<uint4*>(p.v_cache.address), slots,
                         pool_rows, p.kv_heads, words_per_head, p.page_size, hnd, total);
    } else {
      hipLaunchKernelGGL(CacheWriteKernel<uint16_t>, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, Stream(stream),
                         static_cast<const uint16_t*>(p.k.address), static_cast<const uint16_t*>(p.v.address),
                         static_cast<uint16_t*>(p.k_cache.address), static_cast<uint16_t*>(p.v_cache.address), slots,
                         pool_rows, p.kv_heads, words_per_head, p.page_size, hnd, total);
    }
    return FromHip(hipGetLastError(), "CacheWrite launch");
  });
}
