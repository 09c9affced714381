// CacheWrite (ROOST_OP_CACHE_WRITE) for gfx950: new K and V rows scattered into the paged pools at slot_mapping.
//
// Semantics (reference: src/Starlings.Roost.Ops/CpuOps.cs:515-555; the GPU op it replaces is
// kernels/src/m0_ops.cu:362-429): token t with slot s >= 0 goes to page s / page_size, offset s % page_size; head h of
// that token lands in head row (page*page_size + offset)*kv_heads + h of an NHD pool or (page*kv_heads + h)*page_size +
// offset of an HND pool, and its bytes are copied unchanged (cache dtype == activation dtype). A negative slot skips
// the token. Slots are device data and are never range-checked on the host, so a head row that would land past the end
// of either pool is skipped on the device instead of being written out of bounds -- for both layouts the bound is the
// pool's own length in head rows.
//
// Design: pure HBM traffic (2 * tokens * kv_heads * head_dim * elem bytes each way). A work item moves one 16-byte
// vector of one head row (head rows that are multiples of 16 bytes with 16-byte aligned buffers) or one 16-bit word
// otherwise, so consecutive lanes touch consecutive bytes of a row on both sides.

#include "common.h"

namespace {

template <typename W>
__global__ void __launch_bounds__(256) CacheWriteKernel(const W* __restrict__ k, const W* __restrict__ v,
                                                        W* __restrict__ k_cache, W* __restrict__ v_cache,
                                                        const int64_t* __restrict__ slots, uint64_t pool_head_rows,
                                                        uint32_t kv_heads, uint32_t words_per_head, uint32_t page_size,
                                                        uint32_t hnd, uint64_t total_words) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total_words) return;
  const uint64_t words_per_token = static_cast<uint64_t>(kv_heads) * words_per_head;
  const uint64_t token = i / words_per_token;
  const uint64_t within = i - token * words_per_token;
  const int64_t slot = slots[token];
  if (slot < 0) return;
  const uint64_t page = static_cast<uint64_t>(slot) / page_size;
  const uint64_t off = static_cast<uint64_t>(slot) % page_size;
  const uint64_t h = within / words_per_head;
  const uint64_t row = hnd ? (page * kv_heads + h) * page_size + off : (page * page_size + off) * kv_heads + h;
  if (row >= pool_head_rows) return;
  const uint64_t dst = row * words_per_head + (within - h * words_per_head);
  k_cache[dst] = k[i];
  v_cache[dst] = v[i];
}

// The call's rules (reference contract: kernels/src/m0_ops.cu:395-429 refuses the same cases with the same statuses).
RoostStatus Admit(const RoostCacheWriteParams& p) {
  roost::Gate gate("cache_write");
  gate.Expect(p.reserved0 == 0, ROOST_STATUS_INVALID_ARGUMENT, "reserved0 = %u, must be 0", p.reserved0)
      .Expect(p.kv_layout == ROOST_LAYOUT_PAGED_NHD || p.kv_layout == ROOST_LAYOUT_PAGED_HND,
              ROOST_STATUS_INVALID_ARGUMENT, "kv_layout = %u is not a paged layout (NHD or HND)", p.kv_layout)
      .Expect(p.kv_heads > 0 && p.head_dim > 0 && p.page_size > 0, ROOST_STATUS_INVALID_ARGUMENT,
              "kv_heads = %u, head_dim = %u, page_size = %u: each must be positive", p.kv_heads, p.head_dim,
              p.page_size);
  const uint32_t dt = p.k.dtype;
  gate.Expect(dt == ROOST_DTYPE_BF16 || dt == ROOST_DTYPE_F16 || dt == ROOST_DTYPE_F32, ROOST_STATUS_UNSUPPORTED,
              "k is %s; the copy is built for bf16, f16 and f32 rows", roost::Describe(dt).name)
      .Expect(p.v.dtype == dt && p.k_cache.dtype == dt && p.v_cache.dtype == dt, ROOST_STATUS_UNSUPPORTED,
              "k %s, v %s, k_cache %s, v_cache %s: a quantising write (cache type != row type) has no kernel here",
              roost::Describe(dt).name, roost::Describe(p.v.dtype).name, roost::Describe(p.k_cache.dtype).name,
              roost::Describe(p.v_cache.dtype).name)
      .Expect(p.k_scale == 1.0f && p.v_scale == 1.0f, ROOST_STATUS_UNSUPPORTED,
              "k_scale = %g, v_scale = %g: scales other than 1 belong to quantised caches", p.k_scale, p.v_scale);
  ROOST_GATE_RETURN(gate);
  if (p.tokens == 0) return ROOST_STATUS_OK;
  const uint64_t row_elems = static_cast<uint64_t>(p.kv_heads) * p.head_dim;
  gate.Tensor("k", p.k, dt, p.tokens * row_elems)
      .Tensor("v", p.v, dt, p.tokens * row_elems)
      .Tensor("k_cache", p.k_cache, dt, row_elems)
      .Tensor("v_cache", p.v_cache, dt, row_elems)
      .Tensor("slot_mapping", p.slot_mapping, ROOST_DTYPE_I64, p.tokens)
      .Aligned("k", p.k.address, 2)
      .Aligned("v", p.v.address, 2)
      .Aligned("k_cache", p.k_cache.address, 2)
      .Aligned("v_cache", p.v_cache.address, 2)
      .Aligned("slot_mapping", p.slot_mapping.address, 8);
  return gate.status();
}

template <typename W>
void Launch(const RoostCacheWriteParams& p, uint64_t pool_head_rows, uint32_t words_per_head, uint64_t total,
            hipStream_t stream) {
  const auto blocks = static_cast<uint32_t>(roost::CeilDiv(total, 256));
  hipLaunchKernelGGL(CacheWriteKernel<W>, dim3(blocks), dim3(256), 0, stream, static_cast<const W*>(p.k.address),
                     static_cast<const W*>(p.v.address), static_cast<W*>(p.k_cache.address),
                     static_cast<W*>(p.v_cache.address), static_cast<const int64_t*>(p.slot_mapping.address),
                     pool_head_rows, p.kv_heads, words_per_head, p.page_size,
                     p.kv_layout == ROOST_LAYOUT_PAGED_HND ? 1u : 0u, total);
}

}  // namespace

extern "C" ROOST_API RoostStatus roost_cache_write_run(RoostContext*, const void* params, const RoostWorkspace*,
                                                       void* stream) {
  constexpr char kOp[] = "cache_write";
  roost::Gate header(kOp);
  ROOST_GATE_RETURN(header.Header(params, sizeof(RoostCacheWriteParams)));
  const auto& p = *static_cast<const RoostCacheWriteParams*>(params);
  return roost::CatchAll(kOp, [&]() -> RoostStatus {
    ROOST_RETURN_IF_FAILED(Admit(p));
    if (p.tokens == 0) return ROOST_STATUS_OK;
    const uint32_t dt = p.k.dtype;
    const uint64_t head_bytes = static_cast<uint64_t>(p.head_dim) * roost::ElementBytes(dt);
    // Head rows each pool holds in full; a row at or past the shorter pool's count is skipped on the device.
    const uint64_t pool_head_rows = std::min(p.k_cache.length, p.v_cache.length) / p.head_dim;
    const bool vec16 = head_bytes % 16 == 0 && roost::IsAligned(p.k.address, 16) &&
                       roost::IsAligned(p.v.address, 16) && roost::IsAligned(p.k_cache.address, 16) &&
                       roost::IsAligned(p.v_cache.address, 16);
    const uint32_t word_bytes = vec16 ? 16 : 2;
    const auto words_per_head = static_cast<uint32_t>(head_bytes / word_bytes);
    const uint64_t total = static_cast<uint64_t>(p.tokens) * p.kv_heads * words_per_head;
    if (roost::CeilDiv(total, 256) > 0x7FFFFFFFull) {
      return roost::Report(ROOST_STATUS_INVALID_ARGUMENT, kOp, "%u tokens of %llu bytes exceed one launch's grid",
                           p.tokens, static_cast<unsigned long long>(head_bytes * p.kv_heads));
    }
    if (vec16) {
      Launch<uint4>(p, pool_head_rows, words_per_head, total, roost::Stream(stream));
    } else {
      Launch<uint16_t>(p, pool_head_rows, words_per_head, total, roost::Stream(stream));
    }
    return roost::HipStatus(hipGetLastError(), kOp, "kernel launch");
  });
}
