// The plan region of a worker step (batch tables and slot mapping), on the host and on the GPU.
//
// Semantics: PlanRegionWriter.Fill (reference: src/Starlings.Roost.Worker/Eager/PlanRegionWriter.cs:19-64). The rule per
// sequence and per token is stated once, in SequenceTables / TokenSlot below, and both paths call it: the host path
// walks the sequences in order on the calling thread; the device path gives each sequence one workgroup whose lanes
// stride over its blocks and tokens. Every output is a pure function of the inputs (no accumulation), so the two paths
// agree bit for bit.
//
// Design: integer work of a few bytes per token (a step of ~1K tokens writes ~20 KB). The device path exists so that a
// step whose block lists already live in HBM writes its tables without a host round trip; it is one launch of
// max(batch, 1) workgroups, bound by launch latency, not by HBM.

#include <algorithm>
#include <cstddef>
#include <cstring>
#include <vector>

#include "common.h"

namespace {

constexpr char kOp[] = "plan_region";

struct SequenceRow {
  int32_t q_start;      // q_indptr[b] = cu_seqlens[b]
  int32_t kv_start;     // kv_indptr[b]
  int32_t last_page;    // kv_last_page_len[b]
  int32_t block_count;  // blocks of the sequence
};

// PlanRegionWriter.cs:31-41: the sequence's row of the batch tables. The reference counts blocks as it goes
// (blockAt); with block_indptr starting at 0 that count is block_indptr[b].
__host__ __device__ inline SequenceRow SequenceTables(const RoostAmdPlanRegion& r, uint32_t b) {
  SequenceRow row;
  row.q_start = r.token_start[b];
  row.kv_start = r.block_indptr[b] - r.block_indptr[0];
  row.block_count = r.block_indptr[b + 1] - r.block_indptr[b];
  row.last_page = r.kv_length[b] - (row.block_count - 1) * static_cast<int32_t>(r.block_size);
  return row;
}

// PlanRegionWriter.cs:49: the cache slot of `position` in the sequence whose blocks start at `blocks`, or -1 when the
// position has no block.
__host__ __device__ inline int64_t TokenSlot(const int32_t* blocks, int32_t block_count, int32_t position,
                                             uint32_t block_size) {
  const int32_t bs = static_cast<int32_t>(block_size);
  if (position < 0 || position / bs >= block_count) return -1;
  return static_cast<int64_t>(blocks[position / bs]) * bs + position % bs;
}

// PlanRegionWriter.cs:61-63: the closing entries.
__host__ __device__ inline void CloseTables(const RoostAmdPlanRegion& r) {
  const int32_t q_end = r.batch == 0 ? 0 : r.token_start[r.batch - 1] + r.token_count[r.batch - 1];
  r.q_indptr[r.batch] = q_end;
  r.cu_seqlens[r.batch] = q_end;
  r.kv_indptr[r.batch] = r.block_indptr[r.batch] - r.block_indptr[0];
}

__global__ void __launch_bounds__(256) PlanRegionKernel(RoostAmdPlanRegion r) {
  const uint32_t b = blockIdx.x;
  if (r.batch == 0) {
    if (threadIdx.x == 0) CloseTables(r);
    return;
  }
  const SequenceRow row = SequenceTables(r, b);
  if (threadIdx.x == 0) {
    r.q_indptr[b] = row.q_start;
    r.cu_seqlens[b] = row.q_start;
    r.kv_indptr[b] = row.kv_start;
    r.kv_last_page_len[b] = row.last_page;
    if (r.state_slots != nullptr && r.recurrent_slot != nullptr) r.state_slots[b] = r.recurrent_slot[b];
    if (b + 1 == r.batch) CloseTables(r);
  }
  const int32_t* blocks = r.blocks + r.block_indptr[b];
  for (int32_t i = threadIdx.x; i < row.block_count; i += blockDim.x) r.kv_indices[row.kv_start + i] = blocks[i];
  const int32_t count = r.token_count[b], offset = r.position_offset[b];
  for (int32_t t = threadIdx.x; t < count; t += blockDim.x) {
    const int64_t index = static_cast<int64_t>(row.q_start) + t;
    if (index < 0 || index >= static_cast<int64_t>(r.tokens)) continue;
    if (r.positions != nullptr) r.positions[index] = offset + t;
    r.slot_mapping[index] = TokenSlot(blocks, row.block_count, offset + t, r.block_size);
  }
}

RoostStatus AdmitShape(const RoostAmdPlanRegion* r) {
  roost::Gate gate(kOp);
  gate.Expect(r != nullptr, ROOST_STATUS_INVALID_ARGUMENT, "no region was passed");
  ROOST_GATE_RETURN(gate);
  gate.Expect(r->reserved0 == 0, ROOST_STATUS_INVALID_ARGUMENT, "reserved0 = %u, must be 0", r->reserved0)
      .Expect(r->block_size > 0, ROOST_STATUS_INVALID_ARGUMENT, "block_size = 0")
      .Expect(r->batch < 0x7FFFFFFFu && r->tokens < 0x7FFFFFFFu, ROOST_STATUS_INVALID_ARGUMENT,
              "batch = %u, tokens = %u: the tables hold int32 entries", r->batch, r->tokens)
      .Expect(r->block_indptr != nullptr && r->q_indptr != nullptr && r->cu_seqlens != nullptr &&
                  r->kv_indptr != nullptr, ROOST_STATUS_INVALID_ARGUMENT,
              "block_indptr, q_indptr, cu_seqlens and kv_indptr are required");
  ROOST_GATE_RETURN(gate);
  const bool any = r->batch > 0;
  gate.Expect(!any || (r->token_start && r->token_count && r->position_offset && r->kv_length && r->kv_last_page_len),
              ROOST_STATUS_INVALID_ARGUMENT,
              "token_start, token_count, position_offset, kv_length and kv_last_page_len are required")
      .Expect(!any || r->tokens == 0 || r->slot_mapping != nullptr, ROOST_STATUS_INVALID_ARGUMENT,
              "slot_mapping is NULL")
      .Expect(!any || (r->state_slots == nullptr) == (r->recurrent_slot == nullptr), ROOST_STATUS_INVALID_ARGUMENT,
              "state_slots and recurrent_slot come together (both NULL or both set)");
  return gate.status();
}

// The host path's plan checks (the reference's Fill throws on these): block_indptr from 0 and non-decreasing, every
// sequence's tokens inside [0, tokens) and its positions inside its blocks.
RoostStatus AdmitHostPlan(const RoostAmdPlanRegion& r) {
  roost::Gate gate(kOp);
  gate.Expect(r.block_indptr[0] == 0, ROOST_STATUS_INVALID_ARGUMENT, "block_indptr[0] = %d, must be 0",
              r.block_indptr[0]);
  for (uint32_t b = 0; b < r.batch && gate.ok(); ++b) {
    const int32_t nb = r.block_indptr[b + 1] - r.block_indptr[b];
    const int64_t first = r.token_start[b], count = r.token_count[b], pos = r.position_offset[b];
    gate.Expect(nb >= 0, ROOST_STATUS_INVALID_ARGUMENT, "sequence %u: block_indptr goes backwards", b)
        .Expect(nb == 0 || r.blocks != nullptr, ROOST_STATUS_INVALID_ARGUMENT, "blocks is NULL")
        .Expect(count >= 0 && first >= 0 && first + count <= r.tokens, ROOST_STATUS_INVALID_ARGUMENT,
                "sequence %u: tokens %lld .. %lld outside [0, %u)", b, static_cast<long long>(first),
                static_cast<long long>(first + count), r.tokens)
        .Expect(count == 0 || (pos >= 0 && (pos + count - 1) / r.block_size < static_cast<uint64_t>(nb)),
                ROOST_STATUS_INVALID_ARGUMENT, "sequence %u: positions %lld .. %lld reach past its %d blocks of %u", b,
                static_cast<long long>(pos), static_cast<long long>(pos + count - 1), nb, r.block_size);
  }
  return gate.status();
}

// Writes the tables of an admitted region on the calling thread.
void FillHost(const RoostAmdPlanRegion& r) {
  for (uint32_t b = 0; b < r.batch; ++b) {
    const SequenceRow row = SequenceTables(r, b);
    r.q_indptr[b] = row.q_start;
    r.cu_seqlens[b] = row.q_start;
    r.kv_indptr[b] = row.kv_start;
    r.kv_last_page_len[b] = row.last_page;
    if (r.state_slots != nullptr) r.state_slots[b] = r.recurrent_slot[b];
    const int32_t* blocks = r.blocks + r.block_indptr[b];
    for (int32_t i = 0; i < row.block_count; ++i) r.kv_indices[row.kv_start + i] = blocks[i];
    for (int32_t t = 0; t < r.token_count[b]; ++t) {
      const int32_t index = row.q_start + t, position = r.position_offset[b] + t;
      if (r.positions != nullptr) r.positions[index] = position;
      r.slot_mapping[index] = TokenSlot(blocks, row.block_count, position, r.block_size);
    }
  }
  CloseTables(r);
}

// ---- C2 step plans ----------------------------------------------------------------------------------------------------
//
// Private mirrors of the step-plan structs (reference kernels/include/roost_worker_shm.h:41-141); their offsets are the
// reference's layout fixture's (tests/Starlings.Roost.Abstractions.Tests/Layout/abi-layout.golden.txt), pinned below.
namespace shm {

constexpr uint32_t kMagicPlan = 0x4C505352u;  // "RSPL"
constexpr uint32_t kSeqSample = 0x2u;         // the sequence samples after this chunk

struct TableRef {
  uint64_t offset;  // from the buffer start
  uint32_t count;
  uint32_t stride;  // bytes per entry
};

// The header's leading fields up to the block-id table (all this reader needs).
struct PlanHead {
  uint32_t magic, layout_version, header_size, flags;
  uint64_t step_id, total_bytes;
  uint32_t shape_bucket, math_mode, sequence_count, token_count, group_count, rank, mesh_id, reserved0;
  TableRef sequences, token_ids, positions, group_blocks, block_ids;
};
static_assert(offsetof(PlanHead, total_bytes) == 24 && offsetof(PlanHead, sequence_count) == 40 &&
                  offsetof(PlanHead, token_count) == 44 && offsetof(PlanHead, group_count) == 48 &&
                  offsetof(PlanHead, sequences) == 64 && offsetof(PlanHead, token_ids) == 80 &&
                  offsetof(PlanHead, positions) == 96 && offsetof(PlanHead, group_blocks) == 112 &&
                  offsetof(PlanHead, block_ids) == 128 && sizeof(PlanHead) == 144,
              "RoostStepPlanHeader offsets of the reference's layout fixture");

struct Sequence {
  uint64_t sequence_handle;
  uint32_t token_start, token_count, position_offset, group_blocks_start;
  int32_t recurrent_slot, lora_slot, grammar_slot, embedding_slot;
  uint32_t sampling_index, draft_count, flags;
};
static_assert(offsetof(Sequence, token_start) == 8 && offsetof(Sequence, position_offset) == 16 &&
                  offsetof(Sequence, group_blocks_start) == 20 && offsetof(Sequence, recurrent_slot) == 24 &&
                  offsetof(Sequence, flags) == 48,
              "RoostPlanSequence offsets of the reference's layout fixture");
constexpr uint32_t kSequenceBytes = 80;

struct GroupBlocks {
  uint32_t block_start, block_count;
};

}  // namespace shm

// Entry i of table t, whose entries are at least sizeof(T) bytes apart (bounds already checked).
template <typename T>
T Entry(const unsigned char* plan, const shm::TableRef& t, uint64_t i) {
  T v;
  std::memcpy(&v, plan + t.offset + i * t.stride, sizeof(T));
  return v;
}

RoostStatus ReadStepPlan(const unsigned char* plan, uint64_t plan_bytes, RoostAmdStepTables& out) {
  roost::Gate gate(kOp);
  gate.Expect(plan_bytes >= sizeof(shm::PlanHead), ROOST_STATUS_INVALID_ARGUMENT,
              "a step plan of %llu bytes is shorter than its header", static_cast<unsigned long long>(plan_bytes));
  ROOST_GATE_RETURN(gate);
  shm::PlanHead h;
  std::memcpy(&h, plan, sizeof(h));
  gate.Expect(h.magic == shm::kMagicPlan, ROOST_STATUS_INVALID_ARGUMENT, "magic 0x%08X is not a step plan's", h.magic)
      .Expect(h.header_size >= sizeof(shm::PlanHead) && h.total_bytes <= plan_bytes && h.header_size <= h.total_bytes,
              ROOST_STATUS_INVALID_ARGUMENT, "header of %u bytes in a plan of %llu bytes (%llu given)", h.header_size,
              static_cast<unsigned long long>(h.total_bytes), static_cast<unsigned long long>(plan_bytes))
      .Expect(out.block_size > 0 && out.attention_blocks > 0, ROOST_STATUS_INVALID_ARGUMENT,
              "block_size = %u, attention_blocks = %u", out.block_size, out.attention_blocks)
      .Expect(out.attention_group < h.group_count, ROOST_STATUS_INVALID_ARGUMENT,
              "attention_group %u of a plan with %u groups", out.attention_group, h.group_count);
  ROOST_GATE_RETURN(gate);
  auto table = [&](const char* name, const shm::TableRef& t, uint64_t expected, uint32_t entry_bytes) {
    gate.Expect(t.count == expected, ROOST_STATUS_INVALID_ARGUMENT, "%s: %u entries where the header implies %llu",
                name, t.count, static_cast<unsigned long long>(expected))
        .Expect(t.count == 0 || (t.stride >= entry_bytes && t.offset <= h.total_bytes &&
                                 (static_cast<uint64_t>(t.count) - 1) * t.stride + entry_bytes <= h.total_bytes - t.offset),
                ROOST_STATUS_INVALID_ARGUMENT, "table %s (%u entries of %u bytes at %llu) leaves the plan", name,
                t.count, t.stride, static_cast<unsigned long long>(t.offset));
  };
  const uint64_t batch = h.sequence_count, tokens = h.token_count;
  table("sequences", h.sequences, batch, shm::kSequenceBytes);
  table("token_ids", h.token_ids, tokens, 4);
  table("positions", h.positions, tokens, 4);
  table("group_blocks", h.group_blocks, batch * h.group_count, sizeof(shm::GroupBlocks));
  table("block_ids", h.block_ids, h.block_ids.count, 4);
  ROOST_GATE_RETURN(gate);

  std::vector<int32_t> start(batch), count(batch), offset(batch), kv_length(batch), slot(batch), indptr(batch + 1, 0);
  std::vector<int32_t> blocks, rows;
  uint64_t next = 0;
  for (uint64_t b = 0; b < batch && gate.ok(); ++b) {
    const auto s = Entry<shm::Sequence>(plan, h.sequences, b);
    const uint64_t end = static_cast<uint64_t>(s.token_start) + s.token_count;
    gate.Expect(s.token_start == next && s.token_count > 0 && end <= tokens, ROOST_STATUS_INVALID_ARGUMENT,
                "sequence %llu: %u tokens from %u, where a non-empty run from %llu inside the %llu-token table belongs",
                static_cast<unsigned long long>(b), s.token_count, s.token_start, static_cast<unsigned long long>(next),
                static_cast<unsigned long long>(tokens))
        .Expect(static_cast<uint64_t>(s.position_offset) + s.token_count <= 0x7FFFFFFFull, ROOST_STATUS_INVALID_ARGUMENT,
                "sequence %llu: position %u + %u tokens overflows", static_cast<unsigned long long>(b),
                s.position_offset, s.token_count)
        .Expect(s.group_blocks_start == b * h.group_count, ROOST_STATUS_INVALID_ARGUMENT,
                "sequence %llu: group_blocks_start = %u, where its %u lists start at %llu",
                static_cast<unsigned long long>(b), s.group_blocks_start, h.group_count,
                static_cast<unsigned long long>(b * h.group_count));
    if (!gate.ok()) break;
    for (uint32_t t = 0; t < s.token_count && gate.ok(); ++t) {
      gate.Expect(Entry<int32_t>(plan, h.positions, s.token_start + t) == static_cast<int32_t>(s.position_offset + t),
                  ROOST_STATUS_INVALID_ARGUMENT, "sequence %llu: token %u is not at position_offset %u + %u",
                  static_cast<unsigned long long>(b), t, s.position_offset, t);
    }
    const uint64_t kv = static_cast<uint64_t>(s.position_offset) + s.token_count;
    const uint64_t pages = (kv + out.block_size - 1) / out.block_size;
    const auto g = Entry<shm::GroupBlocks>(plan, h.group_blocks, s.group_blocks_start + out.attention_group);
    gate.Expect(g.block_count >= pages && static_cast<uint64_t>(g.block_start) + g.block_count <= h.block_ids.count,
                ROOST_STATUS_INVALID_ARGUMENT,
                "sequence %llu: %llu keys take %llu blocks of %u; its list holds %u from id %u of %u",
                static_cast<unsigned long long>(b), static_cast<unsigned long long>(kv),
                static_cast<unsigned long long>(pages), out.block_size, g.block_count, g.block_start,
                h.block_ids.count);
    if (!gate.ok()) break;
    start[b] = static_cast<int32_t>(s.token_start);
    count[b] = static_cast<int32_t>(s.token_count);
    offset[b] = static_cast<int32_t>(s.position_offset);
    kv_length[b] = static_cast<int32_t>(kv);
    slot[b] = s.recurrent_slot;
    for (uint64_t i = 0; i < pages && gate.ok(); ++i) {
      // A block id outside the pool would send attention reads and KV writes out of the pool: refused here, before
      // anything is written, as the worker's plan reader does (StepPlanReader.cs:322-328).
      const int32_t id = Entry<int32_t>(plan, h.block_ids, g.block_start + i);
      gate.Expect(id >= 0 && static_cast<uint32_t>(id) < out.attention_blocks, ROOST_STATUS_INVALID_ARGUMENT,
                  "sequence %llu: block id %d is outside [0, %u)", static_cast<unsigned long long>(b), id,
                  out.attention_blocks);
      blocks.push_back(id);
    }
    if (!gate.ok()) break;
    indptr[b + 1] = static_cast<int32_t>(blocks.size());
    if (s.flags & shm::kSeqSample) rows.push_back(static_cast<int32_t>(end - 1));
    next = end;
  }
  ROOST_GATE_RETURN(gate);
  gate.Expect(next == tokens, ROOST_STATUS_INVALID_ARGUMENT, "the sequences end at token %llu of %llu",
              static_cast<unsigned long long>(next), static_cast<unsigned long long>(tokens))
      .Expect(batch <= out.max_batch && tokens <= out.max_tokens && blocks.size() <= out.max_blocks,
              ROOST_STATUS_INVALID_ARGUMENT,
              "the plan has %llu sequences, %llu tokens and %zu blocks; the outputs hold %u, %u and %u",
              static_cast<unsigned long long>(batch), static_cast<unsigned long long>(tokens), blocks.size(),
              out.max_batch, out.max_tokens, out.max_blocks)
      .Expect(out.q_indptr && out.cu_seqlens && out.kv_indptr && out.kv_last_page_len &&
                  (tokens == 0 || out.slot_mapping) && (blocks.empty() || out.kv_indices),
              ROOST_STATUS_INVALID_ARGUMENT, "q_indptr, cu_seqlens, kv_indptr, kv_indices, kv_last_page_len and "
              "slot_mapping are required");
  ROOST_GATE_RETURN(gate);

  RoostAmdPlanRegion r{};
  r.batch = static_cast<uint32_t>(batch);
  r.tokens = static_cast<uint32_t>(tokens);
  r.block_size = out.block_size;
  r.token_start = start.data();
  r.token_count = count.data();
  r.position_offset = offset.data();
  r.kv_length = kv_length.data();
  r.block_indptr = indptr.data();
  r.blocks = blocks.data();
  r.recurrent_slot = out.state_slots != nullptr ? slot.data() : nullptr;
  r.q_indptr = out.q_indptr;
  r.cu_seqlens = out.cu_seqlens;
  r.kv_indptr = out.kv_indptr;
  r.kv_indices = out.kv_indices;
  r.kv_last_page_len = out.kv_last_page_len;
  r.state_slots = out.state_slots;
  r.positions = out.positions;
  r.slot_mapping = out.slot_mapping;
  FillHost(r);
  if (out.ids != nullptr) {
    for (uint64_t t = 0; t < tokens; ++t) out.ids[t] = Entry<int32_t>(plan, h.token_ids, t);
  }
  if (out.rows != nullptr) std::copy(rows.begin(), rows.end(), out.rows);
  out.batch = r.batch;
  out.tokens = r.tokens;
  out.blocks = static_cast<uint32_t>(blocks.size());
  out.rows_written = static_cast<uint32_t>(rows.size());
  return ROOST_STATUS_OK;
}

}  // namespace

extern "C" ROOST_API RoostStatus roost_amd_plan_region_fill(const RoostAmdPlanRegion* region) {
  return roost::CatchAll(kOp, [&]() -> RoostStatus {
    ROOST_RETURN_IF_FAILED(AdmitShape(region));
    ROOST_RETURN_IF_FAILED(AdmitHostPlan(*region));
    FillHost(*region);
    return ROOST_STATUS_OK;
  });
}

extern "C" ROOST_API RoostStatus roost_amd_plan_region_from_step(const void* plan, uint64_t plan_bytes,
                                                                 RoostAmdStepTables* tables) {
  return roost::CatchAll(kOp, [&]() -> RoostStatus {
    if (plan == nullptr || tables == nullptr) {
      return roost::Report(ROOST_STATUS_INVALID_ARGUMENT, kOp, "a plan buffer and a tables struct are required");
    }
    return ReadStepPlan(static_cast<const unsigned char*>(plan), plan_bytes, *tables);
  });
}

extern "C" ROOST_API RoostStatus roost_amd_plan_region_run(RoostContext* ctx, const RoostAmdPlanRegion* region,
                                                          void* stream) {
  return roost::CatchAll(kOp, [&]() -> RoostStatus {
    if (ctx == nullptr) return roost::Report(ROOST_STATUS_INVALID_ARGUMENT, kOp, "no context was passed");
    ROOST_RETURN_IF_FAILED(AdmitShape(region));
    const uint32_t blocks = std::max(region->batch, 1u);
    hipLaunchKernelGGL(PlanRegionKernel, dim3(blocks), dim3(256), 0, roost::Stream(stream), *region);
    return roost::HipStatus(hipGetLastError(), kOp, "launch");
  });
}
