// PagedAttention (ROOST_OP_PAGED_ATTENTION) for gfx950: paged GQA decode and varlen causal chunked prefill over a
// block-tabled KV cache, behind the C1 workspace / plan / run entry points.
//
// Semantics are CpuOps.PagedAttention (reference: src/Starlings.Roost.Ops/CpuOps.cs:198-298): sequence b has
// n = q_indptr[b+1]-q_indptr[b] queries and kvLen = (pages-1)*page_size + kv_last_page_len[b] keys; query i sits at
// key position kvLen-n+i and (causal) sees keys j <= that position; a decode query sees every key; query head h reads
// KV head h / (q_heads / kv_heads); score = q.k * scale (scale 0 -> 1/sqrt(head_dim)); softmax; sum p*v; a query that
// sees no key outputs zeros. The entry-point contract is the reference's (kernels/src/paged_attention.cu:78-349):
// workspace() and plan() read the host batch tables, run() never does and refuses with NOT_PLANNED until plan() has
// written a plan record for this batch shape. The optional lse output is the base-2 log-sum-exp of the scaled scores,
// log2(sum_j 2^(s_j * log2 e)), which is the convention of the FlashInfer kernels the reference wraps.
//
// Decode (mode DECODE) -- HBM bound (DecodeKernel, DecodeMergeKernel):
//   * plan() deals the batch's 16-token groups out evenly to one range per resident workgroup slot and cuts sequences
//     at range boundaries (so the variant is DETERMINISTIC but not BATCH_INVARIANT); a workgroup serves the KV heads
//     of its range, its wavefronts take alternate groups;
//   * K and V rows are loaded branch-free into a register double buffer (the next group in flight while the current
//     one is computed), each K/V byte once, shared by the query heads of the GQA group;
//   * bf16: q.k on v_mfma_f32_16x16x32_bf16 (tokens on M, the group's query heads on N), P.V on v_dot2 with P rounded
//     to bf16; f32: q.k as VALU products reduce-scattered across the lanes of a row;
//   * the wavefronts merge through LDS; a sequence cut into pieces writes fp32 partials (o, m, l) that
//     DecodeMergeKernel combines in key order.
// Prefill (mode PREFILL) -- MFMA bound (PrefillTileKernel + PrefillMergeKernel for page sizes that are powers of two
// and multiples of 16; PrefillKernel otherwise):
//   * one workgroup = 64 query tokens x the 4 query heads of one (virtual) KV head, 8 wavefronts; 64-key K and V
//     tiles are copied from the paged cache straight into LDS (global_load_lds), double-buffered;
//   * S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_32x32x16_bf16 with fp32 accumulation; the softmax statistics of a
//     query live in one lane pair; P is rounded to bf16 before the P.V product (as FlashAttention-2 does);
//   * plan() cuts items longer than the average CU load into pieces (bf16 partials merged in key order) and orders the
//     work longest-first so the ragged causal tail does not set the makespan;
//   * single-token sequences of a prefill call run on the decode kernels, beside the tile kernel on the context's
//     second stream when plan() finds that cheaper (ChooseOverlap); an f32 prefill runs every query token as a row of
//     the f32 decode kernel.
// Output gate (roost_amd_paged_attention_gated_run): Qwen3.5's SigmoidMul on the attention output, applied by every
// kernel that stores an output element (decode, both prefill kernels, both merges) to the element already rounded to
// the output type, with the SigmoidMul op's arithmetic (GateMul in common.h), so it equals run() then SigmoidMul.

#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <queue>
#include <type_traits>
#include <vector>

#include "common.h"

namespace {

using namespace roost_dev;

constexpr uint32_t kGroup = 4;                  // query heads per KV head (Qwen3.5: 8 over 2)
constexpr uint32_t kDecodeWgsPerCu = 2;        // decode workgroups resident per CU
constexpr int kMixedDecodeWaves = 8;           // wavefronts of a decode workgroup in the one-launch mixed step
constexpr int kDecodeRing = 2;                  // register ring depth: groups in flight per wavefront = ring - 1
constexpr uint32_t kMaxMergeSplits = 1024;      // partials one sequence may be split into
constexpr uint32_t kPrefillTileQ = 32;          // query tokens per workgroup of the general-page-size prefill
constexpr uint32_t kPrefillTileK = 64;          // keys per LDS tile
constexpr uint32_t kPfTokens = 64;              // query tokens per workgroup of the prefill for page sizes % 16 == 0
constexpr uint32_t kPfRows = kPfTokens * kGroup;  // query rows (token, head) of one such workgroup
constexpr uint32_t kPfMinSplitTiles = 8;        // a split piece covers at least this many 64-key tiles
constexpr uint32_t kAlign = 256;
constexpr uint32_t kPlanMagic = 0x41504752;     // "RGPA"
constexpr float kLog2e = 1.4426950408889634f;

// Logit soft capping (CpuOps.cs:276: s -> cap tanh(s / cap) after the scale), applied to scores in log2 units:
// y -> capl tanh(y / capl) with capl = |cap| log2(e), through tanh(u) = 1 - 2 / (1 + e^(2u)) = 1 - 2 / (1 + 2^(y k)),
// k = 2 log2(e) / capl. capl = 0 turns it off. Masked scores are set to -inf after capping.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Round-to-nearest-even pack of two floats (v_cvt_pk_bf16_f32): the softmax weights, which lie in [0, 256], and the
// tile kernel's outputs (the same rounding as PackBf16 for every finite value; only a NaN, which finite inputs never
// produce here, may keep another NaN pattern than 0x7FC0).
__device__ __forceinline__ uint32_t PackRne(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

struct SoftCap {
  float capl;
  float k;
};
__device__ __forceinline__ float Capped(float y, SoftCap c) {
  return c.capl - 2.0f * c.capl * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(y * c.k));
}

// A decode row is one query token: the last token of its sequence (q_back 0: decode calls and the single-token
// sequences of a prefill call) or, in an f32 prefill, any token, q_back tokens before the sequence's last.
struct DecodeWork {
  int32_t seq;
  int32_t token_begin;  // first key of this piece (a multiple of 16)
  int32_t token_end;    // one past its last key
  int32_t slot;         // partial slot, or -1 when the piece is the whole row (written as the final row)
  int32_t q_back;       // the row's query token sits q_back tokens before its sequence's last token
};
struct DecodeMerge {
  int32_t seq;
  int32_t first;  // first partial slot; the row's pieces own slots first .. first + count - 1 in key order
  int32_t count;
  int32_t q_back;
};
// A prefill work item: query tokens q0 .. q0 + rows - 1 of sequence seq (all kGroup query heads of one KV head)
// against keys [kbeg, kend). slot >= 0 marks one piece of a split key range: it writes partials (its output divided
// by its own sum, in bf16, and its fp32 running max and sum) that PrefillMergeKernel combines; slot -1 writes the final
// rows.
struct PrefillWork {
  int32_t seq;
  int32_t q0;
  int32_t kv_head;
  int32_t rows;
  int32_t kbeg;
  int32_t kend;
  int32_t slot;
  int32_t ends;  // kPieceFirst | kPieceLast: whether this piece starts / ends its item's key range
};
// The kernels re-derive an item's outer key bounds from the device's kv_last_page_len (plan() may have assumed full
// last pages when kv_last_page_len_host was NULL, or the lengths may have changed since): the first piece of an item
// starts at the device's first visible key and the last piece ends at the device's last one.
constexpr int32_t kPieceFirst = 1;
constexpr int32_t kPieceLast = 2;
struct PrefillMerge {
  int32_t seq;
  int32_t q0;
  int32_t kv_head;
  int32_t rows;
  int32_t first;  // the pieces own partial slots first .. first + count - 1
  int32_t count;
  int32_t reserved[2];
};

// What plan() leaves for run(); trivially copyable, read back with memcpy.
struct PlanRecord {
  uint32_t magic;
  uint32_t mode;
  uint32_t batch;
  uint32_t tokens;
  uint32_t page_size;
  uint32_t kv_layout;
  uint32_t head_dim;
  uint32_t kv_heads;
  int32_t window;        // WindowOf(params): the pieces start at the window
  uint32_t merges_two;   // prefill: the leading merge entries of exactly two pieces
  uint32_t overlap;      // prefill with single-token sequences: tile and decode kernels run side by side
  uint32_t reserved1;
  uint64_t pages;        // kv_indptr_host[batch]
  uint64_t work_items;   // decode pieces or prefill tiles
  uint64_t ranges;       // decode: workgroup ranges over the pieces
  uint64_t merges;       // decode: sequences whose pieces are merged
  uint64_t range_offset; // byte offsets in the int region
  uint64_t merge_offset;
  uint64_t counter_offset;
  uint64_t splits;       // decode partial slots
  uint64_t int_bytes;    // [work items | seq splits]
  uint64_t float_offset; // partials start here
  uint64_t float_bytes;
  // Single-token sequences of a prefill call run as decode: their pieces, ranges, merges and partials.
  uint64_t dec_items, dec_ranges, dec_merges, dec_splits;
  uint64_t dec_item_offset, dec_range_offset, dec_merge_offset, dec_float_offset;
};

struct Layout {
  uint64_t work_items = 0;
  uint64_t ranges = 0;
  uint64_t merges = 0;
  uint64_t merges_two = 0;  // prefill: leading merge entries of two pieces
  uint32_t overlap = 0;     // prefill: tile and decode kernels on two streams (ChooseOverlap)
  uint64_t range_offset = 0;
  uint64_t merge_offset = 0;
  uint64_t counter_offset = 0;
  uint64_t splits = 0;
  uint64_t int_bytes = 0;
  uint64_t float_offset = 0;
  uint64_t float_bytes = 0;
  uint64_t total = 0;
  // Decode region (decode calls: the whole plan; prefill calls: the single-token sequences).
  uint64_t dec_items = 0, dec_ranges = 0, dec_merges = 0, dec_splits = 0;
  uint64_t dec_item_offset = 0, dec_range_offset = 0, dec_merge_offset = 0, dec_float_offset = 0;
};

// ---- Admission ---------------------------------------------------------------------------------------------------

// Query heads per KV head the kernels serve: groups of kGroup = 4, or 8, 16 and 32 as 2, 4 and 8 groups of 4 that read
// the same KV rows (the reference builds 4 only).
bool GroupBuilt(uint32_t g) { return g == 4 || g == 8 || g == 16 || g == 32; }
// Groups of kGroup query heads ("virtual" KV heads) and the log2 of how many of them share one real KV head.
uint32_t VirtualHeads(const RoostPagedAttentionParams& p) { return p.q_heads / kGroup; }
uint32_t HeadShift(const RoostPagedAttentionParams& p) {
  return static_cast<uint32_t>(__builtin_ctz(p.q_heads / (p.kv_heads * kGroup)));
}

// Shapes with a kernel here, per mode: head dims 64/128/256 decode; prefill on the tile kernel at 64, 128 and 256
// (64 and 128 need page sizes that are powers of two and multiples of 16), on the general kernel at 256.
bool PrefillShapeBuilt(const RoostPagedAttentionParams& p) {
  // f32 prefills run on the decode kernels (any page size); bf16 ones on the tile kernels.
  if (p.head_dim == 256 || p.q.dtype == ROOST_DTYPE_F32) return true;
  return (p.head_dim == 128 || p.head_dim == 64) && p.page_size % 16 == 0 && roost::IsPow2(p.page_size);
}

// The host batch tables, as workspace() and plan() read them: q_indptr over [0, tokens], both indptrs
// non-decreasing, last-page lengths in [1, page_size] for sequences that have pages, and (CpuOps.cs:326-329) a causal
// prefill sequence holding at least as many keys as queries.
void AdmitHostTables(const RoostPagedAttentionParams& p, roost::Gate& gate) {
  gate.Expect(p.q_indptr_host != nullptr && p.kv_indptr_host != nullptr, ROOST_STATUS_INVALID_ARGUMENT,
              "plan and workspace read q_indptr_host and kv_indptr_host; %s is NULL",
              p.q_indptr_host == nullptr ? "q_indptr_host" : "kv_indptr_host");
  if (!gate.ok()) return;
  const int32_t* qi = p.q_indptr_host;
  const int32_t* ki = p.kv_indptr_host;
  gate.Expect(qi[0] == 0 && qi[p.batch] == static_cast<int32_t>(p.tokens), ROOST_STATUS_INVALID_ARGUMENT,
              "q_indptr_host runs from %d to %d; it must run from 0 to tokens = %u", qi[0], qi[p.batch], p.tokens)
      .Expect(ki[0] == 0, ROOST_STATUS_INVALID_ARGUMENT, "kv_indptr_host[0] = %d, must be 0", ki[0]);
  for (uint32_t b = 0; b < p.batch && gate.ok(); ++b) {
    gate.Expect(qi[b + 1] >= qi[b] && ki[b + 1] >= ki[b], ROOST_STATUS_INVALID_ARGUMENT,
                "sequence %u: q_indptr_host or kv_indptr_host goes backwards", b);
    const int64_t pages = ki[b + 1] - ki[b];
    if (p.kv_last_page_len_host == nullptr || pages <= 0 || !gate.ok()) continue;
    const int32_t last = p.kv_last_page_len_host[b];
    gate.Expect(last >= 1 && last <= static_cast<int32_t>(p.page_size), ROOST_STATUS_INVALID_ARGUMENT,
                "sequence %u: kv_last_page_len_host = %d outside 1..page_size (%u)", b, last, p.page_size);
    if (p.mode == ROOST_ATTENTION_PREFILL && p.causal) {
      const int64_t keys = (pages - 1) * p.page_size + last;
      gate.Expect(keys >= qi[b + 1] - qi[b], ROOST_STATUS_INVALID_ARGUMENT,
                  "sequence %u: causal prefill of %d queries over only %lld keys", b, qi[b + 1] - qi[b],
                  static_cast<long long>(keys));
    }
  }
}

// The call's rules (the reference refuses a subset of these shapes: kernels/src/paged_attention.cu:78-130). `for_run`
// checks the device spans; otherwise (workspace, plan) the host tables.
RoostStatus Admit(const RoostPagedAttentionParams& p, bool for_run) {
  roost::Gate gate("paged_attention");
  const bool prefill = p.mode == ROOST_ATTENTION_PREFILL;
  gate.Expect(p.mode == ROOST_ATTENTION_DECODE || prefill, ROOST_STATUS_INVALID_ARGUMENT,
              "mode = %u is neither DECODE nor PREFILL", p.mode)
      .Expect(p.head_dim == 64 || p.head_dim == 128 || p.head_dim == 256, ROOST_STATUS_UNSUPPORTED,
              "head_dim = %u has no kernel here (built: 64, 128, 256)", p.head_dim)
      .Expect(!prefill || PrefillShapeBuilt(p), ROOST_STATUS_UNSUPPORTED,
              "bf16 prefill at head_dim = %u, page_size = %u has no kernel here (built: 256 at any page size; 64 and 128 "
              "at power-of-two page sizes that are multiples of 16)", p.head_dim, p.page_size)
      .Expect(p.kv_heads > 0 && p.q_heads % p.kv_heads == 0 && GroupBuilt(p.q_heads / std::max(p.kv_heads, 1u)),
              ROOST_STATUS_UNSUPPORTED, "q_heads = %u over kv_heads = %u: built for groups of 4, 8, 16 or 32 query "
              "heads per KV head", p.q_heads, p.kv_heads)
      // CpuOps.cs:180-186: a window of 0 keys is an error; -1 (any negative value) means no window.
      .Expect(p.window_left != 0, ROOST_STATUS_INVALID_ARGUMENT, "window_left = 0 is not a window; pass -1 for none")
      .Expect(std::isfinite(p.logits_soft_cap), ROOST_STATUS_INVALID_ARGUMENT,
              "logits_soft_cap = %g; a finite cap (0 for none) is required", p.logits_soft_cap)
      .Expect(p.kv_layout == ROOST_LAYOUT_PAGED_NHD || p.kv_layout == ROOST_LAYOUT_PAGED_HND,
              ROOST_STATUS_INVALID_ARGUMENT, "kv_layout = %u is not a paged layout (NHD or HND)", p.kv_layout)
      .Expect(p.batch > 0 && p.page_size > 0, ROOST_STATUS_INVALID_ARGUMENT,
              "batch = %u, page_size = %u: both must be positive", p.batch, p.page_size)
      .Expect(prefill || p.tokens == p.batch, ROOST_STATUS_INVALID_ARGUMENT,
              "decode of %u tokens over %u sequences; decode is one query token per sequence", p.tokens, p.batch);
  ROOST_GATE_RETURN(gate);
  if (!for_run) {
    AdmitHostTables(p, gate);
    return gate.status();
  }
  const uint32_t dt = p.q.dtype;
  gate.Expect(dt == ROOST_DTYPE_BF16 || dt == ROOST_DTYPE_F32, ROOST_STATUS_INVALID_ARGUMENT,
              "q is %s; attention reads bf16 or f32", roost::Describe(dt).name);
  ROOST_GATE_RETURN(gate);
  const uint64_t q_elems = static_cast<uint64_t>(p.tokens) * p.q_heads * p.head_dim;
  const uint64_t page_elems = static_cast<uint64_t>(p.page_size) * p.kv_heads * p.head_dim;
  gate.Tensor("q", p.q, dt, q_elems)
      .Tensor("output", p.output, dt, q_elems)
      .OptionalTensor("lse", p.lse, ROOST_DTYPE_F32, static_cast<uint64_t>(p.tokens) * p.q_heads)
      .Tensor("k_cache", p.k_cache, dt, page_elems)
      .Tensor("v_cache", p.v_cache, dt, page_elems)
      .Tensor("q_indptr", p.q_indptr, ROOST_DTYPE_I32, p.batch + 1ull)
      .Tensor("kv_indptr", p.kv_indptr, ROOST_DTYPE_I32, p.batch + 1ull)
      .Tensor("kv_last_page_len", p.kv_last_page_len, ROOST_DTYPE_I32, p.batch)
      .Aligned("q", p.q.address, 16)
      .Aligned("output", p.output.address, 16)
      .Aligned("k_cache", p.k_cache.address, 16)
      .Aligned("v_cache", p.v_cache.address, 16);
  return gate.status();
}

// ---- Host planning ---------------------------------------------------------------------------------------------------

// rows_per_split: partial rows one split slot holds (decode: the query heads of a sequence; prefill: kPfRows).
Layout MakeLayout(uint64_t work_items, uint64_t ranges, uint64_t merges, uint64_t splits, uint32_t rows_per_split,
                  uint32_t head_dim, uint32_t mode) {
  Layout l;
  l.work_items = work_items;
  l.ranges = ranges;
  l.merges = merges;
  l.splits = splits;
  const bool decode = mode == ROOST_ATTENTION_DECODE;
  const uint64_t item_bytes = decode ? sizeof(DecodeWork) : sizeof(PrefillWork);
  const uint64_t merge_bytes = decode ? sizeof(DecodeMerge) : sizeof(PrefillMerge);
  l.range_offset = roost::RoundUp(work_items * item_bytes, 16);
  l.merge_offset = roost::RoundUp(l.range_offset + (ranges > 0 ? (ranges + 1) * sizeof(int32_t) : 0), 16);
  l.int_bytes = l.merge_offset + merges * merge_bytes;
  l.float_offset = roost::RoundUp(l.int_bytes, kAlign);
  // decode partials: fp32 rows then (max, sum); prefill partials: bf16 rows then (max, sum)
  l.float_bytes = splits * rows_per_split *
                  (decode ? (static_cast<uint64_t>(head_dim) + 2) * sizeof(float) : 2 * static_cast<uint64_t>(head_dim) + 8);
  l.total = l.float_offset + l.float_bytes;
  return l;
}

uint32_t KvLenHost(const RoostPagedAttentionParams& p, uint32_t b) {
  const int64_t pages = p.kv_indptr_host[b + 1] - p.kv_indptr_host[b];
  if (pages <= 0) return 0;
  const int64_t last = p.kv_last_page_len_host != nullptr ? p.kv_last_page_len_host[b] : p.page_size;
  return static_cast<uint32_t>((pages - 1) * p.page_size + last);
}

// The sliding window: query position pos sees keys j >= pos - window (reference CpuOps.cs:180-197, 245-252); -1 (any
// negative window_left) means no window.
int32_t WindowOf(const RoostPagedAttentionParams& p) { return p.window_left < 0 ? -1 : p.window_left; }
// The soft cap as the kernels apply it (in log2 units); a cap of 0 is off and the sign of the cap does not matter
// (cap tanh(s / cap) is even in cap).
SoftCap CapOf(const RoostPagedAttentionParams& p) {
  const float cap = std::fabs(p.logits_soft_cap);
  if (cap == 0.0f) return SoftCap{0.0f, 0.0f};
  const float capl = cap * kLog2e;
  return SoftCap{capl, 2.0f * kLog2e / capl};
}
// First key a decode query (position kv - 1) sees.
int64_t DecodeFirstKey(int64_t kv, int32_t window) { return window < 0 ? 0 : std::max<int64_t>(0, kv - 1 - window); }

// Decode: the batch's 16-token groups are dealt out evenly to `ranges` workgroup ranges (kDecodeWgsPerCu workgroups
// per CU), each range cut at sequence boundaries into pieces. Every workgroup then streams the same number of bytes
// and the grid finishes together instead of in ragged rounds. A sequence cut into several pieces owns consecutive
// partial slots and one DecodeMerge entry (merged by DecodeMergeKernel); a sequence without keys is one empty piece
// that writes its zero rows.
// The split depends on the batch, so the variant is deterministic but not batch invariant.
// KV heads one decode workgroup serves: 4, 2 or 1, whichever divides kv_heads first.
uint32_t HeadsPerWorkgroup(uint32_t kv_heads) { return kv_heads % 4 == 0 ? 4 : (kv_heads % 2 == 0 ? 2 : 1); }

struct DecodePlan {
  std::vector<DecodeWork> items;
  std::vector<int32_t> range_ptr;  // ranges + 1 entries; empty when no sequence is planned
  std::vector<DecodeMerge> merges;
  int32_t slots = 0;
  uint64_t ranges() const { return range_ptr.empty() ? 0 : range_ptr.size() - 1; }
};

// One decode row: query token q_back tokens before the last of sequence seq, reading keys [first, end) (host lengths;
// the kernel clamps to the device's).
struct DecodeRow {
  uint32_t seq;
  int32_t q_back;
  int64_t first;
  int64_t end;
};

// Cuts the rows' keys into 16-token groups and the groups into ranges of about equal length, one range per workgroup
// slot (kDecodeWgsPerCu per CU); a row cut across ranges gets partial slots and a DecodeMerge entry.
DecodePlan BuildDecodeRows(const RoostPagedAttentionParams& p, uint32_t cus, const std::vector<DecodeRow>& rows) {
  DecodePlan d;
  if (rows.empty()) return d;
  std::vector<uint64_t> groups(rows.size()), first_group(rows.size());
  uint64_t total = 0;
  for (size_t r = 0; r < rows.size(); ++r) {
    // Keys before the window are never read (their pages may have been released); the first group keeps its
    // 16-alignment and the kernel masks its keys below the window.
    first_group[r] = static_cast<uint64_t>(rows[r].first) / 16;
    groups[r] = rows[r].end > rows[r].first ? roost::CeilDiv(static_cast<uint64_t>(rows[r].end), 16) - first_group[r] : 0;
    total += groups[r];
  }
  const uint64_t slots_wanted = std::max<uint64_t>(
      1, static_cast<uint64_t>(cus) * kDecodeWgsPerCu / (VirtualHeads(p) / HeadsPerWorkgroup(VirtualHeads(p))));
  const uint64_t ranges = std::max<uint64_t>(1, std::min<uint64_t>(slots_wanted, total));
  uint64_t per_range = std::max<uint64_t>(1, roost::CeilDiv(total, ranges));
  // A row spans at most ceil(groups / per_range) + 1 pieces; keep that within what the merge kernel combines.
  const uint64_t longest = *std::max_element(groups.begin(), groups.end());
  per_range = std::max<uint64_t>(per_range, roost::CeilDiv(longest, kMaxMergeSplits - 2));
  d.items.reserve(rows.size() + ranges * 2);
  d.range_ptr.reserve(ranges + 1);
  d.range_ptr.push_back(0);
  uint64_t room = per_range;  // groups left in the current range
  for (size_t r = 0; r < rows.size(); ++r) {
    const auto seq = static_cast<int32_t>(rows[r].seq);
    const int32_t back = rows[r].q_back;
    if (groups[r] == 0) {
      d.items.push_back(DecodeWork{seq, 0, 0, -1, back});
      continue;
    }
    const size_t first_item = d.items.size();
    uint64_t g = 0;
    while (g < groups[r]) {
      if (room == 0) {
        d.range_ptr.push_back(static_cast<int32_t>(d.items.size()));
        room = per_range;
      }
      const uint64_t n = std::min(room, groups[r] - g);
      d.items.push_back(DecodeWork{seq, static_cast<int32_t>((first_group[r] + g) * 16),
                                   static_cast<int32_t>(std::min<uint64_t>((first_group[r] + g + n) * 16,
                                                                           static_cast<uint64_t>(rows[r].end))),
                                   -1, back});
      g += n;
      room -= n;
    }
    const size_t pieces = d.items.size() - first_item;
    if (pieces > 1) {
      d.merges.push_back(DecodeMerge{seq, d.slots, static_cast<int32_t>(pieces), back});
      for (size_t i = first_item; i < d.items.size(); ++i) d.items[i].slot = d.slots++;
    }
  }
  d.range_ptr.push_back(static_cast<int32_t>(d.items.size()));
  return d;
}

// The last-token rows of the sequences b with take(b) (all of them in a decode call, the single-token ones in a
// prefill call).
template <typename Take>
DecodePlan BuildDecode(const RoostPagedAttentionParams& p, uint32_t cus, Take take) {
  std::vector<DecodeRow> rows;
  const int32_t window = WindowOf(p);
  for (uint32_t b = 0; b < p.batch; ++b) {
    if (!take(b)) continue;
    const int64_t kv = KvLenHost(p, b);
    rows.push_back(DecodeRow{b, 0, DecodeFirstKey(kv, window), kv});
  }
  return BuildDecodeRows(p, cus, rows);
}

// Every query token of every sequence as its own row (the f32 prefill, which runs on the VALU decode kernel): token i
// of a sequence of n tokens and kv keys sits at position kv - n + i and reads keys from its window start to itself
// (causal) or to the end.
DecodePlan BuildDecodeAllTokens(const RoostPagedAttentionParams& p, uint32_t cus) {
  std::vector<DecodeRow> rows;
  const int32_t window = WindowOf(p);
  for (uint32_t b = 0; b < p.batch; ++b) {
    const int64_t n = p.q_indptr_host[b + 1] - p.q_indptr_host[b];
    const int64_t kv = KvLenHost(p, b);
    for (int64_t i = 0; i < n; ++i) {
      const int64_t pos = kv - n + i;
      const int64_t end = p.causal ? std::max<int64_t>(0, pos + 1) : kv;
      const int64_t first = window < 0 ? 0 : std::max<int64_t>(0, pos - window);
      rows.push_back(DecodeRow{b, static_cast<int32_t>(n - 1 - i), std::min(first, end), end});
    }
  }
  return BuildDecodeRows(p, cus, rows);
}

// Places a decode plan at the end of the int region [0, l.int_bytes) and its partials at the end of the float region
// (which must not be laid out yet), then writes it to host when given.
void AppendDecode(const RoostPagedAttentionParams& p, const DecodePlan& d, Layout& l, unsigned char* host) {
  l.dec_items = d.items.size();
  l.dec_ranges = d.ranges();
  l.dec_merges = d.merges.size();
  l.dec_splits = static_cast<uint64_t>(d.slots);
  l.dec_item_offset = roost::RoundUp(l.int_bytes, 16);
  l.dec_range_offset = roost::RoundUp(l.dec_item_offset + l.dec_items * sizeof(DecodeWork), 16);
  l.dec_merge_offset = roost::RoundUp(l.dec_range_offset + d.range_ptr.size() * sizeof(int32_t), 16);
  l.int_bytes = l.dec_merge_offset + l.dec_merges * sizeof(DecodeMerge);
  if (host != nullptr) {
    std::memcpy(host + l.dec_item_offset, d.items.data(), d.items.size() * sizeof(DecodeWork));
    std::memcpy(host + l.dec_range_offset, d.range_ptr.data(), d.range_ptr.size() * sizeof(int32_t));
    std::memcpy(host + l.dec_merge_offset, d.merges.data(), d.merges.size() * sizeof(DecodeMerge));
  }
  (void)p;
}

// Lays out the float region after the int region: the prefill partials (prefill_floats bytes), then the decode ones.
void PlaceFloats(const RoostPagedAttentionParams& p, uint64_t prefill_floats, Layout& l) {
  l.float_offset = roost::RoundUp(l.int_bytes, kAlign);
  l.dec_float_offset = l.float_offset + roost::RoundUp(prefill_floats, kAlign);
  l.float_bytes = (l.dec_float_offset - l.float_offset) +
                  l.dec_splits * p.q_heads * (static_cast<uint64_t>(p.head_dim) + 2) * sizeof(float);
  l.total = l.float_offset + l.float_bytes;
}

Layout PlanDecode(const RoostPagedAttentionParams& p, uint32_t cus, unsigned char* host) {
  const DecodePlan d = BuildDecode(p, cus, [](uint32_t) { return true; });
  Layout l;
  AppendDecode(p, d, l, host);
  PlaceFloats(p, 0, l);
  // The decode call's record fields name the same region.
  l.work_items = l.dec_items;
  l.ranges = l.dec_ranges;
  l.merges = l.dec_merges;
  l.splits = l.dec_splits;
  l.range_offset = l.dec_range_offset;
  l.merge_offset = l.dec_merge_offset;
  return l;
}

// Prefill work items: one per (query tile, KV head) -- 64-token tiles when the page size is a multiple of 16 (the
// DMA-fed kernel), 32-token tiles otherwise. For the 64-token kernel the key range of an item longer than 3/4 of the
// average load of a CU is cut into pieces of whole 64-key tiles (at least kPfMinSplitTiles each), so that the longest causal
// tile does not set the makespan; the pieces write partials merged by PrefillMergeKernel. Items are ordered longest
// first. The cuts depend on the whole batch, so the variant is deterministic but not batch invariant.
bool PrefillFastPath(const RoostPagedAttentionParams& p) {
  return p.page_size % 16 == 0 && (p.page_size & (p.page_size - 1)) == 0;
}

// Tiles of a work item (its key range in 64-key tiles), and of the pieces it is cut into with at most `target` each.
int64_t ItemTiles(const PrefillWork& w) { return roost::CeilDiv(static_cast<int64_t>(w.kend - w.kbeg), 64); }
int64_t Pieces(int64_t tiles, int64_t target) { return std::min<int64_t>(roost::CeilDiv(tiles, target), kMaxMergeSplits); }

// The longest-first dispatch of the items cut at `target` onto `cus` workgroup slots, each piece costing its tiles
// plus kPfPieceCost (its set-up and epilogue): the finishing time of the last slot, in tiles.
constexpr int64_t kPfPieceCost = 2;
template <typename Items>
int64_t PrefillMakespan(const Items& items, int64_t target, uint32_t cus) {
  // Piece costs by counting (they are small integers), then longest first onto the least loaded slot.
  std::vector<uint32_t> count;
  for (const auto& it : items) {
    const int64_t tiles = ItemTiles(it.w), n = Pieces(tiles, target);
    for (int64_t i = 0; i < n; ++i) {
      const auto c = static_cast<size_t>(tiles * (i + 1) / n - tiles * i / n + kPfPieceCost);
      if (c >= count.size()) count.resize(c + 1, 0);
      ++count[c];
    }
  }
  // Slots by load (at[L]: how many slots carry L tiles); loads only grow, so the least loaded level only moves up.
  std::vector<uint32_t> at(1, std::max<uint32_t>(cus, 1));
  size_t lo = 0, end = 0;
  for (size_t c = count.size(); c-- > 0;) {
    for (uint32_t k = 0; k < count[c]; ++k) {
      while (at[lo] == 0) ++lo;
      --at[lo];
      const size_t load = lo + c;
      if (load >= at.size()) at.resize(load + 1, 0);
      ++at[load];
      end = std::max(end, load);
    }
  }
  return static_cast<int64_t>(end);
}

// The piece size (in tiles, at least kPfMinSplitTiles) the 64-token kernel cuts key ranges at. Candidates: 3/4, 17/20
// and the whole of the average CU load, and the smallest sizes whose pieces fill the CUs exactly once or twice
// (config 5's two 512-token chunks: 256 pieces of 9 tiles instead of 288 of 8, whose last 32 ran in a second round);
// the one whose longest-first dispatch ends first wins. Config 3 keeps 3/4 (0.197 ms, against 0.203 at 17/20 and
// 0.234 at 13/20); a dense 4 x 4096 batch takes the whole average (1,095 against 950 TFLOP/s at 3/4).
template <typename Items>
int64_t PrefillPieceTiles(const Items& items, int64_t total_tiles, uint32_t cus) {
  const uint32_t slots = std::max<uint32_t>(cus, 1);
  auto of_avg = [&](int64_t num, int64_t den) {
    return std::max<int64_t>(kPfMinSplitTiles, roost::CeilDiv(total_tiles * num, den * int64_t{slots}));
  };
  std::vector<int64_t> cand{of_avg(3, 4), of_avg(17, 20), of_avg(1, 1)};
  int64_t longest = 0;
  for (const auto& it : items) longest = std::max(longest, ItemTiles(it.w));
  for (int64_t rounds = 1; rounds <= 2; ++rounds) {
    if (static_cast<int64_t>(items.size()) > rounds * slots) break;
    // Smallest target whose pieces number at most rounds x slots (the count only falls as the target grows).
    int64_t lo = kPfMinSplitTiles, hi = std::max<int64_t>(longest, kPfMinSplitTiles);
    auto count = [&](int64_t t) {
      int64_t n = 0;
      for (const auto& it : items) n += Pieces(ItemTiles(it.w), t);
      return n;
    };
    if (count(hi) > rounds * slots) continue;
    while (lo < hi) {
      const int64_t mid = (lo + hi) / 2;
      if (count(mid) <= rounds * slots) hi = mid; else lo = mid + 1;
    }
    cand.push_back(lo);
  }
  int64_t best = cand[0], best_end = PrefillMakespan(items, cand[0], slots);
  for (size_t i = 1; i < cand.size(); ++i) {
    const int64_t end = PrefillMakespan(items, cand[i], slots);
    if (end < best_end || (end == best_end && cand[i] > best)) {
      best = cand[i];
      best_end = end;
    }
  }
  return best;
}

// Side by side or one after the other. A prefill call that also holds single-token sequences (a mixed worker step)
// runs MFMA-bound tile pieces and HBM-bound decode ranges. A tile workgroup needs a whole CU (two 256-register
// wavefronts per SIMD and 128 KB of LDS), so the two kinds cannot share CUs; but when the tile items are cut into fewer,
// longer pieces they hold only as many CUs as there are pieces, and decode ranges sized for the remaining CUs stream
// K/V on those, both in one launch (MixedAttentionKernel). ChooseOverlap estimates both schedules with rates measured
// on the MI355X -- a 64-key tile at head dim 256 takes ~3.7 us of a CU (less at smaller head dims), the decode stream
// reaches 5.6 TB/s on 256 CUs and falls off as (CUs / 256)^0.26 (5.2 TB/s on 192), and the merged launch costs ~3 us
// more than its longer side -- and keeps the cheaper. Config 5 (48 decode rows over 831 MB of K/V, two 512-token
// chunks): 64 pieces beside decode ranges for the other 191 CUs. The decode side needs page sizes that are multiples
// of 16 (its fast-page form).
struct OverlapChoice {
  bool use = false;
  int64_t target = 0;    // piece size (tiles) of the tile kernel
  uint32_t dec_cus = 0;  // CUs the decode ranges are sized for
};

constexpr double kTileUsD256 = 3.7;
constexpr double kDecodeBytesPerUs = 5.6e6;
constexpr double kMixedLaunchUs = 3.0;

double TileUs(uint32_t head_dim) { return kTileUsD256 * (0.25 + 0.75 * head_dim / 256.0); }
double DecodeUs(double bytes, uint32_t cus_used, uint32_t cus) {
  return bytes / (kDecodeBytesPerUs * std::pow(static_cast<double>(cus_used) / cus, 0.26));
}

template <typename Items, typename Single>
OverlapChoice ChooseOverlap(const RoostPagedAttentionParams& p, const Items& items, int64_t serial_target, uint32_t cus,
                            Single single) {
  OverlapChoice best;
  double dec_bytes = 0.0;
  for (uint32_t b = 0; b < p.batch; ++b) {
    if (single(b)) dec_bytes += static_cast<double>(KvLenHost(p, b)) * VirtualHeads(p) * p.head_dim * 2.0 * 2.0;
  }
  if (dec_bytes == 0.0 || items.empty() || cus < 2 || p.page_size % 16 != 0) return best;
  int64_t longest = 0;
  for (const auto& it : items) longest = std::max(longest, ItemTiles(it.w));
  const double tile_us = TileUs(p.head_dim);
  double best_us = PrefillMakespan(items, serial_target, cus) * tile_us + DecodeUs(dec_bytes, cus, cus);
  for (int64_t k = 1; k <= 16; ++k) {
    const int64_t target = std::max<int64_t>(1, roost::CeilDiv(longest, k));
    int64_t pieces = 0, piece_max = 0;
    for (const auto& it : items) {
      const int64_t tiles = ItemTiles(it.w), n = Pieces(tiles, target);
      pieces += n;
      piece_max = std::max<int64_t>(piece_max, roost::CeilDiv(tiles, n));
    }
    if (pieces >= static_cast<int64_t>(cus)) break;
    const uint32_t left = cus - static_cast<uint32_t>(pieces);
    const double us = std::max(static_cast<double>(piece_max + kPfPieceCost) * tile_us, DecodeUs(dec_bytes, left, cus)) +
                      kMixedLaunchUs;
    if (us < best_us) {
      best_us = us;
      best.use = true;
      best.target = target;
      best.dec_cus = left;
    }
  }
  return best;
}

Layout PlanPrefill(const RoostPagedAttentionParams& p, uint32_t cus, unsigned char* host) {
  if (p.q.dtype == ROOST_DTYPE_F32) {  // no f32 MFMA tile kernel: every query token is a row of the f32 decode kernel
    Layout l = MakeLayout(0, 0, 0, 0, kPfRows, p.head_dim, ROOST_ATTENTION_PREFILL);
    AppendDecode(p, BuildDecodeAllTokens(p, cus), l, host);
    PlaceFloats(p, 0, l);
    return l;
  }
  const bool fast = PrefillFastPath(p);
  const int64_t tile_q = fast ? kPfTokens : kPrefillTileQ;
  struct Item {
    PrefillWork w;
    int64_t cost;
  };
  std::vector<Item> items;
  int64_t total_tiles = 0;
  const int32_t window = WindowOf(p);
  // A sequence with one query token (a decode row of a mixed step) sees every key whether causal or not: the decode
  // kernel streams it at HBM speed instead of a 64-row MFMA tile holding one row.
  auto single = [&](uint32_t b) { return p.q_indptr_host[b + 1] - p.q_indptr_host[b] == 1; };
  for (uint32_t b = 0; b < p.batch; ++b) {
    if (single(b)) continue;
    const int64_t n = p.q_indptr_host[b + 1] - p.q_indptr_host[b];
    const int64_t kv = KvLenHost(p, b);
    for (int64_t q0 = 0; q0 < n; q0 += tile_q) {
      const int64_t rows = std::min<int64_t>(tile_q, n - q0);
      int64_t kend = p.causal ? std::min<int64_t>(kv, kv - n + q0 + rows) : kv;
      if (kend < 0) kend = 0;
      // With a window the item's first query (position kv - n + q0) sees keys from kv - n + q0 - window on; the
      // range starts at that key rounded down to 16 (a 16-row group never straddles a page), and keys before it are
      // never read.
      int64_t kbeg = window < 0 ? 0 : std::max<int64_t>(0, kv - n + q0 - window) / 16 * 16;
      if (kbeg > kend) kbeg = kend;
      total_tiles += roost::CeilDiv(kend - kbeg, 64) * VirtualHeads(p);
      for (uint32_t h = 0; h < VirtualHeads(p); ++h) {  // item per group of kGroup query heads
        items.push_back(Item{PrefillWork{static_cast<int32_t>(b), static_cast<int32_t>(q0), static_cast<int32_t>(h),
                                         static_cast<int32_t>(rows), static_cast<int32_t>(kbeg),
                                         static_cast<int32_t>(kend), -1, kPieceFirst | kPieceLast},
                             kend - kbeg + 64});
      }
    }
  }
  std::vector<PrefillMerge> merges;
  int32_t slot = 0;
  OverlapChoice overlap;
  if (fast) {
    int64_t target = PrefillPieceTiles(items, total_tiles, cus);
    overlap = ChooseOverlap(p, items, target, cus, single);
    if (overlap.use) target = overlap.target;
    std::vector<Item> cut;
    cut.reserve(items.size());
    for (const Item& it : items) {
      const int64_t tiles = roost::CeilDiv(static_cast<int64_t>(it.w.kend - it.w.kbeg), 64);
      const int64_t pieces = std::min<int64_t>(roost::CeilDiv(tiles, target), kMaxMergeSplits);
      if (pieces <= 1) {
        cut.push_back(it);
        continue;
      }
      merges.push_back(PrefillMerge{it.w.seq, it.w.q0, it.w.kv_head, it.w.rows, slot, static_cast<int32_t>(pieces), {0, 0}});
      for (int64_t i = 0; i < pieces; ++i) {
        const int64_t t0 = tiles * i / pieces, t1 = tiles * (i + 1) / pieces;
        PrefillWork w = it.w;
        w.kbeg = static_cast<int32_t>(it.w.kbeg + t0 * 64);
        w.kend = static_cast<int32_t>(std::min<int64_t>(it.w.kbeg + t1 * 64, it.w.kend));
        w.slot = slot++;
        w.ends = (i == 0 ? kPieceFirst : 0) | (i == pieces - 1 ? kPieceLast : 0);
        cut.push_back(Item{w, (t1 - t0) * 64 + 64});
      }
    }
    items.swap(cut);
  }
  std::stable_sort(items.begin(), items.end(), [](const Item& a, const Item& b) { return a.cost > b.cost; });
  // Merges of exactly two pieces first: they run on the 8-rows-per-block form of the merge kernel.
  std::stable_partition(merges.begin(), merges.end(), [](const PrefillMerge& m) { return m.count == 2; });
  Layout l = MakeLayout(items.size(), 0, merges.size(), static_cast<uint64_t>(slot), kPfRows, p.head_dim,
                        ROOST_ATTENTION_PREFILL);
  l.merges_two = static_cast<uint64_t>(
      std::count_if(merges.begin(), merges.end(), [](const PrefillMerge& m) { return m.count == 2; }));
  if (host != nullptr) {
    auto* w = reinterpret_cast<PrefillWork*>(host);
    for (size_t i = 0; i < items.size(); ++i) w[i] = items[i].w;
    std::memcpy(host + l.merge_offset, merges.data(), merges.size() * sizeof(PrefillMerge));
  }
  const uint64_t prefill_floats = l.float_bytes;
  l.overlap = overlap.use ? 1u : 0u;
  // Side by side, a decode workgroup has 8 wavefronts and a CU to itself: ranges for dec_cus / 2 CUs at
  // kDecodeWgsPerCu 4-wavefront workgroups each are one range per free CU.
  AppendDecode(p, BuildDecode(p, overlap.use ? std::max(1u, overlap.dec_cus / kDecodeWgsPerCu) : cus, single), l, host);
  PlaceFloats(p, prefill_floats, l);
  return l;
}

uint32_t ComputeUnits(const RoostContext* ctx) { return ctx != nullptr && ctx->compute_units > 0 ? ctx->compute_units : 256; }

Layout PlanLayout(const RoostPagedAttentionParams& p, uint32_t cus, unsigned char* host) {
  return p.mode == ROOST_ATTENTION_DECODE ? PlanDecode(p, cus, host) : PlanPrefill(p, cus, host);
}

// ---- Device helpers --------------------------------------------------------------------------------------------------

struct KvView {
  const void* k;
  const void* v;
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  const int32_t* last_len;
  uint64_t pool_pages;  // pages the pools hold; page ids outside [0, pool_pages) are skipped
  uint32_t page_size;
  uint32_t kv_heads;    // real KV heads of the pools (their row strides)
  uint32_t hnd;
  uint32_t head_shift;  // the kernels work on groups of kGroup query heads ("virtual" KV heads, q_heads / kGroup of
                        // them); virtual head v reads the K/V rows of real head v >> head_shift
  uint32_t vheads;      // q_heads / kGroup
  const void* out_gate;  // the output gate ([tokens, q_heads * head_dim] in the output's type), or NULL for none
};

__device__ __forceinline__ uint32_t SeqKvLen(const KvView& kv, int32_t b, int32_t* p0) {
  const int32_t a = kv.kv_indptr[b];
  const int32_t e = kv.kv_indptr[b + 1];
  *p0 = a;
  const int32_t pages = e - a;
  if (pages <= 0) return 0;
  int32_t last = kv.last_len[b];
  last = last < 1 ? 1 : (last > static_cast<int32_t>(kv.page_size) ? static_cast<int32_t>(kv.page_size) : last);
  return static_cast<uint32_t>((pages - 1) * static_cast<int32_t>(kv.page_size) + last);
}

// Element offset of key `j` of a sequence (page table starting at entry p0) for KV head h, or -1 when its page id is
// outside the pool (a released or corrupt entry: the key is treated as absent instead of faulting).
template <int D>
__device__ __forceinline__ int64_t KeyRow(const KvView& kv, int32_t p0, uint32_t j, uint32_t h) {
  const uint32_t pi = j / kv.page_size;
  const uint32_t off = j - pi * kv.page_size;
  const int32_t page = kv.kv_indices[p0 + pi];
  if (page < 0 || static_cast<uint64_t>(page) >= kv.pool_pages) return -1;
  const uint64_t pg = static_cast<uint64_t>(page);
  const uint32_t hr = h >> kv.head_shift;
  const uint64_t row = kv.hnd ? (pg * kv.kv_heads + hr) * kv.page_size + off : (pg * kv.page_size + off) * kv.kv_heads + hr;
  return static_cast<int64_t>(row * D);
}

// Branch-free form for the prefill tile loads: key j (clamped into [0, key_end)) always yields a loadable offset;
// *ok says whether the key exists (j < key_end and its page id is inside the pool).
template <int D>
__device__ __forceinline__ uint64_t KeyRowSafe(const KvView& kv, int32_t p0, int32_t j, int32_t key_end, uint32_t h,
                                               bool* ok) {
  const uint32_t jc = static_cast<uint32_t>(min(j, key_end - 1));
  const uint32_t pi = jc / kv.page_size;
  const uint32_t off = jc - pi * kv.page_size;
  const int32_t page = kv.kv_indices[p0 + pi];
  const bool good = j < key_end && page >= 0 && static_cast<uint64_t>(page) < kv.pool_pages;
  *ok = good;
  const uint64_t pg = good ? static_cast<uint64_t>(page) : 0;
  const uint32_t hr = h >> kv.head_shift;
  const uint64_t row = kv.hnd ? (pg * kv.kv_heads + hr) * kv.page_size + off : (pg * kv.page_size + off) * kv.kv_heads + hr;
  return good ? row * D : 0;
}

template <typename T>
struct Vec;  // 16-byte vector of T, widened to float
template <>
struct Vec<uint16_t> {  // bf16
  static constexpr int N = 8;
  __device__ static void Widen(const uint4& r, float* f) {
    f[0] = Bf16LoToF32(r.x); f[1] = Bf16HiToF32(r.x);
    f[2] = Bf16LoToF32(r.y); f[3] = Bf16HiToF32(r.y);
    f[4] = Bf16LoToF32(r.z); f[5] = Bf16HiToF32(r.z);
    f[6] = Bf16LoToF32(r.w); f[7] = Bf16HiToF32(r.w);
  }
  __device__ static uint16_t Narrow(float x) { return F32ToBf16(x); }
};
template <>
struct Vec<float> {
  static constexpr int N = 4;
  __device__ static void Widen(const uint4& r, float* f) {
    f[0] = __uint_as_float(r.x); f[1] = __uint_as_float(r.y);
    f[2] = __uint_as_float(r.z); f[3] = __uint_as_float(r.w);
  }
  __device__ static float Narrow(float x) { return x; }
};

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// The output gate (SigmoidMul folded into the epilogue): output element e, already rounded to the output type, times
// sigmoid(gate[e]) with SigmoidMul's own arithmetic; unchanged without a gate. GateOut2 takes two packed bf16 pairs.
__device__ __forceinline__ u32x2_t GateOut2(const void* gate, uint64_t e, u32x2_t v) {
  if (gate == nullptr) return v;
  const u32x2_t g = *reinterpret_cast<const u32x2_t*>(static_cast<const uint16_t*>(gate) + e);
  return u32x2_t{GateMulBf16x2(v[0], g[0]), GateMulBf16x2(v[1], g[1])};
}
template <typename T>
__device__ __forceinline__ T GateOut(const void* gate, uint64_t e, T v) {
  return gate == nullptr ? v : GateMul(v, static_cast<const T*>(gate)[e]);
}
// The same in two steps, for epilogues that request the gate before their own loads land: the raw gate words of
// element e (zero without a gate), then the product.
__device__ __forceinline__ u32x2_t GateFetch2(const void* gate, uint64_t e) {
  return gate == nullptr ? u32x2_t{0, 0} : *reinterpret_cast<const u32x2_t*>(static_cast<const uint16_t*>(gate) + e);
}
__device__ __forceinline__ u32x2_t GateApply2(const void* gate, u32x2_t g, u32x2_t v) {
  return gate == nullptr ? v : u32x2_t{GateMulBf16x2(v[0], g[0]), GateMulBf16x2(v[1], g[1])};
}
template <typename T>
__device__ __forceinline__ T GateFetch(const void* gate, uint64_t e) {
  return gate == nullptr ? T{} : static_cast<const T*>(gate)[e];
}
template <typename T>
__device__ __forceinline__ T GateApply(const void* gate, T g, T v) {
  return gate == nullptr ? v : GateMul(v, g);
}

// 16-byte load with the non-temporal hint, for data read exactly once in whole cache lines per instruction (decode V:
// 2 tokens x 512 contiguous bytes per wavefront load). Keeping such a stream out of the caches raises the rate of a
// random-16 KB-page read on the MI355X from about 5.9 to 6.8 TB/s (measured). Decode K is read 64 bytes per token per
// instruction (the MFMA operand layout), so the other half of each 128-byte line is read by the next instruction: K
// stays on plain loads, where that second half hits in L2.
__device__ __forceinline__ uint4 LoadStream16(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// Partial dot product of a 16-byte K vector with the matching 16 bytes of q (both bf16; q kept as packed pairs).
__device__ __forceinline__ float Dot16(const uint4& k, const uint32_t* q, float acc) {
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, k.x), __builtin_bit_cast(bf16x2_t, q[0]), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, k.y), __builtin_bit_cast(bf16x2_t, q[1]), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, k.z), __builtin_bit_cast(bf16x2_t, q[2]), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, k.w), __builtin_bit_cast(bf16x2_t, q[3]), acc, false);
  return acc;
}
__device__ __forceinline__ float Dot16(const uint4& k, const float* q, float acc) {
  acc = fmaf(__uint_as_float(k.x), q[0], acc);
  acc = fmaf(__uint_as_float(k.y), q[1], acc);
  acc = fmaf(__uint_as_float(k.z), q[2], acc);
  acc = fmaf(__uint_as_float(k.w), q[3], acc);
  return acc;
}

__device__ __forceinline__ float ShflXor(float v, int mask) { return __shfl_xor(v, mask, 64); }

// A lane's value combined with that of lane ^ 32 through v_permlane32_swap (registers only, no LDS round trip): the
// swap leaves each lane holding both values, so max and sum need no select and both lanes get the same bits.
__device__ __forceinline__ float MaxXor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float SumXor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// x[i] for a runtime i in [0, 4) without indexing a register array (which would spill it to scratch).
__device__ __forceinline__ float Pick4(const float* x, int i) {
  return i == 0 ? x[0] : (i == 1 ? x[1] : (i == 2 ? x[2] : x[3]));
}

// ---- Decode kernel ---------------------------------------------------------------------------------------------------

template <typename T, int D>
struct DecodeCfg {
  static constexpr int kVec = Vec<T>::N;            // elements per 16-byte vector
  static constexpr int kLpr = D / kVec;              // lanes per K/V row
  static constexpr int kTpi = 64 / kLpr;             // rows (tokens) per wave-wide load
  static constexpr int kNi = 16 / kTpi;              // loads per 16-token group per lane
  static constexpr int kQWords = sizeof(T) == 2 ? kVec / 2 : kVec;  // q registers per head
  static_assert(kLpr <= 64 && 64 % kLpr == 0 && 16 % kTpi == 0, "shape");
  static_assert(kNi * kGroup == kLpr, "each lane must end the reduce-scatter with one (token, head) score");
};

// One wavefront's running state: acc[h][e] is this lane's slice of sum_j p_j v_j for query head h, m[h] the running
// max of the head (wave-uniform), l_lane this lane's share of the head-(r % 4) denominator.
template <typename T, int D>
struct DecodeState {
  float acc[kGroup][DecodeCfg<T, D>::kVec];
  float m[kGroup];
  float l_lane;
};

// Folds one 16-token group (already in registers) into the state.
//
// Lane (ri, r) holds, for K, the 16-byte slice r of token slot i ^ (r >> 2) in register i, and q of head h ^ (r & 3)
// in register h; so its partial score register j = 4i + h stands for the logical (slot, head) index j ^ r. With that
// permutation the reduce-scatter needs no selects: at distance mk the partner's register j + mk stands for the same
// logical index as this lane's register j, so s[j] += partner.s[j + mk]; afterwards register 0 holds the complete score
// of index r (slot r / 4, head r % 4). V register i holds slot i in natural order.
// valid: bit s set when token slot s of this lane's row group is a real key.
template <typename T, int D, typename QW>
__device__ __forceinline__ void DecodeGroup(DecodeState<T, D>& st, const uint4* kr, const uint4* vr, uint32_t valid,
                                            const QW (*qr)[DecodeCfg<T, D>::kQWords], float* x_row, int r, int ri,
                                            int lane, float scale_log2, SoftCap cap) {
  using C = DecodeCfg<T, D>;
  constexpr int kVec = C::kVec, kLpr = C::kLpr, kNi = C::kNi;
  float s[kLpr];
#pragma unroll
  for (int i = 0; i < kNi; ++i)
#pragma unroll
    for (int h = 0; h < (int)kGroup; ++h) s[i * kGroup + h] = Dot16(kr[i], qr[h], 0.0f);
#pragma unroll
  for (int mk = kLpr / 2; mk >= 1; mk >>= 1)
#pragma unroll
    for (int j = 0; j < mk; ++j) s[j] += ShflXor(s[j + mk], mk);
  const int my_head = r % kGroup;
  const bool my_valid = (valid >> (r / kGroup)) & 1u;
  float y = s[0] * scale_log2;
  if (cap.capl != 0.0f) y = Capped(y, cap);
  const float sc = my_valid ? y : -INFINITY;
  // Group max per head (lanes sharing r % 4), then every lane learns all 4.
  float gm = sc;
#pragma unroll
  for (int mk = 4; mk < 64; mk <<= 1) gm = fmaxf(gm, ShflXor(gm, mk));
  const float x1 = ShflXor(gm, 1), x2 = ShflXor(gm, 2), x3 = ShflXor(gm, 3);
  float corr[kGroup];
  bool rescale = false;
#pragma unroll
  for (int h = 0; h < (int)kGroup; ++h) {
    const int dd = h ^ my_head;
    const float hm = dd == 0 ? gm : (dd == 1 ? x1 : (dd == 2 ? x2 : x3));
    const float mn = fmaxf(st.m[h], hm);
    corr[h] = mn == -INFINITY ? 1.0f : exp2f(st.m[h] - mn);
    rescale |= mn != st.m[h];
    st.m[h] = mn;
  }
  const float pw = sc == -INFINITY ? 0.0f : exp2f(sc - Pick4(st.m, my_head));
  st.l_lane = st.l_lane * Pick4(corr, my_head) + pw;
  if (rescale) {
#pragma unroll
    for (int h = 0; h < (int)kGroup; ++h)
#pragma unroll
      for (int e = 0; e < kVec; ++e) st.acc[h][e] *= corr[h];
  }
  if constexpr (sizeof(T) == 2) {
    // bf16: the weights of slots 2a and 2a+1 (lanes r and r ^ 4) travel as one packed bf16 pair per head, and P.V runs
    // on v_dot2 over token pairs (P rounded to bf16 before the product, fp32 accumulation).
    const float po = ShflXor(pw, 4);
    auto* xw = reinterpret_cast<uint32_t*>(x_row);
    if ((r & 4) == 0) xw[ri * (kLpr / 2) + (r >> 3) * kGroup + my_head] = PackBf16(pw, po);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    uint32_t pp[kNi / 2][kGroup];
#pragma unroll
    for (int a = 0; a < kNi / 2; ++a) {
      const uint4 t4 = *reinterpret_cast<const uint4*>(&xw[ri * (kLpr / 2) + a * kGroup]);
      pp[a][0] = t4.x; pp[a][1] = t4.y; pp[a][2] = t4.z; pp[a][3] = t4.w;
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int a = 0; a < kNi / 2; ++a) {
      const uint32_t* v0 = reinterpret_cast<const uint32_t*>(&vr[2 * a]);
      const uint32_t* v1 = reinterpret_cast<const uint32_t*>(&vr[2 * a + 1]);
#pragma unroll
      for (int w = 0; w < kVec / 2; ++w) {
        const uint32_t lo = __builtin_amdgcn_perm(v1[w], v0[w], 0x05040100u);  // (v[2a][2w], v[2a+1][2w])
        const uint32_t hi = __builtin_amdgcn_perm(v1[w], v0[w], 0x07060302u);  // (v[2a][2w+1], v[2a+1][2w+1])
#pragma unroll
        for (int h = 0; h < (int)kGroup; ++h) {
          const bf16x2_t ph = __builtin_bit_cast(bf16x2_t, pp[a][h]);
          st.acc[h][2 * w] = __builtin_amdgcn_fdot2_f32_bf16(ph, __builtin_bit_cast(bf16x2_t, lo), st.acc[h][2 * w], false);
          st.acc[h][2 * w + 1] =
              __builtin_amdgcn_fdot2_f32_bf16(ph, __builtin_bit_cast(bf16x2_t, hi), st.acc[h][2 * w + 1], false);
        }
      }
    }
  } else {
    x_row[lane] = pw;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float pv[kLpr];
#pragma unroll
    for (int i = 0; i < kLpr; i += 4) {
      const float4 t4 = *reinterpret_cast<const float4*>(&x_row[ri * kLpr + i]);
      pv[i] = t4.x; pv[i + 1] = t4.y; pv[i + 2] = t4.z; pv[i + 3] = t4.w;
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < kNi; ++i) {
      float vf[kVec];
      Vec<T>::Widen(vr[i], vf);
#pragma unroll
      for (int h = 0; h < (int)kGroup; ++h) {
        const float w = pv[i * kGroup + h];
#pragma unroll
        for (int e = 0; e < kVec; ++e) st.acc[h][e] = fmaf(w, vf[e], st.acc[h][e]);
      }
    }
  }
}

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// bf16 form of one 16-token group. q.k runs on v_mfma_f32_16x16x32_bf16 with the 16 tokens on M and the 4 query heads
// (padded to 16 with zero columns) on N: K register kc of lane l holds token l % 16, dims 32*kc + 8*(l / 16) .. +8,
// q register kc the same dims of head l % 16 (zero for l % 16 >= 4), and the result lane l holds the scores of tokens
// 4*(l / 16) + j, j = 0..3, for head l % 16. No cross-lane reduction is needed for the scores; the per-head maximum is
// two exchanges and four readlanes, so the running maxima are wave-uniform scalars. The weights go through 256 bytes of
// LDS into the P.V layout (lane (ri, r): V register i = token kTpi*i + ri, 16-byte slice r), where P.V runs on v_dot2
// over token pairs with P rounded to bf16 and fp32 accumulation.
template <int D>
__device__ __forceinline__ void DecodeGroupMfma(DecodeState<uint16_t, D>& st, const uint4* kr, const uint4* vr,
                                                uint32_t validmask, const u32x4_t* qb, float* x_row, int r, int ri,
                                                int lane, float scale_log2, SoftCap cap) {
  using C = DecodeCfg<uint16_t, D>;
  constexpr int kVec = C::kVec, kTpi = C::kTpi, kNi = C::kNi, kChunks = D / 32;
  f32x4_t acc4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int kc = 0; kc < kChunks; ++kc) {
    acc4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kr[kc]),
                                                    __builtin_bit_cast(bf16x8_t, qb[kc]), acc4, 0, 0, 0);
  }
  const int col = lane & 15;
  const int tok0 = (lane >> 4) * 4;
  float sc[4];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool ok = col < (int)kGroup && ((validmask >> (tok0 + j)) & 1u);
    float y = acc4[j] * scale_log2;
    if (cap.capl != 0.0f) y = Capped(y, cap);
    sc[j] = ok ? y : -INFINITY;
    mx = fmaxf(mx, sc[j]);
  }
  mx = fmaxf(mx, ShflXor(mx, 16));
  mx = MaxXor32(mx);
  float corr[kGroup];
  bool rescale = false;
#pragma unroll
  for (int h = 0; h < (int)kGroup; ++h) {
    const float hm = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), h));  // lane h holds head h
    const float mn = fmaxf(st.m[h], hm);
    corr[h] = mn == -INFINITY ? 1.0f : exp2f(st.m[h] - mn);
    rescale |= mn != st.m[h];
    st.m[h] = mn;
  }
  const float mine = Pick4(st.m, col & 3);
  float pf[4];
  float psum = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    pf[j] = sc[j] == -INFINITY ? 0.0f : exp2f(sc[j] - mine);
    psum += pf[j];
  }
  st.l_lane = st.l_lane * Pick4(corr, col & 3) + psum;
  if (rescale) {
#pragma unroll
    for (int h = 0; h < (int)kGroup; ++h)
#pragma unroll
      for (int e = 0; e < kVec; ++e) st.acc[h][e] *= corr[h];
  }
  // Weights to LDS as [token][head] floats, then each P.V lane packs the bf16 pairs it needs.
  if (col < (int)kGroup) {
#pragma unroll
    for (int j = 0; j < 4; ++j) x_row[(tok0 + j) * kGroup + col] = pf[j];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  uint32_t pp[kNi / 2][kGroup];
#pragma unroll
  for (int a = 0; a < kNi / 2; ++a) {
    const float4 p0 = *reinterpret_cast<const float4*>(&x_row[(kTpi * (2 * a) + ri) * kGroup]);
    const float4 p1 = *reinterpret_cast<const float4*>(&x_row[(kTpi * (2 * a + 1) + ri) * kGroup]);
    pp[a][0] = PackRne(p0.x, p1.x);
    pp[a][1] = PackRne(p0.y, p1.y);
    pp[a][2] = PackRne(p0.z, p1.z);
    pp[a][3] = PackRne(p0.w, p1.w);
  }
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int a = 0; a < kNi / 2; ++a) {
    const uint32_t* v0 = reinterpret_cast<const uint32_t*>(&vr[2 * a]);
    const uint32_t* v1 = reinterpret_cast<const uint32_t*>(&vr[2 * a + 1]);
#pragma unroll
    for (int w = 0; w < kVec / 2; ++w) {
      const uint32_t lo = __builtin_amdgcn_perm(v1[w], v0[w], 0x05040100u);
      const uint32_t hi = __builtin_amdgcn_perm(v1[w], v0[w], 0x07060302u);
#pragma unroll
      for (int h = 0; h < (int)kGroup; ++h) {
        const bf16x2_t ph = __builtin_bit_cast(bf16x2_t, pp[a][h]);
        st.acc[h][2 * w] = __builtin_amdgcn_fdot2_f32_bf16(ph, __builtin_bit_cast(bf16x2_t, lo), st.acc[h][2 * w], false);
        st.acc[h][2 * w + 1] =
            __builtin_amdgcn_fdot2_f32_bf16(ph, __builtin_bit_cast(bf16x2_t, hi), st.acc[h][2 * w + 1], false);
      }
    }
  }
  (void)r;
}

// A workgroup barrier that orders LDS only: the wavefront's LDS operations complete, global loads and stores stay in
// flight. `__syncthreads()` also waits for every outstanding global access (`vmcnt(0)`); at a piece's end that is the
// round trip of its output stores and of the ring's loads past the piece's last group, none of which the barrier
// protects. The empty asm's memory clobber keeps the compiler from moving memory operations across it.
__device__ __forceinline__ void LdsBarrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left at their maxima
  asm volatile("s_barrier" ::: "memory");
}

// Split-K paged decode. kFastPage: page_size is a multiple of 16, so a 16-token group (16-aligned within its
// sequence) lies in one page and its page id is one wave-uniform scalar load; otherwise each lane looks its own
// token's page up. Loads are branch-free (an absent key reads a valid address and is masked) and the next group's
// K/V is fetched into a second register buffer while the current group is computed. Workgroup (range, KV head)
// processes the pieces of its range in turn; a piece that is not a whole sequence writes fp32 partials that
// DecodeMergeKernel combines in key order.
template <typename T, int D, bool kFastPage, int kWaves>
__device__ __forceinline__ void DecodeBody(const T* __restrict__ q, T* __restrict__ out, float* __restrict__ lse,
                                           KvView kv, const int32_t* __restrict__ kv_indices,
                                           const DecodeWork* __restrict__ work, const int32_t* __restrict__ range_ptr,
                                           float* __restrict__ part_o, float* __restrict__ part_ml,
                                           const int32_t* __restrict__ q_rows, uint32_t q_heads, uint32_t heads_per_wg,
                                           float scale_log2, int32_t window, uint32_t causal, SoftCap cap,
                                           uint32_t block, float* x_lds, float* m_lds, float* l_lds, float* o_lds) {
  // LDS (the caller's): x_lds [kWaves][64], m_lds and l_lds [kWaves][kGroup], o_lds [kWaves][kGroup][D] floats.
  using C = DecodeCfg<T, D>;
  constexpr int kVec = C::kVec, kLpr = C::kLpr, kTpi = C::kTpi, kNi = C::kNi;
  constexpr bool kMfma = sizeof(T) == 2;  // bf16: q.k on MFMA; f32: the VALU reduce-scatter path

  // Both KV heads of a range are adjacent in launch order, so the two halves of each NHD page row are read together.
  // A workgroup serves heads_per_wg (1, 2 or 4) KV heads of one range, 4 / heads_per_wg wavefronts per head, so the
  // KV heads of each page row (adjacent in an NHD pool) are read by one CU at the same time.
  const uint32_t hblocks = kv.vheads / heads_per_wg;
  const uint32_t range = block / hblocks;
  const int lane = threadIdx.x & 63;
  // The wavefront index is uniform within a wavefront; saying so lets the group's page id be a scalar load.
  const int wave_id = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t kvh = (block % hblocks) * heads_per_wg + wave_id % heads_per_wg;
  const int wave = wave_id / static_cast<int>(heads_per_wg);           // index among this head's wavefronts
  const int waves_per_head = kWaves / static_cast<int>(heads_per_wg);
  const int r = lane % kLpr;   // which 16-byte slice of a row
  const int ri = lane / kLpr;  // which row of a wave-wide load
  const int kperm = r / static_cast<int>(kGroup);  // this lane's token-slot permutation for K
  const T* kbase = static_cast<const T*>(kv.k);
  const T* vbase = static_cast<const T*>(kv.v);

  const int32_t it_end = range_ptr[range + 1];
  for (int32_t it = range_ptr[range]; it < it_end; ++it) {
  const DecodeWork wk = work[it];
  int32_t p0 = 0;
  const uint32_t kv_len = SeqKvLen(kv, wk.seq, &p0);
  // The row's query token: its sequence's index in a decode call; in a prefill call q_back tokens before the
  // sequence's last, q_indptr[seq + 1] - 1 (the last token; the only one of a single-token sequence).
  // (Clamped into the sequence's own rows, so that device tables that disagree with the plan cannot move it outside.)
  const uint64_t tok = q_rows != nullptr
                           ? static_cast<uint64_t>(max(q_rows[wk.seq], q_rows[wk.seq + 1] - 1 - wk.q_back))
                           : static_cast<uint64_t>(wk.seq);
  // The query's position; it sees keys up to itself (causal) or all of them, and from its window start on.
  const int32_t qpos = static_cast<int32_t>(kv_len) - 1 - wk.q_back;
  const uint32_t t_begin = static_cast<uint32_t>(wk.token_begin);
  uint32_t t_end = min(kv_len, static_cast<uint32_t>(wk.token_end));
  if (causal) t_end = min(t_end, static_cast<uint32_t>(max(0, qpos + 1)));
  // The sliding window's first visible key; the piece may start up to 15 keys before it, which are masked.
  const uint32_t lo = window < 0 || kv_len == 0 ? 0u : static_cast<uint32_t>(max(0, qpos - window));

  using QW = typename std::conditional<sizeof(T) == 2, uint32_t, float>::type;
  QW qr[kGroup][C::kQWords];   // VALU path (f32)
  u32x4_t qb[kMfma ? D / 32 : 1];  // MFMA path (bf16): B operand of q.k
  if constexpr (kMfma) {
    const int col = lane & 15;
    const T* qrow = q + (tok * q_heads + kvh * kGroup + (col & 3)) * D + (lane >> 4) * 8;
#pragma unroll
    for (int kc = 0; kc < D / 32; ++kc) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(qrow + kc * 32);
      qb[kc] = col < (int)kGroup ? v : u32x4_t{0, 0, 0, 0};
    }
  } else {
    const T* qrow = q + (tok * q_heads + kvh * kGroup) * D + r * kVec;
#pragma unroll
    for (int h = 0; h < (int)kGroup; ++h) {
      const uint4 v = *reinterpret_cast<const uint4*>(qrow + (h ^ (r & 3)) * D);
      const QW* w = reinterpret_cast<const QW*>(&v);
#pragma unroll
      for (int i = 0; i < C::kQWords; ++i) qr[h][i] = w[i];
    }
  }

  DecodeState<T, D> st;
#pragma unroll
  for (int h = 0; h < (int)kGroup; ++h) {
    st.m[h] = -INFINITY;
#pragma unroll
    for (int e = 0; e < kVec; ++e) st.acc[h][e] = 0.0f;
  }
  st.l_lane = 0.0f;

  // Byte stride between the rows of consecutive tokens of one KV head inside a page.
  const uint32_t tok_bytes = (kv.hnd ? D : kv.kv_heads * D) * static_cast<uint32_t>(sizeof(T));
  // Group gi (0-based, 16 tokens) of this wavefront: key g = t_begin + 16 * (wave + waves_per_head * gi).
  const uint32_t ngroups = (t_end > t_begin) ? (t_end - t_begin + 15) / 16 : 0;
  const uint32_t nw = ngroups > static_cast<uint32_t>(wave)
                          ? (ngroups - wave + waves_per_head - 1) / waves_per_head : 0;
  // Every load is unconditional: a group index past the end is clamped to the wave's last group and its keys are
  // masked, so the number of loads in flight is the same on every path and the compiler can wait for exactly the
  // current group's data (vmcnt) while the next group's loads stay in flight.
  auto load = [&](uint32_t gi, uint4* kr, uint4* vr, uint32_t& valid) {
    valid = 0;
    const uint32_t g0 = t_begin + 16u * (wave + waves_per_head * min(gi, nw - 1));
    const bool live = gi < nw;
    if constexpr (kFastPage) {
      const uint32_t pi = g0 / kv.page_size;
      const uint32_t off0 = g0 - pi * kv.page_size;
      const int32_t page = kv_indices[p0 + pi];  // uniform address: a scalar load
      const bool page_ok = page >= 0 && static_cast<uint64_t>(page) < kv.pool_pages;
      const uint64_t pg = page_ok ? static_cast<uint64_t>(page) : 0;
      const uint32_t kvr = kvh >> kv.head_shift;  // the real KV head this group of query heads reads
      const uint64_t row0 = kv.hnd ? (pg * kv.kv_heads + kvr) * kv.page_size + off0
                                   : (pg * kv.page_size + off0) * kv.kv_heads + kvr;
      const char* kg = reinterpret_cast<const char*>(kbase + row0 * D);
      const char* vg = reinterpret_cast<const char*>(vbase + row0 * D);
#pragma unroll
      for (int i = 0; i < kNi; ++i) {
        const uint32_t tv = i * kTpi + ri;  // V register i: slot i
        const bool okv = live && page_ok && g0 + tv < t_end && g0 + tv >= lo;
        vr[i] = LoadStream16(vg + ((okv ? tv : 0) * tok_bytes + r * 16));
        if constexpr (kMfma) {
          const uint32_t tk = lane & 15;  // K register i: dims 32 i + 8 (lane / 16) of token lane % 16
          const bool okk = page_ok && g0 + tk < t_end;
          kr[i] = *reinterpret_cast<const uint4*>(kg + ((okk ? tk : 0) * tok_bytes + i * 64 + (lane >> 4) * 16));
        } else {
          const uint32_t tk = (i ^ kperm) * kTpi + ri;  // K register i: slot i ^ kperm
          const bool okk = page_ok && g0 + tk < t_end;
          kr[i] = LoadStream16(kg + ((okk ? tk : 0) * tok_bytes + r * 16));
          valid |= static_cast<uint32_t>(okv) << i;
        }
      }
      if constexpr (kMfma) {
        const uint32_t n = live && page_ok ? min(16u, t_end - g0) : 0u;
        valid = (1u << n) - 1u;  // bit t: token t of the group is a real key
        if (g0 < lo) valid &= ~((1u << min(16u, lo - g0)) - 1u);  // before the window
      }
    } else {
      bool kok = false;
#pragma unroll
      for (int i = 0; i < kNi; ++i) {
        bool okk, okv;
        const int32_t tk = kMfma ? static_cast<int32_t>(g0 + (lane & 15))
                                 : static_cast<int32_t>(g0 + (i ^ kperm) * kTpi + ri);
        const uint64_t rowk = KeyRowSafe<D>(kv, p0, tk, static_cast<int32_t>(t_end), kvh, &okk);
        const uint64_t rowv = KeyRowSafe<D>(kv, p0, static_cast<int32_t>(g0 + i * kTpi + ri),
                                            static_cast<int32_t>(t_end), kvh, &okv);
        okk = okk && tk >= static_cast<int32_t>(lo);
        okv = okv && g0 + i * kTpi + ri >= lo;
        kr[i] = *reinterpret_cast<const uint4*>(kMfma ? kbase + rowk + i * 32 + (lane >> 4) * 8 : kbase + rowk + r * kVec);
        vr[i] = LoadStream16(vbase + rowv + r * kVec);
        if constexpr (!kMfma) valid |= static_cast<uint32_t>(okv && live) << i;
        kok = okk;
      }
      if constexpr (kMfma) {
        // Lanes 0..15 hold tokens 0..15 of the group: their K validity is the key mask.
        valid = static_cast<uint32_t>(__ballot(kok && live)) & 0xFFFFu;
      }
    }
  };

  if (nw > 0) {
    // A ring of kDecodeRing register buffers: group gi is computed while groups gi+1 .. gi+kDecodeRing-1 are in
    // flight (kDecodeRing - 1 groups of 16 loads stay below the 63 outstanding vector loads a wavefront can count).
    uint4 kbuf[kDecodeRing][kNi], vbuf[kDecodeRing][kNi];
    uint32_t valid[kDecodeRing];
#pragma unroll
    for (int s = 0; s < kDecodeRing - 1; ++s) load(s, kbuf[s], vbuf[s], valid[s]);
    for (uint32_t gi = 0; gi < nw; gi += kDecodeRing) {
#pragma unroll
      for (int s = 0; s < kDecodeRing; ++s) {
        constexpr int kLast = kDecodeRing - 1;
        const int nxt = (s + kLast) % kDecodeRing;
        load(gi + s + kLast, kbuf[nxt], vbuf[nxt], valid[nxt]);
        if (gi + s < nw) {
          if constexpr (kMfma) {
            DecodeGroupMfma<D>(st, kbuf[s], vbuf[s], valid[s], qb, x_lds + 64 * wave_id, r, ri, lane, scale_log2, cap);
          } else {
            DecodeGroup<T, D, QW>(st, kbuf[s], vbuf[s], valid[s], qr, x_lds + 64 * wave_id, r, ri, lane, scale_log2, cap);
          }
        }
      }
    }
  }

  // Wave: fold the row groups (lanes sharing r) and total the per-lane denominators per head.
#pragma unroll
  for (int mk = kLpr; mk < 64; mk <<= 1)
#pragma unroll
    for (int h = 0; h < (int)kGroup; ++h)
#pragma unroll
      for (int e = 0; e < kVec; ++e) st.acc[h][e] += ShflXor(st.acc[h][e], mk);
  // Per-lane denominators: VALU path, lanes with r % 4 == h hold head h; MFMA path, lanes with lane % 16 == h.
  float lsum = st.l_lane;
#pragma unroll
  for (int mk = kMfma ? 16 : 4; mk < 64; mk <<= 1) lsum += ShflXor(lsum, mk);
  if (lane < (int)kGroup) {
    m_lds[wave_id * kGroup + lane] = Pick4(st.m, lane);
    l_lds[wave_id * kGroup + lane] = lsum;  // lane h holds the total of head h
  }
  if (ri == 0) {
#pragma unroll
    for (int h = 0; h < (int)kGroup; ++h)
#pragma unroll
      for (int e = 0; e < kVec; ++e) o_lds[(wave_id * kGroup + h) * D + r * kVec + e] = st.acc[h][e];
  }
  LdsBarrier();

  // Workgroup: merge the wavefronts of each KV head, then write the final row or this piece's partial.
  const int split = wk.slot;
  for (int idx = threadIdx.x; idx < (int)(heads_per_wg * kGroup * D); idx += 64 * kWaves) {
    const int hk = idx / (kGroup * D);  // local KV head: wavefronts hk, hk + heads_per_wg, ...
    const int h = (idx / D) % kGroup;
    const int d = idx % D;
    float M = -INFINITY;
    for (int w = hk; w < kWaves; w += heads_per_wg) M = fmaxf(M, m_lds[w * kGroup + h]);
    float o = 0.0f, L = 0.0f;
    for (int w = hk; w < kWaves; w += heads_per_wg) {
      const float f = m_lds[w * kGroup + h] == -INFINITY ? 0.0f : exp2f(m_lds[w * kGroup + h] - M);
      o += o_lds[(w * kGroup + h) * D + d] * f;
      L += l_lds[w * kGroup + h] * f;
    }
    const uint32_t qh = ((block % hblocks) * heads_per_wg + hk) * kGroup + h;
    if (split < 0) {
      const uint64_t row = tok * q_heads + qh;
      out[row * D + d] = GateOut<T>(kv.out_gate, row * D + d, Vec<T>::Narrow(L > 0.0f ? o / L : 0.0f));
      if (lse != nullptr && d == 0) lse[row] = L > 0.0f ? M + log2f(L) : -INFINITY;
    } else {
      const uint64_t prow = static_cast<uint64_t>(split) * q_heads + qh;
      part_o[prow * D + d] = o;
      if (d == 0) {
        part_ml[prow * 2] = M;
        part_ml[prow * 2 + 1] = L;
      }
    }
  }
  LdsBarrier();  // the next piece reuses the LDS merge buffers
  }
}


// Split-K paged decode, one workgroup of 4 wavefronts per (range, head block): DecodeBody with LDS of its own.
template <typename T, int D, bool kFastPage>
__global__ void __launch_bounds__(256, kDecodeWgsPerCu) DecodeKernel(const T* __restrict__ q, T* __restrict__ out, float* __restrict__ lse,
                                                    KvView kv, const int32_t* __restrict__ kv_indices,
                                                    const DecodeWork* __restrict__ work,
                                                    const int32_t* __restrict__ range_ptr,
                                                    float* __restrict__ part_o, float* __restrict__ part_ml,
                                                    const int32_t* __restrict__ q_rows,
                                                    uint32_t q_heads, uint32_t heads_per_wg, float scale_log2,
                                                    int32_t window, uint32_t causal, SoftCap cap) {
  __shared__ float x_lds[4][64];
  __shared__ float m_lds[4][kGroup];
  __shared__ float l_lds[4][kGroup];
  __shared__ float o_lds[4][kGroup][D];
  DecodeBody<T, D, kFastPage, 4>(q, out, lse, kv, kv_indices, work, range_ptr, part_o, part_ml, q_rows, q_heads,
                                 heads_per_wg, scale_log2, window, causal, cap, blockIdx.x, &x_lds[0][0], &m_lds[0][0],
                                 &l_lds[0][0], &o_lds[0][0][0]);
}

// Combines the pieces of each split sequence in key order: one workgroup per (sequence, query head), D threads, one
// output element each. Wavefront 0 computes the per-piece rescale factors into LDS (lanes over pieces), then every
// thread sums its element over the pieces with independent loads.
struct DecodeMergeArgs {
  const DecodeMerge* merges;
  const float* part_o;
  const float* part_ml;
  const int32_t* q_rows;  // the call's q_indptr in a prefill call, NULL in a decode call
};

template <typename T, int D>
__device__ __forceinline__ void DecodeMergeBody(T* __restrict__ out, float* __restrict__ lse, const DecodeMergeArgs& m,
                                                uint32_t q_heads, const void* out_gate, uint32_t bx) {
  __shared__ float f_lds[kMaxMergeSplits];
  __shared__ float inv_lds;
  const float* __restrict__ part_o = m.part_o;
  const float* __restrict__ part_ml = m.part_ml;
  const int32_t* __restrict__ q_rows = m.q_rows;
  const DecodeMerge mg = m.merges[bx / q_heads];
  const uint64_t tok = q_rows != nullptr
                           ? static_cast<uint64_t>(max(q_rows[mg.seq], q_rows[mg.seq + 1] - 1 - mg.q_back))
                           : static_cast<uint64_t>(mg.seq);
  const uint32_t qh = bx % q_heads;
  const int n = min(mg.count, static_cast<int32_t>(kMaxMergeSplits));
  const uint64_t base = static_cast<uint64_t>(mg.first) * q_heads + qh;  // partial row of piece c: base + c * q_heads
  // This thread's partial outputs of the first kPre pieces are requested first, so that they arrive while the pieces'
  // weights are being computed (a sequence is usually cut into fewer than kPre pieces).
  constexpr int kPre = 16;
  const int d = threadIdx.x;
  const float* po = part_o + base * D + d;
  const uint64_t step = static_cast<uint64_t>(q_heads) * D;
  const uint64_t e = (tok * q_heads + qh) * D + d;
  const T gv = GateFetch<T>(out_gate, e);  // requested with the partials, applied at the end
  float pre[kPre];
#pragma unroll
  for (int c = 0; c < kPre; ++c) pre[c] = c < n ? po[c * step] : 0.0f;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    // Piece `lane` (and lane + 64, ... for longer splits): its max and sum, read once.
    const float m0 = lane < n ? part_ml[(base + static_cast<uint64_t>(lane) * q_heads) * 2] : -INFINITY;
    const float l0 = lane < n ? part_ml[(base + static_cast<uint64_t>(lane) * q_heads) * 2 + 1] : 0.0f;
    float M = m0;
    for (int c = lane + 64; c < n; c += 64) M = fmaxf(M, part_ml[(base + static_cast<uint64_t>(c) * q_heads) * 2]);
    for (int mk = 32; mk >= 1; mk >>= 1) M = fmaxf(M, __shfl_xor(M, mk, 64));
    float L = 0.0f;
    if (lane < n) {
      const float f = m0 == -INFINITY ? 0.0f : exp2f(m0 - M);
      f_lds[lane] = f;
      L = l0 * f;
    }
    for (int c = lane + 64; c < n; c += 64) {
      const uint64_t prow = base + static_cast<uint64_t>(c) * q_heads;
      const float mc = part_ml[prow * 2];
      const float f = mc == -INFINITY ? 0.0f : exp2f(mc - M);
      f_lds[c] = f;
      L += part_ml[prow * 2 + 1] * f;
    }
    for (int mk = 32; mk >= 1; mk >>= 1) L += __shfl_xor(L, mk, 64);
    if (lane == 0) {
      inv_lds = L > 0.0f ? 1.0f / L : 0.0f;
      if (lse != nullptr) lse[tok * q_heads + qh] = L > 0.0f ? M + log2f(L) : -INFINITY;
    }
  }
  __syncthreads();
  // Pieces in key order, piece c into accumulator c % 4 (a fixed order: deterministic).
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int c = 0; c < kPre; ++c) {
    if (c < n) acc[c & 3] = fmaf(pre[c], f_lds[c], acc[c & 3]);
  }
  for (int c = kPre; c < n; ++c) acc[c & 3] = fmaf(po[c * step], f_lds[c], acc[c & 3]);
  const float o0 = acc[0], o1 = acc[1], o2 = acc[2], o3 = acc[3];
  out[e] = GateApply<T>(out_gate, gv, Vec<T>::Narrow(((o0 + o1) + (o2 + o3)) * inv_lds));
}

template <typename T, int D>
__global__ void __launch_bounds__(D) DecodeMergeKernel(T* __restrict__ out, float* __restrict__ lse, DecodeMergeArgs m,
                                                       uint32_t q_heads, const void* out_gate) {
  DecodeMergeBody<T, D>(out, lse, m, q_heads, out_gate, blockIdx.x);
}

// ---- Prefill kernel (bf16, head_dim 256, MFMA) -----------------------------------------------------------------------

constexpr int kPD = 256;                 // head_dim
constexpr int kKStride = kPD + 8;        // K tile row stride in LDS (elements): 528 bytes
constexpr int kVtStride = kPrefillTileK + 8;  // V^T tile row stride (elements): 144 bytes

__device__ __forceinline__ f32x16_t Mfma32(const u32x4_t& a, const u32x4_t& b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c, 0,
                                                 0, 0);
}

__global__ void __launch_bounds__(256, 1)
    PrefillKernel(const uint16_t* __restrict__ q, uint16_t* __restrict__ out, float* __restrict__ lse, KvView kv,
                  const int32_t* __restrict__ q_indptr, const PrefillWork* __restrict__ work, uint32_t q_heads,
                  uint32_t causal, float scale_log2, int32_t window, SoftCap cap) {
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[kPrefillTileK * kKStride];
  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[kPD * kVtStride];

  const PrefillWork wk = work[blockIdx.x];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int hl = lane >> 5;   // half of the wave
  const int col = lane & 31;  // MFMA N index: this lane's query within the tile
  const uint32_t kvh = static_cast<uint32_t>(wk.kv_head);
  const uint32_t head = kvh * kGroup + wave;
  const uint16_t* kbase = static_cast<const uint16_t*>(kv.k);
  const uint16_t* vbase = static_cast<const uint16_t*>(kv.v);

  int32_t p0 = 0;
  const uint32_t kv_len = SeqKvLen(kv, wk.seq, &p0);
  const int32_t qbeg = q_indptr[wk.seq];
  const int32_t n = q_indptr[wk.seq + 1] - qbeg;
  const int32_t q0 = wk.q0;
  const int32_t rows = wk.rows;
  // Key position of this lane's query, and of the tile's first / last query.
  const int32_t base_pos = static_cast<int32_t>(kv_len) - n + q0;
  const int32_t my_pos = base_pos + col;
  int32_t key_end = static_cast<int32_t>(kv_len);
  if (causal) key_end = min(key_end, base_pos + rows);  // last query sees keys <= base_pos + rows - 1
  if (key_end < 0) key_end = 0;

  // Q^T operand: lane holds q[query col][ks*16 + hl*8 .. +8] for ks = 0..15.
  u32x4_t qreg[16];
  {
    const bool ok = col < rows;
    const uint16_t* qrow = q + (static_cast<uint64_t>(qbeg + q0 + (ok ? col : 0)) * q_heads + head) * kPD + hl * 8;
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) {
      qreg[ks] = ok ? *reinterpret_cast<const u32x4_t*>(qrow + ks * 16) : u32x4_t{0, 0, 0, 0};
    }
  }

  f32x16_t o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[dt][v] = 0.0f;
  float m_run = -INFINITY;
  float l_run = 0.0f;

  // K/V of the next 64-key tile are fetched into registers while the current tile is computed (software pipeline).
  u32x4_t kpre[8];
  u32x4_t vpre[2][4];
  auto fetch = [&](int32_t kb) {
    const u32x4_t zero{0, 0, 0, 0};
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int vi = tid + 256 * it;
      bool ok;
      const uint64_t row = KeyRowSafe<kPD>(kv, p0, kb + (vi >> 5), key_end, kvh, &ok);
      const u32x4_t x = *reinterpret_cast<const u32x4_t*>(kbase + row + (vi & 31) * 8);
      kpre[it] = ok ? x : zero;
    }
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int vi = tid + 256 * it;  // 16 groups of 4 keys x 32 slices of 8 dims
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        bool ok;
        const uint64_t row = KeyRowSafe<kPD>(kv, p0, kb + (vi >> 5) * 4 + t, key_end, kvh, &ok);
        const u32x4_t x = *reinterpret_cast<const u32x4_t*>(vbase + row + (vi & 31) * 8);
        vpre[it][t] = ok ? x : zero;
      }
    }
  };
  // With a window the tile's first query (position base_pos) sees keys from base_pos - window on; keys before that
  // are never read.
  const int32_t key_beg = window < 0 ? 0 : min(max(0, base_pos - window), key_end);
  if (key_end > key_beg) fetch(key_beg);

  for (int32_t kb = key_beg; kb < key_end; kb += kPrefillTileK) {
    __syncthreads();  // every wavefront is done reading the previous tile
    // K row-major; V transposed: 4 keys x 8 dims become 8 rows (dims) of 4 keys.
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int vi = tid + 256 * it;
      *reinterpret_cast<u32x4_t*>(&k_lds[(vi >> 5) * kKStride + (vi & 31) * 8]) = kpre[it];
    }
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int vi = tid + 256 * it;
      const int kg = vi >> 5;
      const int c = vi & 31;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int w = e >> 1;
        uint32_t k01, k23;
        if ((e & 1) == 0) {
          k01 = (vpre[it][0][w] & 0xFFFFu) | (vpre[it][1][w] << 16);
          k23 = (vpre[it][2][w] & 0xFFFFu) | (vpre[it][3][w] << 16);
        } else {
          k01 = (vpre[it][0][w] >> 16) | (vpre[it][1][w] & 0xFFFF0000u);
          k23 = (vpre[it][2][w] >> 16) | (vpre[it][3][w] & 0xFFFF0000u);
        }
        *reinterpret_cast<u32x2_t*>(&vt_lds[(c * 8 + e) * kVtStride + kg * 4]) = u32x2_t{k01, k23};
      }
    }
    __syncthreads();
    if (kb + static_cast<int32_t>(kPrefillTileK) < key_end) fetch(kb + kPrefillTileK);

    // S^T = K Q^T for two 32-key halves: lane holds keys 8i + 4hl + jj of half kt for query col.
    f32x16_t s[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int v = 0; v < 16; ++v) s[kt][v] = 0.0f;
#pragma unroll
      for (int ks = 0; ks < 16; ++ks) {
        const u32x4_t a = *reinterpret_cast<const u32x4_t*>(&k_lds[(kt * 32 + col) * kKStride + ks * 16 + hl * 8]);
        s[kt] = Mfma32(a, qreg[ks], s[kt]);
      }
    }
    // Scale, mask, online softmax for this lane's query.
    const bool need_mask = (kb + static_cast<int32_t>(kPrefillTileK) > key_end) ||
                           (causal && kb + static_cast<int32_t>(kPrefillTileK) - 1 > base_pos) ||
                           (window >= 0 && kb < base_pos + rows - 1 - window);
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int32_t key = kb + kt * 32 + (v >> 2) * 8 + hl * 4 + (v & 3);
        float x = s[kt][v] * scale_log2;
        if (cap.capl != 0.0f) x = Capped(x, cap);
        if (need_mask && (key >= key_end || (causal && key > my_pos) || (window >= 0 && key < my_pos - window))) {
          x = -INFINITY;
        }
        s[kt][v] = x;
        mx = fmaxf(mx, x);
      }
    mx = MaxXor32(mx);
    // Lazy rescaling: the running max only moves when a score exceeds it by more than 2^8, so P stays below 256 (safe
    // in fp32 and bf16) and the O accumulators are rescaled on a handful of tiles instead of every tile.
    const bool grow = mx > m_run + 8.0f;
    if (__any(grow)) {
      const float m_new = grow ? mx : m_run;
      const float corr = m_run == -INFINITY ? 0.0f : exp2f(m_run - m_new);
      l_run *= corr;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[dt][v] *= corr;
      m_run = m_new;
    }
    const float m_use = m_run == -INFINITY ? 0.0f : m_run;  // a query with no visible key yet keeps p = 0
    float psum = 0.0f;
    u32x4_t pb[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int kt = c >> 1;
      const int i0 = (c & 1) * 2;
      float pf[8];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        pf[t] = exp2f(s[kt][i0 * 4 + t] - m_use);
        pf[4 + t] = exp2f(s[kt][(i0 + 1) * 4 + t] - m_use);
      }
#pragma unroll
      for (int t = 0; t < 8; ++t) psum += pf[t];
      pb[c] = u32x4_t{PackBf16(pf[0], pf[1]), PackBf16(pf[2], pf[3]), PackBf16(pf[4], pf[5]), PackBf16(pf[6], pf[7])};
    }
    l_run += psum;
    // O^T += V^T P^T: A = V^T rows (dims) with the keys in the order the P^T operand holds them.
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint16_t* vrow = &vt_lds[(dt * 32 + col) * kVtStride + c * 16 + hl * 4];
        const u32x2_t lo = *reinterpret_cast<const u32x2_t*>(vrow);
        const u32x2_t hi = *reinterpret_cast<const u32x2_t*>(vrow + 8);
        o[dt] = Mfma32(u32x4_t{lo[0], lo[1], hi[0], hi[1]}, pb[c], o[dt]);
      }
    }
  }

  // Normalise and write: lane holds dims dt*32 + 8i + 4hl + jj of query col.
  const float l_tot = SumXor32(l_run);
  if (col < rows) {
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    const uint64_t orow = (static_cast<uint64_t>(qbeg + q0 + col) * q_heads + head) * kPD;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = dt * 32 + i * 8 + hl * 4;
        const u32x2_t w{PackBf16(o[dt][i * 4] * inv, o[dt][i * 4 + 1] * inv),
                        PackBf16(o[dt][i * 4 + 2] * inv, o[dt][i * 4 + 3] * inv)};
        *reinterpret_cast<u32x2_t*>(out + orow + d) = GateOut2(kv.out_gate, orow + d, w);
      }
    if (lse != nullptr && hl == 0) {
      lse[static_cast<uint64_t>(qbeg + q0 + col) * q_heads + head] = l_tot > 0.0f ? m_run + log2f(l_tot) : -INFINITY;
    }
  }
}

// ---- Prefill kernel for page sizes that are multiples of 16 (bf16, head_dim 64/128/256, MFMA, DMA-fed) --------------
//
// One workgroup = 64 query tokens x the 4 query heads of one KV head, 8 wavefronts (two per SIMD, so one wavefront's
// softmax runs under the other's MFMAs): wavefront w is query head 4 kvh + (w & 3) for tokens 32 (w >> 2) .. +31.
// Per 64-key tile each wavefront copies 8 K rows and a quarter of the V tile (16-aligned groups of rows never straddle
// a page when the page size is a multiple of 16) from the paged cache straight into LDS with global_load_lds,
// double-buffered, so the copy of tile t + 1 runs under the products of tile t. The tile is consumed in two 32-key
// halves:
//   S^T = K Q^T  (v_mfma_f32_32x32x16_bf16; K rows from LDS as the A operand, Q^T held in registers as B),
//   online softmax per query (lane pair l, l ^ 32 holds one query's 32 scores; lazy rescaling: the running max only
//   moves when a score exceeds it by more than 2^8, so P stays below 256),
//   O^T += V^T P^T (V^T operands read from the V tile with ds_read_b64_tr_b16, P^T from registers).
// ds_read_b64_tr_b16 works within groups of 16 lanes: output lane 4a + b, element e, is element b of the 8 bytes that
// lane 4e + a addressed. So when lane 4e + a of a group addresses keys k0 + e, dims d0 + 4a .. +3, output lane j of the
// group receives V[k0 + e][d0 + j], e = 0..3: a V^T operand row.
// K rows are 512 bytes in LDS with 16-byte pieces at swizzled positions: piece p of row r at p ^ (r & 15) (the A-operand
// reads of 16 consecutive rows hit 16 distinct bank groups). The V tile is stored in the order the transposed reads
// consume it: 1 KB block (c16, dt) holds keys 16 c16 .. +15 x dims 32 dt .. +31, each read instruction takes one
// contiguous 512-byte half of a block (conflict-free, and every read is one base register plus an immediate). Each
// copy instruction then fetches 16 rows x 64 bytes; storing K the same way (32 rows x 32 bytes per copy) was measured
// 8% slower overall, the copy's wider spread of cache lines costing more than the cheaper reads gain.

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) unsigned char lds_byte_t;

__device__ __forceinline__ uint32_t LdsAddr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const lds_byte_t*)p));
}

// global -> LDS copy of 16 bytes per lane (lane l lands at lds + 16 l; lds wave-uniform), from inline assembly so that
// the compiler does not make every later LDS access wait on it; the kernel waits for it itself. M0 is restored.
__device__ __forceinline__ void Dma16(const void* g, uint32_t lds) {
  uint32_t save;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
               : "=&s"(save) : "v"(g), "s"(lds));
}

// The same with a wave-uniform 64-bit base in SGPRs and a 32-bit per-lane byte offset.
__device__ __forceinline__ void Dma16(const void* sbase, uint32_t voff, uint32_t lds) {
  uint32_t save;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\tglobal_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
               : "=&s"(save) : "v"(voff), "s"(sbase), "s"(lds));
}

// Both copies again with an immediate byte offset kOff (below 4096) on the global address. The instruction adds its
// offset to the LDS address as well, so M0 is set to lds - kOff and the 16 bytes of lane l still land at lds + 16 l.
template <int kOff>
__device__ __forceinline__ void Dma16At(const void* sbase, uint32_t voff, uint32_t lds) {
  uint32_t save;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\tglobal_load_lds_dwordx4 %1, %2 offset:%4\n\ts_mov_b32 m0, %0"
               : "=&s"(save) : "v"(voff), "s"(sbase), "s"(lds - kOff), "i"(kOff));
}

template <int kN, typename F>
__device__ __forceinline__ void StaticFor(F&& f) {
  if constexpr (kN > 0) {
    StaticFor<kN - 1>(f);
    f(std::integral_constant<int, kN - 1>{});
  }
}

__device__ __forceinline__ void WaitVmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0) only

__device__ __forceinline__ u32x2_t LdsTr16(const unsigned char* base, uint32_t off) {
  auto* ptr = reinterpret_cast<__attribute__((address_space(3))) i16x4_t*>(
      const_cast<lds_byte_t*>((const lds_byte_t*)base + off));
  return __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(ptr));
}


// Head dims 256, 128 and 64: a row is 2 D bytes = D / 8 16-byte pieces (32, 16 or 8). K pieces are swizzled by the
// row index modulo min(16, D / 8), which keeps every swizzled piece inside its row and any 8 consecutive rows (the
// lanes one LDS read cycle serves) on distinct 16-byte bank groups; the V offsets (at most 12 pieces) stay inside a row.
// kCap: the call caps its logits; `cap` is then the cap in the kernel's unscaled score units (the log2-unit cap divided
// by scale_log2, its slope multiplied by it), so that a capped score stays unscaled like an uncapped one. A separate
// instantiation keeps the cap's registers out of the uncapped kernel, which otherwise spills at head dim 256.
template <int D>
constexpr int kPfTileBytes = kPrefillTileK * 2 * D;  // one 64-key K or V tile in LDS

// The tile kernel's work for item `item`; `tiles` is the caller's LDS, [2 buffers][K, V][kPfTileBytes<D>].
template <int D, bool kCap>
__device__ __forceinline__ void PrefillTileBody(const uint16_t* __restrict__ q, uint16_t* __restrict__ out,
                                                float* __restrict__ lse, KvView kv,
                                                const int32_t* __restrict__ kv_indices,
                                                const int32_t* __restrict__ q_indptr,
                                                const PrefillWork* __restrict__ work, uint16_t* __restrict__ part_o,
                                                float* __restrict__ part_ml, uint32_t q_heads, uint32_t causal,
                                                uint32_t ps_shift, float scale_log2, int32_t window, SoftCap cap,
                                                uint32_t item, unsigned char (*tiles)[2][kPfTileBytes<D>]) {
  static_assert(D == 64 || D == 128 || D == 256, "the tile kernel is built for head dims 64, 128 and 256");
  constexpr int kRowB = 2 * D;                  // bytes of one K or V row in LDS
  constexpr int kPieces = D / 8;                // 16-byte pieces per row
  constexpr int kRowsPerDma = 1024 / kRowB;     // rows one 64-lane global_load_lds_dwordx4 fills
  constexpr int kKs = D / 16;                   // K = 16 steps of S^T = K Q^T
  constexpr int kDt = D / 32;                   // 32-dim blocks of O^T
  constexpr int kNv = kDt / 2;                  // V blocks each wavefront copies per tile (4 kDt blocks / 8)
  constexpr int kSw = (kPieces < 16 ? kPieces : 16) - 1;  // K swizzle mask

  const PrefillWork wk = work[item];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hq = w & 3;       // query head within the KV head's group
  const int qt = w >> 2;      // 32-token half of the item
  const int hl = lane >> 5;   // half of the wave: MFMA k-slot group
  const int col = lane & 31;  // MFMA N index: this lane's query within the wavefront's 32
  const uint32_t kvh = static_cast<uint32_t>(wk.kv_head);
  const uint32_t head = kvh * kGroup + hq;
  const uint16_t* kbase = static_cast<const uint16_t*>(kv.k);
  const uint16_t* vbase = static_cast<const uint16_t*>(kv.v);
  const uint32_t ps = kv.page_size;  // a power of two, 1 << ps_shift

  int32_t p0 = 0;
  const uint32_t kv_len = SeqKvLen(kv, wk.seq, &p0);
  const int32_t qbeg = q_indptr[wk.seq];
  const int32_t n = q_indptr[wk.seq + 1] - qbeg;
  const int32_t r = 32 * qt + col;  // this lane's query within the item
  const bool row_ok = r < wk.rows;
  const int32_t last_pos = static_cast<int32_t>(kv_len) - n + wk.q0 + 32 * qt + 31;  // the wavefront's last query
  // The item's key range by the device's lengths: keys up to its last query (causal) or all keys, from its first
  // query's window start rounded down to 16. The plan's cuts between pieces stay; the outer bounds follow the device.
  const int32_t dev_first = static_cast<int32_t>(kv_len) - n + wk.q0;  // the item's first query position
  const int32_t dev_end = max(0, causal ? min(static_cast<int32_t>(kv_len), dev_first + wk.rows)
                                        : static_cast<int32_t>(kv_len));
  const int32_t dev_beg = window < 0 ? 0 : (max(0, dev_first - window) & ~15);
  const int32_t kbeg = (wk.ends & kPieceFirst) ? dev_beg : wk.kbeg;
  const int32_t kend = (wk.ends & kPieceLast) ? dev_end : min(wk.kend, dev_end);
  const int ntiles = kend > kbeg ? (kend - kbeg + 63) / 64 : 0;

  // Q^T operands: qreg[ks] = q[query r][dims 16 ks + 8 hl .. +8].
  u32x4_t qreg[kKs];
  {
    const uint16_t* qrow = q + (static_cast<uint64_t>(qbeg + wk.q0 + (row_ok ? r : 0)) * q_heads + head) * D + hl * 8;
#pragma unroll
    for (int ks = 0; ks < kKs; ++ks) {
      const u32x4_t x = *reinterpret_cast<const u32x4_t*>(qrow + ks * 16);
      qreg[ks] = row_ok ? x : u32x4_t{0, 0, 0, 0};
    }
  }

  // Page ids of the four 16-row groups of tile t (rows clamped into the item's keys); loaded one tile before the
  // copy that needs them, so the scalar loads never stall the loop.
  // With 16-token pages, a tile wholly inside the key range takes its four ids as one 16-byte scalar load of
  // consecutive page-table entries (all of them exist: the sequence has a page for every key below kend).
  auto load_ids = [&](int t, int32_t (&ids)[4]) {
    const int32_t kb = kbeg + 64 * t;
    if (ps_shift == 4 && kb + 64 <= kend) {
      int4 v;
      __builtin_memcpy(&v, kv_indices + p0 + (kb >> 4), sizeof(v));
      ids[0] = v.x;
      ids[1] = v.y;
      ids[2] = v.z;
      ids[3] = v.w;
    } else {
#pragma unroll
      for (int g = 0; g < 4; ++g) ids[g] = kv_indices[p0 + (min(kb + 16 * g, kend - 1) >> ps_shift)];
    }
  };
  // id in [0, pool_pages) as one unsigned 32-bit compare (pool page counts above 2^31 - 1 are clamped: ids are int32).
  const uint32_t pool32 = static_cast<uint32_t>(min(kv.pool_pages, static_cast<uint64_t>(0x7FFFFFFF)));
  auto good_page = [&](int32_t id) { return static_cast<uint32_t>(id) < pool32; };
  // Element offsets inside a page: a row at in-page position `within` starts at row_mul * within + row_add.
  const uint32_t row_mul = kv.hnd ? D : kv.kv_heads * D;
  const uint32_t kvr = kvh >> kv.head_shift;  // the real KV head the item's query heads read
  const uint32_t row_add = kv.hnd ? kvr * ps * D : kvr * D;
  const uint64_t page_elems = static_cast<uint64_t>(ps) * kv.kv_heads * D;
  // This wavefront's share of the copy of tile t: K rows 8w .. 8w + 7 (kRowsPerDma rows per instruction) and kNv
  // blocks of V.
  auto issue = [&](int t, int buf, const int32_t (&ids)[4], int ln) {
    const int32_t kb = kbeg + 64 * t;
    const int32_t pos0 = kb + 8 * w;  // this wavefront's first row; all 8 lie in one page
    const int32_t id = ids[w >> 1];
    const uint64_t pg = good_page(id) ? static_cast<uint64_t>(id) : 0;  // a bad page's rows are masked, not read
    const int32_t page_first = min(pos0, kend - 1) & ~((1 << ps_shift) - 1);
    const uint16_t* kpage = kbase + pg * page_elems + row_add;
    const uint32_t kdst = LdsAddr(tiles[buf][0]) + 8 * w * kRowB;
    const int c = ln % kPieces, hh = ln / kPieces;
#pragma unroll
    for (int i = 0; i < 8 / kRowsPerDma; ++i) {
      const int rr = kRowsPerDma * i + hh;  // row 8w + rr of the tile
      const uint32_t within = static_cast<uint32_t>(min(pos0 + rr, kend - 1) - page_first);
      const uint32_t off = 2 * row_mul * within;
      const uint32_t kp = 16 * static_cast<uint32_t>(c ^ ((8 * w + rr) & kSw));
      Dma16(kpage, off + kp, kdst + i * 1024);
    }
    {  // V blocks (c16, dt0 + i): lane ln fetches key 16 c16 + 8 hi + 4 ((mm >> 4) & 1) + ((mm & 7) >> 1),
       // dims 32 (dt0 + i) + 16 ((mm >> 3) & 1) + 8 (mm & 1); the block's 16 keys lie in one page
      const int mm = ln & 31, hi = ln >> 5;
      const int c16 = w >> 1, dt0 = (w & 1) * kNv;
      const int32_t vid = ids[c16];
      const uint16_t* vpage = vbase + (good_page(vid) ? static_cast<uint64_t>(vid) : 0) * page_elems + row_add;
      const int key = 16 * c16 + 8 * hi + 4 * ((mm >> 4) & 1) + ((mm & 7) >> 1);
      const uint32_t within = static_cast<uint32_t>(min(kb + key, kend - 1)) & ((1u << ps_shift) - 1);
      const uint32_t voff = 2 * (row_mul * within + 32 * dt0 + 16 * ((mm >> 3) & 1) + 8 * (mm & 1));
      const uint32_t dst = LdsAddr(tiles[buf][1]) + 1024 * (c16 * kDt + dt0);
      StaticFor<kNv>([&](auto i) { Dma16At<64 * i.value>(vpage, voff, dst + 1024 * i.value); });
    }
  };

  f32x16_t o[kDt];
#pragma unroll
  for (int dt = 0; dt < kDt; ++dt)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[dt][v] = 0.0f;
  float m_run = -INFINITY;
  float l_run = 0.0f;

  int32_t ids_cur[4] = {0, 0, 0, 0}, ids_nxt[4] = {0, 0, 0, 0};
  if (ntiles > 0) {
    load_ids(0, ids_cur);
    issue(0, 0, ids_cur, lane);
    load_ids(min(1, ntiles - 1), ids_nxt);
  }
  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    WaitVmem();       // this wavefront's copies of tile t have landed
    __syncthreads();  // ... and everyone's; everyone is also done reading the other buffer
    // Every lane-dependent value the loop needs is re-derived here from the thread index, so that only the index
    // stays live across the loop (the register budget at two wavefronts per SIMD holds nothing more).
    int tx = static_cast<int>(threadIdx.x);
    asm volatile("" : "+v"(tx));
    const int ln = tx & 63, lc = ln & 31, lh = ln >> 5;
    if (t + 1 < ntiles) issue(t + 1, buf ^ 1, ids_nxt, ln);
    uint32_t bad = 0;  // 16-key groups of this tile whose page id lies outside the pool
#pragma unroll
    for (int g = 0; g < 4; ++g) bad |= good_page(ids_cur[g]) ? 0u : (1u << g);
#pragma unroll
    for (int g = 0; g < 4; ++g) ids_cur[g] = ids_nxt[g];
    load_ids(min(t + 2, ntiles - 1), ids_nxt);
    const int32_t kb = kbeg + 64 * t;
    // K operand: row 32 half + lc, piece 2 ks + lh at position (2 ks + lh) ^ (lc & kSw) (32 half keeps row & kSw =
    // lc & kSw); in bytes 16 ((2 ks + lh) ^ (lc & kSw)) = 32 ks ^ 16 (lh ^ (lc & kSw)).
    const int krow = lc * kRowB, kx = 16 * (lh ^ (lc & kSw));
    // V^T operands, read transposed: in lane group g = ln / 16, lane j = ln % 16 addresses key +(j / 4) at dims
    // +4 (j % 4), keys based at 16 c16 + 4 (g >> 1) (+8 for the operand's second half), dims at 32 dt + 16 (g & 1);
    // block (c16, dt) of the V tile holds exactly those 8 bytes at 8 ln (and the second half's at 512 + 8 ln).
    const int32_t qpos = static_cast<int32_t>(kv_len) - n + wk.q0 + 32 * qt + lc;  // this lane's query position
    // Every term is wave-uniform; readfirstlane says so, so that the masking below is skipped by a scalar branch
    // instead of running under an empty exec mask on every tile.
    const bool need_mask = __builtin_amdgcn_readfirstlane(
        static_cast<int>((kb + 64 > kend) | (causal && kb + 63 > last_pos - 31) | (bad != 0) |
                         (window >= 0 && kb < last_pos - window))) != 0;
    const unsigned char* ktile = tiles[buf][0];
    const unsigned char* vtile = tiles[buf][1];
    const unsigned char* vl = vtile + 8 * ln;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      f32x16_t sc;
#pragma unroll
      for (int v = 0; v < 16; ++v) sc[v] = 0.0f;
      const unsigned char* krow_p = ktile + 32 * half * kRowB + krow;
      constexpr int kRing = 2;  // K operands in flight ahead of the multiply that uses them
      u32x4_t ka[kRing];
#pragma unroll
      for (int j = 0; j < kRing; ++j) ka[j] = *reinterpret_cast<const u32x4_t*>(krow_p + ((32 * j) ^ kx));
#pragma unroll
      for (int ks = 0; ks < kKs; ++ks) {
        const u32x4_t a = ka[ks % kRing];
        if (ks + kRing < kKs) ka[ks % kRing] = *reinterpret_cast<const u32x4_t*>(krow_p + ((32 * (ks + kRing)) ^ kx));
        sc = Mfma32(a, qreg[ks], sc);
      }
      // Keep kRing operand reads in flight (left alone, the compiler waits out every read before its multiply at this
      // register budget): the reads of the first kRing steps, then one multiply and one read in turn.
      __builtin_amdgcn_sched_group_barrier(0x100, kRing, 0);
#pragma unroll
      for (int ks = 0; ks < kKs - kRing; ++ks) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, kRing, 0);
      if constexpr (kCap) {
#pragma unroll
        for (int v = 0; v < 16; ++v) sc[v] = Capped(sc[v], cap);
      }
      if (need_mask) {  // one uniform branch around branch-free selects
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int kk = 32 * half + (v >> 2) * 8 + lh * 4 + (v & 3);  // key within the tile
          const int32_t key = kb + kk;
          // Bitwise ors: no short-circuit branches (each would be an exec-mask change per score).
          const bool off = (key >= kend) | ((causal != 0) & (key > qpos)) | (((bad >> (kk >> 4)) & 1u) != 0) |
                           ((window >= 0) & (key < qpos - window));
          sc[v] = off ? -INFINITY : sc[v];
        }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, sc[v]);
      mx = MaxXor32(mx);
      mx *= scale_log2;  // scores stay unscaled until the exponent: the scale is positive, so this is the scaled max
      const bool grow = mx > m_run + 8.0f;
      if (__any(grow)) {
        const float m_new = grow ? mx : m_run;
        const float corr = m_run == -INFINITY ? 0.0f : exp2f(m_run - m_new);
        l_run *= corr;
#pragma unroll
        for (int dt = 0; dt < kDt; ++dt)
#pragma unroll
          for (int v = 0; v < 16; ++v) o[dt][v] *= corr;
        m_run = m_new;
      }
      const float m_use = m_run == -INFINITY ? 0.0f : m_run;
      float psum = 0.0f;
      u32x4_t pb[2];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        float pf[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pf[e] = __builtin_amdgcn_exp2f(fmaf(sc[(2 * c) * 4 + e], scale_log2, -m_use));
          pf[4 + e] = __builtin_amdgcn_exp2f(fmaf(sc[(2 * c + 1) * 4 + e], scale_log2, -m_use));
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) psum += pf[e];
        pb[c] = u32x4_t{PackRne(pf[0], pf[1]), PackRne(pf[2], pf[3]), PackRne(pf[4], pf[5]), PackRne(pf[6], pf[7])};
      }
      l_run += psum;
      // O^T += V^T P^T over this half's two 16-key steps.
      // V^T operands of the 16 multiplies (c, dt) in order, read kVRing ahead of use.
      constexpr int kVRing = 2;
      auto vread = [&](int j) {
        const int c = j / kDt, dt = j % kDt;
        const uint32_t off = 1024 * ((2 * half + c) * kDt + dt);
        const u32x2_t lo = LdsTr16(vl, off);
        const u32x2_t hi = LdsTr16(vl, off + 512);
        return u32x4_t{lo[0], lo[1], hi[0], hi[1]};
      };
      u32x4_t va[kVRing];
#pragma unroll
      for (int j = 0; j < kVRing; ++j) va[j] = vread(j);
#pragma unroll
      for (int j = 0; j < 2 * kDt; ++j) {
        const u32x4_t av = va[j % kVRing];
        if (j + kVRing < 2 * kDt) va[j % kVRing] = vread(j + kVRing);
        o[j % kDt] = Mfma32(av, pb[j / kDt], o[j % kDt]);
      }
    }
  }

  // Lane holds dims 32 dt + 8 i + 4 hl + jj of query r.
  const float l_tot = SumXor32(l_run);
  if (!row_ok) return;
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (wk.slot >= 0) {  // a piece of a split item: its normalised output in bf16 and its (max, sum)
    const uint64_t prow = static_cast<uint64_t>(wk.slot) * kPfRows + static_cast<uint64_t>(r) * kGroup + hq;
    uint16_t* po = part_o + prow * D;
#pragma unroll
    for (int dt = 0; dt < kDt; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = dt * 32 + i * 8 + hl * 4;
        const u32x2_t v{PackRne(o[dt][i * 4] * inv, o[dt][i * 4 + 1] * inv),
                        PackRne(o[dt][i * 4 + 2] * inv, o[dt][i * 4 + 3] * inv)};
        *reinterpret_cast<u32x2_t*>(po + d) = v;
      }
    if (hl == 0) {
      part_ml[2 * prow] = m_run;
      part_ml[2 * prow + 1] = l_tot;
    }
    return;
  }
  const uint64_t orow = (static_cast<uint64_t>(qbeg + wk.q0 + r) * q_heads + head) * D;
#pragma unroll
  for (int dt = 0; dt < kDt; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = dt * 32 + i * 8 + hl * 4;
      const u32x2_t v{PackRne(o[dt][i * 4] * inv, o[dt][i * 4 + 1] * inv),
                      PackRne(o[dt][i * 4 + 2] * inv, o[dt][i * 4 + 3] * inv)};
      *reinterpret_cast<u32x2_t*>(out + orow + d) = GateOut2(kv.out_gate, orow + d, v);
    }
  if (lse != nullptr && hl == 0) {
    lse[static_cast<uint64_t>(qbeg + wk.q0 + r) * q_heads + head] = l_tot > 0.0f ? m_run + log2f(l_tot) : -INFINITY;
  }
}


template <int D, bool kCap>
__global__ void __launch_bounds__(512, 1)
    PrefillTileKernel(const uint16_t* __restrict__ q, uint16_t* __restrict__ out, float* __restrict__ lse, KvView kv,
                      const int32_t* __restrict__ kv_indices, const int32_t* __restrict__ q_indptr,
                      const PrefillWork* __restrict__ work, uint16_t* __restrict__ part_o, float* __restrict__ part_ml,
                      uint32_t q_heads, uint32_t causal, uint32_t ps_shift, float scale_log2, int32_t window,
                      SoftCap cap) {
  __shared__ __attribute__((aligned(16))) unsigned char tiles[2][2][kPfTileBytes<D>];  // [buffer][K, V]
  PrefillTileBody<D, kCap>(q, out, lse, kv, kv_indices, q_indptr, work, part_o, part_ml, q_heads, causal, ps_shift,
                           scale_log2, window, cap, blockIdx.x, tiles);
}

// A mixed step's attention in one launch: workgroups [0, items) run the tile pieces, the rest the decode ranges with 8
// wavefronts each (one range of one KV-head block per CU, 8 / heads_per_wg wavefronts per head). Tile workgroups come
// first in launch order, so they take their CUs before the decode ranges fill the others. Both kinds use the one LDS
// buffer in their own layout (a decode workgroup needs far less than a tile one, and neither shares its CU).
template <int D>
constexpr int kMixedDecodeLds = 4 * (kMixedDecodeWaves * 64 + 2 * kMixedDecodeWaves * kGroup +
                                     kMixedDecodeWaves * kGroup * D);

template <int D, bool kCap>
__global__ void __launch_bounds__(512, 1)
    MixedAttentionKernel(const uint16_t* __restrict__ q, uint16_t* __restrict__ out, float* __restrict__ lse,
                         KvView kv, const int32_t* __restrict__ kv_indices, const int32_t* __restrict__ q_indptr,
                         const PrefillWork* __restrict__ work, uint16_t* __restrict__ part_o,
                         float* __restrict__ part_ml, uint32_t q_heads, uint32_t causal, uint32_t ps_shift,
                         float scale_log2, int32_t window, SoftCap raw_cap, uint32_t items,
                         const DecodeWork* __restrict__ dec_work, const int32_t* __restrict__ dec_range_ptr,
                         float* __restrict__ dec_part_o, float* __restrict__ dec_part_ml, uint32_t heads_per_wg,
                         SoftCap cap) {
  constexpr int kTileLds = 2 * 2 * kPfTileBytes<D>;
  constexpr int kLds = kTileLds > kMixedDecodeLds<D> ? kTileLds : kMixedDecodeLds<D>;
  __shared__ __attribute__((aligned(16))) unsigned char lds[kLds];
  if (blockIdx.x < items) {
    PrefillTileBody<D, kCap>(q, out, lse, kv, kv_indices, q_indptr, work, part_o, part_ml, q_heads, causal, ps_shift,
                             scale_log2, window, raw_cap, blockIdx.x,
                             reinterpret_cast<unsigned char (*)[2][kPfTileBytes<D>]>(lds));
    return;
  }
  constexpr int W = kMixedDecodeWaves;
  float* x_lds = reinterpret_cast<float*>(lds);
  float* m_lds = x_lds + W * 64;
  float* l_lds = m_lds + W * kGroup;
  float* o_lds = l_lds + W * kGroup;
  DecodeBody<uint16_t, D, true, W>(q, out, lse, kv, kv_indices, dec_work, dec_range_ptr, dec_part_o, dec_part_ml,
                                   q_indptr, q_heads, heads_per_wg, scale_log2, window, causal, cap,
                                   blockIdx.x - items, x_lds, m_lds, l_lds, o_lds);
}

// Combines the pieces of a split prefill item: block (merge, group of kRows tokens) of kGroup * D / 4 threads; thread t
// handles query head t / (D / 4), dims 4 (t % (D / 4)) .. +3 of each of the group's tokens. Pieces are combined in
// key order (deterministic). Merges of two pieces (the plan puts them first) run 8 tokens per block with every load
// issued before any is combined; the others one token per block.
constexpr int kPfMergeRows = 8;

template <int D>
__device__ __forceinline__ void MergeWrite(uint16_t* __restrict__ out, float* __restrict__ lse, const void* gate,
                                           u32x2_t g, uint64_t token, uint32_t q_heads, uint32_t head, int d,
                                           float4 acc, float l, float mx) {
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  const u32x2_t v{PackBf16(acc.x * inv, acc.y * inv), PackBf16(acc.z * inv, acc.w * inv)};
  const uint64_t e = (token * q_heads + head) * D + d;
  *reinterpret_cast<u32x2_t*>(out + e) = GateApply2(gate, g, v);
  if (lse != nullptr && d == 0) lse[token * q_heads + head] = l > 0.0f ? mx + log2f(l) : -INFINITY;
}

// acc += o * f for one piece's bf16 output slice (already divided by the piece's own sum).
__device__ __forceinline__ void MergeAdd(float4& acc, u32x2_t raw, float f) {
  acc.x = fmaf(__uint_as_float(raw[0] << 16), f, acc.x);
  acc.y = fmaf(__uint_as_float(raw[0] & 0xFFFF0000u), f, acc.y);
  acc.z = fmaf(__uint_as_float(raw[1] << 16), f, acc.z);
  acc.w = fmaf(__uint_as_float(raw[1] & 0xFFFF0000u), f, acc.w);
}

template <int D, int kRows>
__device__ __forceinline__ void PrefillMergeRows(uint16_t* __restrict__ out, float* __restrict__ lse,
                                                 const PrefillMerge& mg, int r0, const uint16_t* __restrict__ part_o,
                                                 const float* __restrict__ part_ml,
                                                 const int32_t* __restrict__ q_indptr, uint32_t q_heads,
                                                 const void* gate) {
  if (r0 >= mg.rows) return;
  const int hq = threadIdx.x / (D / 4);
  const int d = 4 * (threadIdx.x % (D / 4));
  const uint32_t head = mg.kv_head * kGroup + hq;
  const uint64_t tok0 = static_cast<uint64_t>(q_indptr[mg.seq] + mg.q0);
  // Partial row of piece i for token row r: (first + i) * kPfRows + r * kGroup + hq.
  auto prow = [&](int i, int r) {
    return (static_cast<uint64_t>(mg.first) + i) * kPfRows + static_cast<uint64_t>(r) * kGroup + hq;
  };
  if constexpr (kRows > 1) {  // merges of exactly two pieces
    float2 ml[kRows][2];
    u32x2_t o[kRows][2], gw[kRows];
#pragma unroll
    for (int j = 0; j < kRows; ++j) {
      const int r = min(r0 + j, mg.rows - 1);  // rows past the item's end re-read its last row and are not written
      gw[j] = GateFetch2(gate, ((tok0 + r) * q_heads + head) * D + d);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        ml[j][i] = *reinterpret_cast<const float2*>(part_ml + 2 * prow(i, r));
        o[j][i] = *reinterpret_cast<const u32x2_t*>(part_o + prow(i, r) * D + d);
      }
    }
#pragma unroll
    for (int j = 0; j < kRows; ++j) {
      if (r0 + j >= mg.rows) break;
      const float mx = fmaxf(ml[j][0].x, ml[j][1].x);
      float l = 0.0f;
      float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (mx != -INFINITY) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          // The piece's weight is its sum rescaled to the common max (mx is finite here, so a piece without keys,
          // max -inf, gets exp2(-inf) = 0).
          const float f = ml[j][i].y * exp2f(ml[j][i].x - mx);
          l += f;
          MergeAdd(acc, o[j][i], f);
        }
      }
      MergeWrite<D>(out, lse, gate, gw[j], tok0 + r0 + j, q_heads, head, d, acc, l, mx);
    }
  } else {  // any count, one token row per block; the piece loops are unrolled so several pieces' loads are in flight
    const u32x2_t gw = GateFetch2(gate, ((tok0 + r0) * q_heads + head) * D + d);
    float mx = -INFINITY;
#pragma unroll 8
    for (int i = 0; i < mg.count; ++i) mx = fmaxf(mx, part_ml[2 * prow(i, r0)]);
    float l = 0.0f;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (mx != -INFINITY) {
#pragma unroll 4
      for (int i = 0; i < mg.count; ++i) {
        const float2 m = *reinterpret_cast<const float2*>(part_ml + 2 * prow(i, r0));
        const float f = m.y * exp2f(m.x - mx);
        l += f;
        MergeAdd(acc, *reinterpret_cast<const u32x2_t*>(part_o + prow(i, r0) * D + d), f);
      }
    }
    MergeWrite<D>(out, lse, gate, gw, tok0 + r0, q_heads, head, d, acc, l, mx);
  }
}

// One launch for both forms: the first `two` merges (exactly two pieces) as blocks of kPfMergeRows token rows, the
// rest one token row per block (two merge launches one after the other cost a second launch's latency).
struct PrefillMergeArgs {
  const PrefillMerge* merges;
  const uint16_t* part_o;
  const float* part_ml;
  const int32_t* q_indptr;
  uint32_t two;     // merges of exactly two pieces, listed first
  uint32_t blocks;  // blocks of the launch's prefill share
};

template <int D>
__device__ __forceinline__ void PrefillMergeBody(uint16_t* __restrict__ out, float* __restrict__ lse,
                                                 const PrefillMergeArgs& m, uint32_t q_heads, const void* gate,
                                                 uint32_t b) {
  constexpr uint32_t kTwoBlocks = kPfTokens / kPfMergeRows;  // blocks per two-piece merge
  const PrefillMerge* __restrict__ merges = m.merges;
  const uint16_t* __restrict__ part_o = m.part_o;
  const float* __restrict__ part_ml = m.part_ml;
  const int32_t* __restrict__ q_indptr = m.q_indptr;
  const uint32_t two = m.two;
  if (b < two * kTwoBlocks) {
    PrefillMergeRows<D, kPfMergeRows>(out, lse, merges[b / kTwoBlocks], static_cast<int>(b % kTwoBlocks) * kPfMergeRows,
                                      part_o, part_ml, q_indptr, q_heads, gate);
  } else {
    const uint32_t k = b - two * kTwoBlocks;
    PrefillMergeRows<D, 1>(out, lse, merges[two + k / kPfTokens], static_cast<int>(k % kPfTokens), part_o, part_ml,
                           q_indptr, q_heads, gate);
  }
}

template <int D>
__global__ void __launch_bounds__(256) PrefillMergeKernel(uint16_t* __restrict__ out, float* __restrict__ lse,
                                                          PrefillMergeArgs m, uint32_t q_heads, const void* gate) {
  PrefillMergeBody<D>(out, lse, m, q_heads, gate, blockIdx.x);
}

// A mixed step's two merges in one launch (both take D threads per block): the tile pieces' merge blocks first, then
// the decode ranges'. One launch instead of two saves the second's latency.
template <int D>
__global__ void __launch_bounds__(D) MixedMergeKernel(uint16_t* __restrict__ out, float* __restrict__ lse,
                                                      PrefillMergeArgs pm, DecodeMergeArgs dm, uint32_t q_heads,
                                                      const void* gate) {
  static_assert(kGroup * D / 4 == D, "a prefill merge block has D threads");
  if (blockIdx.x < pm.blocks) {
    PrefillMergeBody<D>(out, lse, pm, q_heads, gate, blockIdx.x);
  } else {
    DecodeMergeBody<uint16_t, D>(out, lse, dm, q_heads, gate, blockIdx.x - pm.blocks);
  }
}

// The decode pieces' partials: fp32 rows (dec_splits x q_heads x D), then their (max, sum) pairs.
DecodeMergeArgs DecodeMergeArgsOf(const RoostPagedAttentionParams& p, const PlanRecord& rec, unsigned char* dev,
                                  uint32_t d) {
  DecodeMergeArgs m{};
  m.merges = reinterpret_cast<const DecodeMerge*>(dev + rec.dec_merge_offset);
  m.part_o = reinterpret_cast<const float*>(dev + rec.dec_float_offset);
  m.part_ml = m.part_o + rec.dec_splits * p.q_heads * d;
  m.q_rows = p.mode == ROOST_ATTENTION_PREFILL ? static_cast<const int32_t*>(p.q_indptr.address) : nullptr;
  return m;
}

template <typename T, int D>
RoostStatus LaunchDecodeMerge(const RoostPagedAttentionParams& p, const PlanRecord& rec, unsigned char* dev,
                              const KvView& kv, hipStream_t stream) {
  if (rec.dec_merges == 0) return ROOST_STATUS_OK;
  hipLaunchKernelGGL((DecodeMergeKernel<T, D>), dim3(static_cast<uint32_t>(rec.dec_merges * p.q_heads)), dim3(D), 0,
                     stream, static_cast<T*>(p.output.address), static_cast<float*>(p.lse.address),
                     DecodeMergeArgsOf(p, rec, dev, D), p.q_heads, kv.out_gate);
  return roost::HipStatus(hipGetLastError(), "paged_attention", "decode merge launch");
}

template <typename T, int D>
RoostStatus LaunchDecode(const RoostPagedAttentionParams& p, const PlanRecord& rec, unsigned char* dev, const KvView& kv,
                         float scale_log2, hipStream_t stream) {
  if (rec.dec_ranges == 0) return ROOST_STATUS_OK;
  const auto* items = reinterpret_cast<const DecodeWork*>(dev + rec.dec_item_offset);
  const auto* range_ptr = reinterpret_cast<const int32_t*>(dev + rec.dec_range_offset);
  auto* part_o = reinterpret_cast<float*>(dev + rec.dec_float_offset);
  auto* part_ml = part_o + rec.dec_splits * p.q_heads * D;
  // In a prefill call the decode pieces are its single-token sequences, whose query rows are q_indptr[seq].
  const auto* q_rows =
      p.mode == ROOST_ATTENTION_PREFILL ? static_cast<const int32_t*>(p.q_indptr.address) : nullptr;
  auto* out = static_cast<T*>(p.output.address);
  auto* lse = static_cast<float*>(p.lse.address);
  const uint32_t hpw = HeadsPerWorkgroup(VirtualHeads(p));
  const dim3 grid(static_cast<uint32_t>(rec.dec_ranges * (VirtualHeads(p) / hpw)));
  if (p.page_size % 16 == 0) {
    hipLaunchKernelGGL((DecodeKernel<T, D, true>), grid, dim3(256), 0, stream, static_cast<const T*>(p.q.address), out,
                       lse, kv, kv.kv_indices, items, range_ptr, part_o, part_ml, q_rows, p.q_heads, hpw, scale_log2,
                       WindowOf(p), p.causal, CapOf(p));
  } else {
    hipLaunchKernelGGL((DecodeKernel<T, D, false>), grid, dim3(256), 0, stream, static_cast<const T*>(p.q.address), out,
                       lse, kv, kv.kv_indices, items, range_ptr, part_o, part_ml, q_rows, p.q_heads, hpw, scale_log2,
                       WindowOf(p), p.causal, CapOf(p));
  }
  ROOST_RETURN_IF_FAILED(roost::HipStatus(hipGetLastError(), "paged_attention", "decode launch"));
  return LaunchDecodeMerge<T, D>(p, rec, dev, kv, stream);
}

// Partials of the tile pieces: bf16 rows of the pieces' normalised outputs, then their fp32 (max, sum) pairs.
uint16_t* PrefillPartO(const RoostPagedAttentionParams& p, const PlanRecord& rec, unsigned char* dev) {
  return reinterpret_cast<uint16_t*>(dev + rec.float_offset);
}
float* PrefillPartMl(const RoostPagedAttentionParams& p, const PlanRecord& rec, unsigned char* dev) {
  return reinterpret_cast<float*>(PrefillPartO(p, rec, dev) + rec.splits * kPfRows * p.head_dim);
}

PrefillMergeArgs PrefillMergeArgsOf(const RoostPagedAttentionParams& p, const PlanRecord& rec, unsigned char* dev) {
  PrefillMergeArgs m{};
  m.merges = reinterpret_cast<const PrefillMerge*>(dev + rec.merge_offset);
  m.part_o = PrefillPartO(p, rec, dev);
  m.part_ml = PrefillPartMl(p, rec, dev);
  m.q_indptr = static_cast<const int32_t*>(p.q_indptr.address);
  m.two = static_cast<uint32_t>(rec.merges_two);
  m.blocks = m.two * (kPfTokens / kPfMergeRows) + (static_cast<uint32_t>(rec.merges) - m.two) * kPfTokens;
  return m;
}

RoostStatus LaunchPrefillMerge(const RoostPagedAttentionParams& p, const PlanRecord& rec, unsigned char* dev,
                               const KvView& kv, hipStream_t stream) {
  if (rec.merges == 0) return ROOST_STATUS_OK;
  auto* outp = static_cast<uint16_t*>(p.output.address);
  auto* lsep = static_cast<float*>(p.lse.address);
  const PrefillMergeArgs m = PrefillMergeArgsOf(p, rec, dev);
  const dim3 block(kGroup * p.head_dim / 4), g(m.blocks);
  if (p.head_dim == 64) {
    hipLaunchKernelGGL(PrefillMergeKernel<64>, g, block, 0, stream, outp, lsep, m, p.q_heads, kv.out_gate);
  } else if (p.head_dim == 128) {
    hipLaunchKernelGGL(PrefillMergeKernel<128>, g, block, 0, stream, outp, lsep, m, p.q_heads, kv.out_gate);
  } else {
    hipLaunchKernelGGL(PrefillMergeKernel<256>, g, block, 0, stream, outp, lsep, m, p.q_heads, kv.out_gate);
  }
  return roost::HipStatus(hipGetLastError(), "paged_attention", "prefill merge launch");
}

// A mixed step the plan chose to run in one launch (PlanRecord::overlap): the tile pieces and decode ranges on
// MixedAttentionKernel, then both merges in one MixedMergeKernel launch, all on the caller's stream.
RoostStatus LaunchMixed(const RoostPagedAttentionParams& p, const PlanRecord& rec, unsigned char* dev, const KvView& kv,
                        float scale_log2, hipStream_t stream) {
  const auto* q16 = static_cast<const uint16_t*>(p.q.address);
  const auto* q_indptr = static_cast<const int32_t*>(p.q_indptr.address);
  auto* outp = static_cast<uint16_t*>(p.output.address);
  auto* lsep = static_cast<float*>(p.lse.address);
  const auto* items = reinterpret_cast<const PrefillWork*>(dev);
  const uint32_t ps_shift = static_cast<uint32_t>(__builtin_ctz(p.page_size));
  const SoftCap cap = CapOf(p);
  const SoftCap raw{cap.capl / scale_log2, cap.k * scale_log2};
  const bool capped = cap.capl != 0.0f;
  const uint32_t hpw = HeadsPerWorkgroup(VirtualHeads(p));
  const uint32_t n_items = static_cast<uint32_t>(rec.work_items);
  const dim3 grid(n_items + static_cast<uint32_t>(rec.dec_ranges * (VirtualHeads(p) / hpw)));
  const auto* dec_items = reinterpret_cast<const DecodeWork*>(dev + rec.dec_item_offset);
  const auto* dec_ranges = reinterpret_cast<const int32_t*>(dev + rec.dec_range_offset);
  auto* dec_o = reinterpret_cast<float*>(dev + rec.dec_float_offset);
  auto* dec_ml = dec_o + rec.dec_splits * p.q_heads * p.head_dim;
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(512), 0, stream, q16, outp, lsep, kv, kv.kv_indices, q_indptr, items,
                       PrefillPartO(p, rec, dev), PrefillPartMl(p, rec, dev), p.q_heads, p.causal, ps_shift,
                       scale_log2, WindowOf(p), raw, n_items, dec_items, dec_ranges, dec_o, dec_ml, hpw, cap);
  };
  if (p.head_dim == 64) {
    capped ? launch(MixedAttentionKernel<64, true>) : launch(MixedAttentionKernel<64, false>);
  } else if (p.head_dim == 128) {
    capped ? launch(MixedAttentionKernel<128, true>) : launch(MixedAttentionKernel<128, false>);
  } else {
    capped ? launch(MixedAttentionKernel<256, true>) : launch(MixedAttentionKernel<256, false>);
  }
  ROOST_RETURN_IF_FAILED(roost::HipStatus(hipGetLastError(), "paged_attention", "mixed attention launch"));
  const PrefillMergeArgs pm = rec.merges != 0 ? PrefillMergeArgsOf(p, rec, dev) : PrefillMergeArgs{};
  const DecodeMergeArgs dm = DecodeMergeArgsOf(p, rec, dev, p.head_dim);
  const uint64_t blocks = uint64_t{pm.blocks} + rec.dec_merges * p.q_heads;
  if (blocks == 0) return ROOST_STATUS_OK;
  const dim3 g(static_cast<uint32_t>(blocks)), block(p.head_dim);
  auto* merge = p.head_dim == 64 ? MixedMergeKernel<64> : p.head_dim == 128 ? MixedMergeKernel<128> : MixedMergeKernel<256>;
  hipLaunchKernelGGL(merge, g, block, 0, stream, outp, lsep, pm, dm, p.q_heads, kv.out_gate);
  return roost::HipStatus(hipGetLastError(), "paged_attention", "mixed merge launch");
}

RoostStatus LaunchPrefill(const RoostPagedAttentionParams& p, const PlanRecord& rec, unsigned char* dev, const KvView& kv,
                          float scale_log2, hipStream_t stream) {
  if (rec.work_items == 0) return ROOST_STATUS_OK;
  const auto* items = reinterpret_cast<const PrefillWork*>(dev);
  const auto* q_indptr = static_cast<const int32_t*>(p.q_indptr.address);
  auto* outp = static_cast<uint16_t*>(p.output.address);
  auto* lsep = static_cast<float*>(p.lse.address);
  if (PrefillFastPath(p)) {
    uint16_t* part_o = PrefillPartO(p, rec, dev);
    float* part_ml = PrefillPartMl(p, rec, dev);
    const dim3 grid(static_cast<uint32_t>(rec.work_items));
    const auto* q16 = static_cast<const uint16_t*>(p.q.address);
    const uint32_t ps_shift = static_cast<uint32_t>(__builtin_ctz(p.page_size));
    // The cap in unscaled score units: Capped(s * scale_log2, cap) / scale_log2 == Capped(s, raw).
    const SoftCap cap = CapOf(p);
    const SoftCap raw{cap.capl / scale_log2, cap.k * scale_log2};
    const bool capped = cap.capl != 0.0f;
    auto launch = [&](auto kernel) {
      hipLaunchKernelGGL(kernel, grid, dim3(512), 0, stream, q16, outp, lsep, kv, kv.kv_indices, q_indptr, items,
                         part_o, part_ml, p.q_heads, p.causal, ps_shift, scale_log2, WindowOf(p), raw);
    };
    if (p.head_dim == 64) {
      capped ? launch(PrefillTileKernel<64, true>) : launch(PrefillTileKernel<64, false>);
    } else if (p.head_dim == 128) {
      capped ? launch(PrefillTileKernel<128, true>) : launch(PrefillTileKernel<128, false>);
    } else {
      capped ? launch(PrefillTileKernel<256, true>) : launch(PrefillTileKernel<256, false>);
    }
    ROOST_RETURN_IF_FAILED(roost::HipStatus(hipGetLastError(), "paged_attention", "prefill launch"));
    return LaunchPrefillMerge(p, rec, dev, kv, stream);
  }
  hipLaunchKernelGGL(PrefillKernel, dim3(static_cast<uint32_t>(rec.work_items)), dim3(256), 0, stream,
                     static_cast<const uint16_t*>(p.q.address), outp, lsep, kv, q_indptr, items, p.q_heads, p.causal,
                     scale_log2, WindowOf(p), CapOf(p));
  return roost::HipStatus(hipGetLastError(), "paged_attention", "prefill launch");
}


constexpr char kOp[] = "paged_attention";

const RoostPagedAttentionParams* Params(const void* params) {
  return static_cast<const RoostPagedAttentionParams*>(params);
}

// The plan record plan() leaves for run(): the batch shape it was made for and where its tables sit.
PlanRecord MakeRecord(const RoostPagedAttentionParams& p, const Layout& l) {
  PlanRecord r{};
  r.magic = kPlanMagic;
  r.mode = p.mode;
  r.batch = p.batch;
  r.tokens = p.tokens;
  r.page_size = p.page_size;
  r.kv_layout = p.kv_layout;
  r.head_dim = p.head_dim;
  r.kv_heads = p.kv_heads;
  r.window = WindowOf(p);
  r.merges_two = static_cast<uint32_t>(l.merges_two);
  r.overlap = l.overlap;
  r.pages = static_cast<uint64_t>(p.kv_indptr_host[p.batch]);
  r.work_items = l.work_items;
  r.ranges = l.ranges;
  r.merges = l.merges;
  r.range_offset = l.range_offset;
  r.merge_offset = l.merge_offset;
  r.counter_offset = l.counter_offset;
  r.splits = l.splits;
  r.int_bytes = l.int_bytes;
  r.float_offset = l.float_offset;
  r.float_bytes = l.float_bytes;
  r.dec_items = l.dec_items;
  r.dec_ranges = l.dec_ranges;
  r.dec_merges = l.dec_merges;
  r.dec_splits = l.dec_splits;
  r.dec_item_offset = l.dec_item_offset;
  r.dec_range_offset = l.dec_range_offset;
  r.dec_merge_offset = l.dec_merge_offset;
  r.dec_float_offset = l.dec_float_offset;
  return r;
}

bool RecordFits(const PlanRecord& r, const RoostPagedAttentionParams& p) {
  return r.mode == p.mode && r.batch == p.batch && r.tokens == p.tokens && r.page_size == p.page_size &&
         r.kv_layout == p.kv_layout && r.head_dim == p.head_dim && r.kv_heads == p.kv_heads && r.window == WindowOf(p);
}

}  // namespace

extern "C" ROOST_API RoostStatus roost_paged_attention_workspace(RoostContext* ctx, const void* params,
                                                                 RoostWorkspaceSizes* sizes) {
  roost::Gate gate(kOp);
  gate.Header(params, sizeof(RoostPagedAttentionParams))
      .Expect(sizes != nullptr, ROOST_STATUS_INVALID_ARGUMENT, "the sizes out-pointer is NULL");
  ROOST_GATE_RETURN(gate);
  const auto& p = *Params(params);
  return roost::CatchAll(kOp, [&]() -> RoostStatus {
    ROOST_RETURN_IF_FAILED(Admit(p, false));
    const Layout l = PlanLayout(p, ComputeUnits(ctx), nullptr);
    *sizes = RoostWorkspaceSizes{};
    sizes->device_bytes = l.total;
    sizes->pinned_host_bytes = l.int_bytes;
    sizes->plan_bytes = sizeof(PlanRecord);
    sizes->device_alignment = kAlign;
    return ROOST_STATUS_OK;
  });
}

extern "C" ROOST_API RoostStatus roost_paged_attention_plan(RoostContext* ctx, const void* params, const RoostWorkspace* ws,
                                                            void* stream) {
  roost::Gate gate(kOp);
  ROOST_GATE_RETURN(gate.Header(params, sizeof(RoostPagedAttentionParams)));
  const auto& p = *Params(params);
  return roost::CatchAll(kOp, [&]() -> RoostStatus {
    ROOST_RETURN_IF_FAILED(Admit(p, false));
    gate.Expect(ws != nullptr && ws->plan != nullptr, ROOST_STATUS_INVALID_ARGUMENT,
                "plan() writes its record into ws->plan, which is missing");
    ROOST_GATE_RETURN(gate);
    const uint32_t cus = ComputeUnits(ctx);
    const Layout l = PlanLayout(p, cus, nullptr);
    const bool fits = ws->plan_bytes >= sizeof(PlanRecord) && ws->pinned_host_bytes >= l.int_bytes &&
                      (l.int_bytes == 0 || ws->pinned_host != nullptr) && roost::HasDeviceRegion(ws, l.total, kAlign);
    gate.Expect(fits, ROOST_STATUS_WORKSPACE_TOO_SMALL,
                "this batch needs %llu device bytes (%u-aligned), %llu pinned bytes and a %zu-byte plan record; the "
                "workspace has %llu, %llu and %llu", static_cast<unsigned long long>(l.total), kAlign,
                static_cast<unsigned long long>(l.int_bytes), sizeof(PlanRecord),
                static_cast<unsigned long long>(ws->device_bytes), static_cast<unsigned long long>(ws->pinned_host_bytes),
                static_cast<unsigned long long>(ws->plan_bytes));
    ROOST_GATE_RETURN(gate);
    if (l.int_bytes > 0) {
      auto* host = static_cast<unsigned char*>(ws->pinned_host);
      std::memset(host, 0, l.int_bytes);
      PlanLayout(p, cus, host);
      ROOST_RETURN_IF_FAILED(roost::HipStatus(
          hipMemcpyAsync(ws->device, host, l.int_bytes, hipMemcpyHostToDevice, roost::Stream(stream)), kOp,
          "copy of the work tables to the device"));
    }
    const PlanRecord rec = MakeRecord(p, l);
    std::memcpy(ws->plan, &rec, sizeof(rec));
    return ROOST_STATUS_OK;
  });
}

namespace {

// run() of an admitted-or-not call; out_gate (NULL for none) folds SigmoidMul into every kernel that writes an output
// row.
RoostStatus RunAttention(RoostContext* ctx, const void* params, const RoostWorkspace* ws, void* stream,
                         const void* out_gate) {
  using namespace roost;
  Gate gate(kOp);
  ROOST_GATE_RETURN(gate.Header(params, sizeof(RoostPagedAttentionParams)));
  const auto& p = *Params(params);
  return CatchAll(kOp, [&]() -> RoostStatus {
    ROOST_RETURN_IF_FAILED(Admit(p, true));
    // C1: run() before plan() in this workspace is NOT_PLANNED (the caller then plans and runs again).
    if (ws == nullptr || ws->plan == nullptr || ws->plan_bytes < sizeof(PlanRecord)) {
      return Report(ROOST_STATUS_NOT_PLANNED, kOp, "the workspace carries no plan record; call plan() first");
    }
    PlanRecord rec;
    std::memcpy(&rec, ws->plan, sizeof(rec));
    if (rec.magic != kPlanMagic) {
      return Report(ROOST_STATUS_NOT_PLANNED, kOp, "the plan record is blank; call plan() first");
    }
    gate.Expect(RecordFits(rec, p), ROOST_STATUS_INVALID_ARGUMENT,
                "the plan record describes batch %u / tokens %u / mode %u / window %d; this call is batch %u / tokens "
                "%u / mode %u / window %d (or its page size, layout, head shape differ)", rec.batch, rec.tokens,
                rec.mode, rec.window, p.batch, p.tokens, p.mode, WindowOf(p))
        .Tensor("kv_indices", p.kv_indices, ROOST_DTYPE_I32, rec.pages)
        .Expect(HasDeviceRegion(ws, rec.float_offset + rec.float_bytes, kAlign), ROOST_STATUS_WORKSPACE_TOO_SMALL,
                "the plan placed %llu bytes in the device workspace, which holds %llu",
                static_cast<unsigned long long>(rec.float_offset + rec.float_bytes),
                static_cast<unsigned long long>(ws->device_bytes));
    ROOST_GATE_RETURN(gate);
    const float scale = p.sm_scale != 0.0f ? p.sm_scale : 1.0f / std::sqrt(static_cast<float>(p.head_dim));
    const float scale_log2 = scale * kLog2e;
    KvView kv{};
    kv.k = p.k_cache.address;
    kv.v = p.v_cache.address;
    kv.kv_indptr = static_cast<const int32_t*>(p.kv_indptr.address);
    kv.kv_indices = static_cast<const int32_t*>(p.kv_indices.address);
    kv.last_len = static_cast<const int32_t*>(p.kv_last_page_len.address);
    const uint64_t page_elems = static_cast<uint64_t>(p.page_size) * p.kv_heads * p.head_dim;
    kv.pool_pages = std::min(p.k_cache.length, p.v_cache.length) / page_elems;
    kv.page_size = p.page_size;
    kv.kv_heads = p.kv_heads;
    kv.head_shift = HeadShift(p);
    kv.vheads = VirtualHeads(p);
    kv.hnd = p.kv_layout == ROOST_LAYOUT_PAGED_HND ? 1u : 0u;
    kv.out_gate = out_gate;
    auto* dev = static_cast<unsigned char*>(ws->device);
    hipStream_t s = Stream(stream);
    if (p.mode == ROOST_ATTENTION_DECODE) {
      const bool bf16 = p.q.dtype == ROOST_DTYPE_BF16;
      switch (p.head_dim) {
        case 64: return bf16 ? LaunchDecode<uint16_t, 64>(p, rec, dev, kv, scale_log2, s)
                             : LaunchDecode<float, 64>(p, rec, dev, kv, scale_log2, s);
        case 128: return bf16 ? LaunchDecode<uint16_t, 128>(p, rec, dev, kv, scale_log2, s)
                              : LaunchDecode<float, 128>(p, rec, dev, kv, scale_log2, s);
        default: return bf16 ? LaunchDecode<uint16_t, 256>(p, rec, dev, kv, scale_log2, s)
                             : LaunchDecode<float, 256>(p, rec, dev, kv, scale_log2, s);
      }
    }
    // The multi-token sequences on the tile kernels, then the single-token ones on the decode kernels (bf16 in prefill
    // mode, at the call's head dim), or both in one launch when the plan chose that (ChooseOverlap).
    if (p.q.dtype == ROOST_DTYPE_F32) {  // every query token is a row of the f32 decode kernel
      switch (p.head_dim) {
        case 64: return LaunchDecode<float, 64>(p, rec, dev, kv, scale_log2, s);
        case 128: return LaunchDecode<float, 128>(p, rec, dev, kv, scale_log2, s);
        default: return LaunchDecode<float, 256>(p, rec, dev, kv, scale_log2, s);
      }
    }
    if (rec.overlap != 0) return LaunchMixed(p, rec, dev, kv, scale_log2, s);
    ROOST_RETURN_IF_FAILED(LaunchPrefill(p, rec, dev, kv, scale_log2, s));
    switch (p.head_dim) {
      case 64: return LaunchDecode<uint16_t, 64>(p, rec, dev, kv, scale_log2, s);
      case 128: return LaunchDecode<uint16_t, 128>(p, rec, dev, kv, scale_log2, s);
      default: return LaunchDecode<uint16_t, 256>(p, rec, dev, kv, scale_log2, s);
    }
  });
}

}  // namespace

extern "C" ROOST_API RoostStatus roost_paged_attention_run(RoostContext* ctx, const void* params,
                                                           const RoostWorkspace* ws, void* stream) {
  return RunAttention(ctx, params, ws, stream, nullptr);
}

// PagedAttention followed by SigmoidMul on its output, in one call: the gate multiplies each output element where the
// kernels write it (the tile, decode and merge kernels' epilogues), with SigmoidMul's arithmetic on the output already
// rounded to its type, so the result equals run() then roost_sigmoid_mul_run bit for bit and the output is written once.
extern "C" ROOST_API RoostStatus roost_amd_paged_attention_gated_run(RoostContext* ctx, const void* params,
                                                                     const void* gate_params, const RoostWorkspace* ws,
                                                                     void* stream) {
  using namespace roost;
  Gate gate(kOp);
  ROOST_GATE_RETURN(gate.Header(params, sizeof(RoostPagedAttentionParams)));
  gate.Expect(gate_params != nullptr, ROOST_STATUS_INVALID_ARGUMENT, "no SigmoidMul params struct was passed");
  ROOST_GATE_RETURN(gate);
  ROOST_GATE_RETURN(gate.Header(gate_params, sizeof(RoostSigmoidMulParams)));
  const auto& p = *Params(params);
  const auto& sm = *static_cast<const RoostSigmoidMulParams*>(gate_params);
  return CatchAll(kOp, [&]() -> RoostStatus {
    ROOST_RETURN_IF_FAILED(Admit(p, true));
    const uint32_t dt = p.output.dtype;
    const uint64_t dim = static_cast<uint64_t>(p.q_heads) * p.head_dim, n = dim * p.tokens;
    gate.Expect(sm.rows == p.tokens && sm.dim == dim, ROOST_STATUS_INVALID_ARGUMENT,
                "the gate covers %u rows x %u; the attention output is %u tokens x %llu", sm.rows, sm.dim, p.tokens,
                static_cast<unsigned long long>(dim))
        .Expect(sm.input.address == p.output.address && sm.output.address == p.output.address,
                ROOST_STATUS_INVALID_ARGUMENT,
                "the gate applies in place: its input and output must both be the attention output (%p), not %p and %p",
                p.output.address, sm.input.address, sm.output.address)
        .Tensor("gate input", sm.input, dt, n)
        .Tensor("gate output", sm.output, dt, n)
        .Tensor("gate", sm.gate, dt, n)
        .Aligned("gate", sm.gate.address, 8);
    ROOST_GATE_RETURN(gate);
    const auto g0 = reinterpret_cast<uintptr_t>(sm.gate.address), o0 = reinterpret_cast<uintptr_t>(p.output.address);
    const uint64_t bytes = n * ElementBytes(dt);
    gate.Expect(n == 0 || g0 + bytes <= o0 || o0 + bytes <= g0, ROOST_STATUS_INVALID_ARGUMENT,
                "the gate (%p) overlaps the output (%p, %llu bytes)", sm.gate.address, p.output.address,
                static_cast<unsigned long long>(bytes));
    ROOST_GATE_RETURN(gate);
    return RunAttention(ctx, params, ws, stream, sm.gate.address);
  });
}
